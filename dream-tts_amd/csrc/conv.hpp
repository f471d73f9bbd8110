// Channels-last conv entry points shared by the C ABI and the codec driver.
#pragma once

#include <cstring>

#include "common.hpp"

namespace dtts {

// "mfma" when the tiled matrix-core kernel takes the descriptor's shape, else "direct".
const char *conv_path_name(const dtts_conv_desc *d);
// The kernel the descriptor launches, in the form a profiler's demangled name contains.
const char *conv_kernel_name(const dtts_conv_desc *d);
int conv1d_nlc_f16(const dtts_conv_desc *d, hipStream_t stream);

// The f32 form (conv_nlc_f32.hip): same descriptor, f32 operands.
const char *conv_f32_kernel_name(const dtts_conv_desc *d);
int conv1d_nlc_f32(const dtts_conv_desc *d, hipStream_t stream);

// True for a codec made by dtts_codec_create_f32 (codec.hip).
bool codec_is_f32(const dtts_codec *c);

// The fused residual unit (ru.hip).
bool residual_unit_supported(const dtts_ru_desc *d);
const char *residual_unit_kernel_name(const dtts_ru_desc *d);
int residual_unit_nlc_f16(const dtts_ru_desc *d, hipStream_t stream);

// The f32 codec's convs on the f16 matrix cores (conv_split.hip): activations stored as f16 pairs,
// rows [hi(C) | lo(C)]; weights scaled by 2^s and split into [wh | wh | wl] per tap (split_weight),
// so a conv over cs channels is an f16 GEMM over 3 cs. The output is written in its consumer's
// layout: GEMM column n = p * cv + c of input position l goes to position l * (cout / cv) + p,
// channel c (cv = cout for an ordinary conv; cout / rate for a transposed one).
struct SplitConv {
    int64_t lanes, len, cs, cout, k, dil, pad_left, cv;
    const half_t *x;               // split input [lanes, len, 2 cs]
    const half_t *w;               // split weight [cout, k * 3 cs]
    float w_inv;                   // 2^-s
    const float *bias;             // [cout] f32, or null
    const half_t *res;             // split residual in the output's layout (cv == cout), or null
    half_t *y_pre, *y;             // split outputs (y_pre: before the SnakeBeta, or null)
    const float *a_out, *r_out;    // SnakeBeta per GEMM column, or null
};
bool conv_split_supported(int64_t lanes, int64_t len, int64_t cs, int64_t cout, int64_t k, int64_t dil);
const char *conv_split_kernel_name(int64_t lanes, int64_t len, int64_t cs, int64_t cout, int64_t k, int64_t dil);
int conv1d_nlc_split(const SplitConv &s, hipStream_t stream);
// Tap-major f32 [cout, k cs] -> the split weight w3 [cout, k * 3 cs] (synchronises `stream` once to
// read the weight's largest magnitude).
int split_weight(const float *w, int64_t cout, int64_t k, int64_t cs, half_t *w3, float &w_inv, hipStream_t stream,
                 const char *name = "dtts_codec_create_f32 (split weights)");
// f32 [rows, C] -> split rows.
int split_activations(const float *x, half_t *y, int64_t rows, int64_t C, hipStream_t stream);
// The f32 single-output-channel conv (conv_nlc_f32.hip) reading a split input (d->x: rows
// [hi(cin) | lo(cin)]); every other operand as dtts_conv1d_nlc_f32_ex takes it.
bool conv_f32_narrow_split_eligible(const dtts_conv_desc *d);
int conv1d_nlc_f32_narrow_split(const dtts_conv_desc *d, hipStream_t stream);

// The single-output-channel kernel (conv_narrow.hip).
bool conv_narrow_eligible(const dtts_conv_desc *d);
hipError_t conv_narrow_launch(const dtts_conv_desc *d, hipStream_t stream);
const char *conv_narrow_kernel_name(const dtts_conv_desc *d);  // the kernel a narrow launch runs

}  // namespace dtts
