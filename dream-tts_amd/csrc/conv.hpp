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

// The single-output-channel kernel (conv_narrow.hip).
bool conv_narrow_eligible(const dtts_conv_desc *d);
hipError_t conv_narrow_launch(const dtts_conv_desc *d, hipStream_t stream);
const char *conv_narrow_kernel_name(const dtts_conv_desc *d);  // the kernel a narrow launch runs

}  // namespace dtts
