/*
 * dtts -- MI355X (gfx950) kernels for dream-tts's tts-nn fused-op hot path, as a plain C ABI.
 *
 * Every entry point takes device pointers, sizes and a hipStream_t, enqueues its kernels on
 * that stream and returns without synchronising. Outputs are caller-allocated (the KV caches
 * are updated in place). The return value is DTTS_OK or a negative status; on failure
 * dtts_last_error() holds a message naming the op (per thread, valid until the next call).
 *
 * Each entry point names the reference interface it replaces: a tts-nn function or candle
 * CustomOp in drmhse/dream-tts (paths relative to that repository's root). f16 tensors are
 * IEEE binary16 bit patterns (uint16_t); conversions round to nearest-even.
 *
 * Layouts: row-major. NLC = [lanes, L, C] (channels-last), NCL = [lanes, C, L].
 */
#ifndef DTTS_H
#define DTTS_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DTTS_OK 0
#define DTTS_ERR_INVALID (-1)  /* bad pointer, shape or layout: nothing was enqueued */
#define DTTS_ERR_HIP (-2)      /* the HIP runtime refused a launch or call */
#define DTTS_ERR_UNSUPPORTED (-3) /* a shape this build has no kernel for */

typedef uint16_t dtts_f16;

/* ------------------------------------------------------------------ lifecycle */

/* Message for the last failed call on this thread ("" if none). Replaces the text of candle's
 * `bail!` errors (e.g. crates/tts-nn/src/nlcconv.rs:86-91). */
const char *dtts_last_error(void);

/* ABI version, (major << 16) | minor. */
int dtts_version(void);

/* Optional: binds the library to the current HIP device and checks it is gfx950. Every entry
 * point works without it. Replaces the pipeline cache set-up of crates/tts-nn/src/mtl.rs:1409-1458
 * (HIP code objects load with the library). */
int dtts_init(void);

/* ------------------------------------------------------------------ a1/a2 snake */

/* y = x + brecip[c] * sin^2(alpha[c] * x), per channel c.
 *
 * NCL (x, y [lanes, chan, len]) replaces fused::snake_beta / SnakeBeta::metal_fwd
 * (crates/tts-nn/src/fused.rs:187-286, 665-681), which takes lanes == 1; any lane count here.
 * NLC (x, y [rows, chan]) replaces fused::snake_beta_nlc / SnakeBetaNlc
 * (crates/tts-nn/src/fused.rs:526-659). f16 variants compute in f32 and round once
 * (fused.rs:573-598). alpha and brecip are f32 [chan]. x == y (in place) is allowed. */
int dtts_snake_ncl_f32(const float *x, const float *alpha, const float *brecip, float *y,
                       int64_t lanes, int64_t chan, int64_t len, hipStream_t stream);
int dtts_snake_ncl_f16(const dtts_f16 *x, const float *alpha, const float *brecip, dtts_f16 *y,
                       int64_t lanes, int64_t chan, int64_t len, hipStream_t stream);
int dtts_snake_nlc_f32(const float *x, const float *alpha, const float *brecip, float *y,
                       int64_t rows, int64_t chan, hipStream_t stream);
int dtts_snake_nlc_f16(const dtts_f16 *x, const float *alpha, const float *brecip, dtts_f16 *y,
                       int64_t rows, int64_t chan, hipStream_t stream);

/* ------------------------------------------------------------------ a3-a5 channels-last conv */

/* One channels-last conv1d with its neighbours fused (the general form behind
 * nlc::causal_conv1d, nlc::snake_conv_residual and the transposed conv):
 *
 *   s[l, n] = bias[n] + residual[l, n] + sum_t sum_c xs[l + t*dilation - pad_left, c] * w_tm[n, t*cin + c]
 *   y_pre   = f16(act(s))                        (stored when y_pre != NULL)
 *   y       = f16(SnakeBeta_out(y_pre))          (or y_pre itself when out_alpha == NULL)
 *
 * per lane, with xs = x, or f16(SnakeBeta_in(x)) when in_alpha != NULL, and zero for taps
 * outside [0, len). pad_left = (k-1)*dilation is causal (the reference's only form on this
 * path, crates/tts-nn/src/nlc.rs:70-132); smaller values give the centred conv of
 * crates/tts-nn/src/lib.rs:736-767. The reference computes the same sum in f32 on one lane
 * (NlcConv, crates/tts-nn/src/nlcconv.rs:15-175; kernel mtl.rs:937-1065, whose has_snake /
 * has_res flags are in_alpha / residual here). f16 storage, f32 accumulation.
 *
 * Weight layout w_tm is [cout, k*cin] (tap-major rows: tap_major_weight, crates/tts-nn/src/
 * lib.rs:630-635), not NlcConv's [k*cin, cout]: both GEMM operands then run along K, which is
 * what the matrix cores consume. dtts_tap_weight_to_tap_major converts. x, w_tm, y, bias,
 * residual and y_pre must be 16-byte aligned for the matrix-core kernel; other shapes or
 * alignments take a direct (slow, exact-semantics) kernel. act: 0 none, 1 tanh. */
typedef struct dtts_conv_desc {
    int64_t lanes, len, cin, cout, k, dilation, pad_left;
    const void *x;          /* [lanes, len, cin] */
    const void *w;          /* [cout, k*cin] */
    const void *bias;       /* [cout] or NULL */
    const float *in_alpha;  /* [cin] prologue SnakeBeta, or NULL */
    const float *in_brecip;
    const void *residual;   /* [lanes, len, cout] or NULL */
    void *y_pre;            /* [lanes, len, cout] or NULL */
    const float *out_alpha; /* [cout] epilogue SnakeBeta, or NULL */
    const float *out_brecip;
    void *y;                /* [lanes, len, cout] */
    int32_t act;
} dtts_conv_desc;

int dtts_conv1d_nlc_f16_ex(const dtts_conv_desc *desc, hipStream_t stream);

/* nlc::causal_conv1d (crates/tts-nn/src/nlc.rs:70-132): causal, pad (k-1)*dilation. Any lane
 * count (the reference requires one, crates/tts-nn/src/nlcconv.rs:192). */
int dtts_causal_conv1d_nlc_f16(const dtts_f16 *x, const dtts_f16 *w_tm, const dtts_f16 *bias,
                               dtts_f16 *y, int64_t lanes, int64_t len, int64_t cin, int64_t cout,
                               int64_t k, int64_t dilation, hipStream_t stream);

/* nlc::snake_conv_residual (crates/tts-nn/src/nlc.rs:40-68): residual + conv(SnakeBeta(x)). */
int dtts_snake_conv_residual_nlc_f16(const dtts_f16 *x, const dtts_f16 *w_tm, const dtts_f16 *bias,
                                     int64_t dilation, const float *alpha, const float *brecip,
                                     const dtts_f16 *residual, dtts_f16 *y, int64_t lanes,
                                     int64_t len, int64_t cin, int64_t cout, int64_t k,
                                     hipStream_t stream);

/* ------------------------------------------------------------------ weight layouts (host) */

/* Host-side load-time rearrangements (the reference also does these on the host,
 * crates/tts-nn/src/lib.rs:1252-1298). Element-size generic permutations: elem_size 2 (f16) or
 * 4 (f32); src and dst must not overlap. */

/* tap_major_weight (crates/tts-nn/src/lib.rs:630-635): torch [cout, cin, k] -> [cout, k*cin]. */
int dtts_tap_major_weight(const void *w_oik, void *w_tm, int64_t cout, int64_t cin, int64_t k,
                          int64_t elem_size);

/* nlc::tap_weight's layout [k, cin, cout] (crates/tts-nn/src/nlc.rs:30-33) -> [cout, k*cin]. */
int dtts_tap_weight_to_tap_major(const void *w_kio, void *w_tm, int64_t k, int64_t cin,
                                 int64_t cout, int64_t elem_size);

/* nlc::transpose_tap_weight (crates/tts-nn/src/nlc.rs:158-174) in tap-major form: a
 * ConvTranspose1d weight [cin, cout, kernel], kernel = m*stride, becomes the causal conv weight
 * [stride*cout, m*cin] whose output column p*cout + co is phase p of channel co; run it with
 * k = m, dilation 1, and read the [lanes, len, stride*cout] result as [lanes, len*stride, cout]. */
int dtts_transpose_tap_major_weight(const void *w_iok, void *w_tm, int64_t cin, int64_t cout,
                                    int64_t kernel, int64_t stride, int64_t elem_size);

/* nlc::transpose_bias (crates/tts-nn/src/nlc.rs:177-183): [cout] -> [stride*cout]. */
int dtts_transpose_bias(const void *b, void *out, int64_t cout, int64_t stride,
                        int64_t elem_size);

#ifdef __cplusplus
}
#endif
#endif /* DTTS_H */
