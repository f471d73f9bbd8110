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

#ifdef __cplusplus
}
#endif
#endif /* DTTS_H */
