/*
 * CPU oracle for the tts-nn fused-op hot path. TEST INFRASTRUCTURE ONLY: tests/ use it as the
 * parity checker and bench.py's cpu_baseline leg times it; the product never calls it.
 *
 * Reference: drmhse/dream-tts (Rust, candle 0.10.2). Its candle CPU path cannot be built here
 * (no Rust toolchain, candle not vendored), so this file restates that path's arithmetic. Each
 * function names the reference file:line it follows; where the arithmetic lives in candle (not
 * in the reference tree) the restated semantics are marked "believed" and the test that pins
 * them is named in the function's comment.
 *
 * Built with -ffp-contract=off: every product and sum rounds separately, as Rust's f32
 * arithmetic does (rustc never contracts a*b+c into an fma on its own).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ f16 storage points */

/* IEEE binary16 round-to-nearest-even, the conversion `half::f16::from_f32` performs.
 * Pinned by tests/test_oracle_core.py against numpy's float16 cast on edge cases and 2^20
 * random bit patterns. */
uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf, nan */
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    const int e = (int)(ax >> 23);
    const uint32_t mant = ax & 0x7fffffu;
    if (ax >= 0x38800000u) { /* normal half */
        uint32_t h = ((uint32_t)(e - 112) << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (e < 102) return (uint16_t)sign; /* below half the smallest subnormal */
    const uint32_t m24 = mant | 0x800000u;
    const int shift = 126 - e; /* 14..24 */
    uint32_t h = m24 >> shift;
    const uint32_t rem = m24 & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    const uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
        memcpy(&x, &v, 4);
        x |= sign;
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void or_f32_to_f16_array(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = or_f32_to_f16(src[i]);
}

void or_f16_to_f32_array(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = or_f16_to_f32(src[i]);
}

/* ------------------------------------------------------------------ a1/a2 snake */

/* snake_beta's composed candle form, crates/tts-nn/src/fused.rs:675-680 (and snake_full,
 * lib.rs:1090-1093): u = x*alpha; x + sin(u)^2 * r. Rust's f32::sin is the platform libm sinf,
 * which is what this calls. */
static inline float snake1(float v, float a, float r) {
    const float s = sinf(v * a);
    const float s2 = s * s;
    return v + s2 * r;
}

void or_snake_ncl_f32(const float *x, const float *alpha, const float *brecip, float *y,
                      int64_t lanes, int64_t chan, int64_t len) {
    for (int64_t b = 0; b < lanes; ++b)
        for (int64_t c = 0; c < chan; ++c) {
            const int64_t o = (b * chan + c) * len;
            for (int64_t l = 0; l < len; ++l) y[o + l] = snake1(x[o + l], alpha[c], brecip[c]);
        }
}

/* SnakeBetaNlc::cpu_fwd, fused.rs:564-599: dst = v + br*(a*v).sin().powi(2). */
void or_snake_nlc_f32(const float *x, const float *alpha, const float *brecip, float *y,
                      int64_t rows, int64_t chan) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < chan; ++c) {
            const int64_t i = r * chan + c;
            y[i] = snake1(x[i], alpha[c], brecip[c]);
        }
}

/* f16 activations: widened to f32, computed in f32, rounded back once (fused.rs:573-598). */
void or_snake_nlc_f16(const uint16_t *x, const float *alpha, const float *brecip, uint16_t *y,
                      int64_t rows, int64_t chan) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < chan; ++c) {
            const int64_t i = r * chan + c;
            y[i] = or_f32_to_f16(snake1(or_f16_to_f32(x[i]), alpha[c], brecip[c]));
        }
}

void or_snake_ncl_f16(const uint16_t *x, const float *alpha, const float *brecip, uint16_t *y,
                      int64_t lanes, int64_t chan, int64_t len) {
    for (int64_t b = 0; b < lanes; ++b)
        for (int64_t c = 0; c < chan; ++c) {
            const int64_t o = (b * chan + c) * len;
            for (int64_t l = 0; l < len; ++l)
                y[o + l] = or_f32_to_f16(snake1(or_f16_to_f32(x[o + l]), alpha[c], brecip[c]));
        }
}

/* The folded snakes' candle forms: snake_folded's off-Metal `x + x.sin()?.sqr()?`
 * (crates/tts-nn/src/fused.rs:501-508; SnakeFolded::cpu_fwd, fused.rs:25-40, is x + sin(x)^2 too)
 * and tts_nn::snake's `u = x * alpha; u + u.sin().sqr()` (lib.rs:1080-1083; SnakeAlpha::cpu_fwd,
 * fused.rs:105-129). */
void or_snake_folded_f32(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float s = sinf(x[i]);
        y[i] = x[i] + s * s;
    }
}

void or_snake_alpha_f32(const float *x, const float *alpha, float *y, int64_t lanes, int64_t chan,
                        int64_t len) {
    for (int64_t b = 0; b < lanes; ++b)
        for (int64_t c = 0; c < chan; ++c) {
            const int64_t o = (b * chan + c) * len;
            for (int64_t l = 0; l < len; ++l) {
                const float u = x[o + l] * alpha[c];
                const float s = sinf(u);
                y[o + l] = u + s * s;
            }
        }
}

/* Double-precision form, the target the reference's accuracy tests measure against
 * (fused.rs:2356-2391). */
void or_snake_nlc_f64(const double *x, const double *alpha, const double *brecip, double *y,
                      int64_t rows, int64_t chan) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < chan; ++c) {
            const int64_t i = r * chan + c;
            const double s = sin(alpha[c] * x[i]);
            y[i] = x[i] + brecip[c] * s * s;
        }
}

/* ------------------------------------------------------------------ a7 im2col */

/* Im2ColTapMajor::cpu_fwd, crates/tts-nn/src/im2col.rs:59-84: one [1, cin, len] input to
 * [k*cin, len], row t*cin+c holding x[c, l + t*dil - pad_left], zero out of range. */
void or_im2col_tap_major_f32(const float *x, float *cols, int64_t cin, int64_t len, int64_t k,
                             int64_t dil, int64_t pad_left) {
    for (int64_t t = 0; t < k; ++t)
        for (int64_t c = 0; c < cin; ++c) {
            float *row = cols + (t * cin + c) * len;
            for (int64_t l = 0; l < len; ++l) {
                const int64_t s = l + t * dil - pad_left;
                row[l] = (s >= 0 && s < len) ? x[c * len + s] : 0.0f;
            }
        }
}

/* ------------------------------------------------------------------ weight layouts */

/* nlc::tap_weight, crates/tts-nn/src/nlc.rs:30-33: torch [out, in, k] -> [k, in, out]. */
void or_tap_weight_f32(const float *w_oik, float *w_kio, int64_t cout, int64_t cin, int64_t k) {
    for (int64_t o = 0; o < cout; ++o)
        for (int64_t i = 0; i < cin; ++i)
            for (int64_t t = 0; t < k; ++t)
                w_kio[(t * cin + i) * cout + o] = w_oik[(o * cin + i) * k + t];
}

/* tap_major_weight, crates/tts-nn/src/lib.rs:630-635: [out, in, k] -> [out, k*in]. */
void or_tap_major_weight_f32(const float *w_oik, float *w_tm, int64_t cout, int64_t cin,
                             int64_t k) {
    for (int64_t o = 0; o < cout; ++o)
        for (int64_t i = 0; i < cin; ++i)
            for (int64_t t = 0; t < k; ++t)
                w_tm[o * k * cin + t * cin + i] = w_oik[(o * cin + i) * k + t];
}

/* nlc::transpose_weights + transpose_tap_weight, crates/tts-nn/src/nlc.rs:141-174: a
 * ConvTranspose1d weight [in, out, K] with K = m*stride becomes a causal conv weight
 * [m, in, stride*out] whose tap groups are reversed: out[t][ci][p*out+co] =
 * w[ci][co][(m-1-t)*stride + p]. */
void or_transpose_tap_weight_f32(const float *w_iok, float *w_tap, int64_t cin, int64_t cout,
                                 int64_t k, int64_t stride) {
    const int64_t m = k / stride;
    const int64_t wide = stride * cout;
    for (int64_t i = 0; i < m; ++i) {       /* tap group i of transpose_weights */
        const int64_t t = m - 1 - i;          /* its place after the reversal */
        for (int64_t ci = 0; ci < cin; ++ci)
            for (int64_t p = 0; p < stride; ++p)
                for (int64_t co = 0; co < cout; ++co)
                    w_tap[(t * cin + ci) * wide + p * cout + co] =
                        w_iok[(ci * cout + co) * k + i * stride + p];
    }
}

/* nlc::transpose_bias, crates/tts-nn/src/nlc.rs:177-183: b repeated across stride phases. */
void or_transpose_bias_f32(const float *b, float *out, int64_t cout, int64_t stride) {
    for (int64_t p = 0; p < stride; ++p)
        for (int64_t co = 0; co < cout; ++co) out[p * cout + co] = b[co];
}

/* ------------------------------------------------------------------ a3/a4 NLC conv, direct */

/* NlcConv::cpu_fwd, crates/tts-nn/src/nlcconv.rs:33-73, generalised as the Metal kernel is
 * (mtl.rs:937-1065): SnakeBeta applied to x as it loads (a padded tap stays 0 since
 * snake(0) = 0) and a residual added on the way out; `pad_left` = (k-1)*dil is causal.
 * Accumulation order: bias, then t, then ci (the cpu_fwd order). Lanes are independent. */
void or_conv1d_nlc_f32(const float *x, const float *w_tap, const float *bias, const float *alpha,
                       const float *brecip, const float *res, float *y, int64_t lanes,
                       int64_t len, int64_t cin, int64_t cout, int64_t k, int64_t dil,
                       int64_t pad_left) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < lanes; ++b)
        for (int64_t l = 0; l < len; ++l) {
            float *row = y + (b * len + l) * cout;
            for (int64_t co = 0; co < cout; ++co) row[co] = bias ? bias[co] : 0.0f;
            for (int64_t t = 0; t < k; ++t) {
                const int64_t s = l + t * dil - pad_left;
                if (s < 0 || s >= len) continue;
                const float *xr = x + (b * len + s) * cin;
                for (int64_t ci = 0; ci < cin; ++ci) {
                    float xv = xr[ci];
                    if (alpha) xv = snake1(xv, alpha[ci], brecip[ci]);
                    const float *wr = w_tap + (t * cin + ci) * cout;
                    for (int64_t co = 0; co < cout; ++co) row[co] += xv * wr[co];
                }
            }
            if (res) {
                const float *rr = res + (b * len + l) * cout;
                for (int64_t co = 0; co < cout; ++co) row[co] += rr[co];
            }
        }
}

void or_conv1d_nlc_f64(const double *x, const double *w_tap, const double *bias,
                       const double *alpha, const double *brecip, const double *res, double *y,
                       int64_t lanes, int64_t len, int64_t cin, int64_t cout, int64_t k,
                       int64_t dil, int64_t pad_left) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < lanes; ++b)
        for (int64_t l = 0; l < len; ++l) {
            double *row = y + (b * len + l) * cout;
            for (int64_t co = 0; co < cout; ++co) row[co] = bias ? bias[co] : 0.0;
            for (int64_t t = 0; t < k; ++t) {
                const int64_t s = l + t * dil - pad_left;
                if (s < 0 || s >= len) continue;
                const double *xr = x + (b * len + s) * cin;
                for (int64_t ci = 0; ci < cin; ++ci) {
                    double xv = xr[ci];
                    if (alpha) {
                        const double sn = sin(alpha[ci] * xv);
                        xv = xv + brecip[ci] * sn * sn;
                    }
                    const double *wr = w_tap + (t * cin + ci) * cout;
                    for (int64_t co = 0; co < cout; ++co) row[co] += xv * wr[co];
                }
            }
            if (res) {
                const double *rr = res + (b * len + l) * cout;
                for (int64_t co = 0; co < cout; ++co) row[co] += rr[co];
            }
        }
}

/* The f16 codec's storage points (the config-5 form of the conv above): activations, weights,
 * bias and residual live in f16; a snaked input is computed in f32 and rounded to f16 (the
 * value an unfused snake_beta_nlc f16 pass would have stored); products accumulate in f32;
 * bias then residual are added in f32 and the sum is rounded once. `act_tanh` applies tanh
 * before that rounding (the decoder's output conv). */
/* gelu_exact (crates/tts-nn/src/lib.rs:1129-1131; CPU op cpu.rs:173-191): 0.5 x (1 + erf(x /
 * sqrt 2)). erf here is the C library's; the reference's CPU path evaluates a clamped rational
 * approximation of erf (cpu.rs:10-26) that agrees with it to ~1e-7 absolute. */
float or_gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

void or_conv1d_nlc_f16_ex(const uint16_t *x, const uint16_t *w_tap, const uint16_t *bias,
                          const float *alpha, const float *brecip, const uint16_t *res,
                          uint16_t *y, int64_t lanes, int64_t len, int64_t cin, int64_t cout,
                          int64_t k, int64_t dil, int64_t pad_left, int32_t act,
                          const float *scale) {
    float *wf = (float *)malloc(sizeof(float) * (size_t)(k * cin * cout));
    for (int64_t i = 0; i < k * cin * cout; ++i) wf[i] = or_f16_to_f32(w_tap[i]);
#pragma omp parallel
    {
        float *acc = (float *)malloc(sizeof(float) * (size_t)cout);
        float *xs = (float *)malloc(sizeof(float) * (size_t)cin);
#pragma omp for collapse(2) schedule(static)
        for (int64_t b = 0; b < lanes; ++b)
            for (int64_t l = 0; l < len; ++l) {
                for (int64_t co = 0; co < cout; ++co) acc[co] = 0.0f;
                for (int64_t t = 0; t < k; ++t) {
                    const int64_t s = l + t * dil - pad_left;
                    if (s < 0 || s >= len) continue;
                    const uint16_t *xr = x + (b * len + s) * cin;
                    for (int64_t ci = 0; ci < cin; ++ci) {
                        float v = or_f16_to_f32(xr[ci]);
                        if (alpha) v = or_f16_to_f32(or_f32_to_f16(snake1(v, alpha[ci], brecip[ci])));
                        xs[ci] = v;
                    }
                    for (int64_t ci = 0; ci < cin; ++ci) {
                        const float xv = xs[ci];
                        const float *wr = wf + (t * cin + ci) * cout;
                        for (int64_t co = 0; co < cout; ++co) acc[co] += xv * wr[co];
                    }
                }
                uint16_t *yr = y + (b * len + l) * cout;
                const uint16_t *rr = res ? res + (b * len + l) * cout : NULL;
                for (int64_t co = 0; co < cout; ++co) {
                    float v = acc[co];
                    if (bias) v += or_f16_to_f32(bias[co]);
                    if (scale) v = v * scale[co];  /* ConvNeXt's gamma (codec.rs:193) */
                    if (rr) v += or_f16_to_f32(rr[co]);
                    if (act == 1) v = tanhf(v);
                    if (act == 2) v = or_gelu_erf(v);
                    if (act == 3) v = v < -1.0f ? -1.0f : (v > 1.0f ? 1.0f : v);
                    yr[co] = or_f32_to_f16(v);
                }
            }
        free(acc);
        free(xs);
    }
    free(wf);
}

void or_conv1d_nlc_f16(const uint16_t *x, const uint16_t *w_tap, const uint16_t *bias,
                       const float *alpha, const float *brecip, const uint16_t *res,
                       uint16_t *y, int64_t lanes, int64_t len, int64_t cin, int64_t cout,
                       int64_t k, int64_t dil, int64_t pad_left, int32_t act_tanh) {
    or_conv1d_nlc_f16_ex(x, w_tap, bias, alpha, brecip, res, y, lanes, len, cin, cout, k, dil,
                         pad_left, act_tanh ? 1 : 0, NULL);
}

/* ------------------------------------------------------------------ a5 transposed conv */

/* torch/candle ConvTranspose1d by its definition (scatter form), then the trailing k - stride
 * outputs dropped: causal_conv_transpose1d, crates/tts-nn/src/lib.rs:962-982. NLC: x [len, cin],
 * w [cin, cout, k], y [len*stride, cout]. Double precision; this is the independent definition
 * the polyphase weight algebra (transpose_tap_weight) is checked against. */
void or_conv_transpose1d_causal_f64(const double *x, const double *w_iok, const double *bias,
                                    double *y, int64_t len, int64_t cin, int64_t cout,
                                    int64_t k, int64_t stride) {
    const int64_t out_len = len * stride;
    for (int64_t o = 0; o < out_len; ++o)
        for (int64_t co = 0; co < cout; ++co) y[o * cout + co] = bias ? bias[co] : 0.0;
    for (int64_t l = 0; l < len; ++l)
        for (int64_t j = 0; j < k; ++j) {
            const int64_t o = l * stride + j;
            if (o >= out_len) continue; /* the cropped tail */
            for (int64_t ci = 0; ci < cin; ++ci) {
                const double xv = x[l * cin + ci];
                for (int64_t co = 0; co < cout; ++co)
                    y[o * cout + co] += xv * w_iok[(ci * cout + co) * k + j];
            }
        }
}

/* ------------------------------------------------------------------ blocked SGEMM */

/* C[m,n] (+)= A[m,k] B[k,n], row-major, f32. The CPU baseline's GEMM: candle's CPU matmul is
 * the `gemm` crate (Cargo.lock:1061-1084), a packed, register-blocked kernel; this is the same
 * structure (B packed in 16-wide strips, A in 6-tall strips, a 6x16 register tile), threaded
 * over row blocks. */
#define GEMM_MR 6
#define GEMM_NR 16
#define GEMM_KC 256
#define GEMM_MC 96
#define GEMM_NC 3072

typedef float v8f __attribute__((vector_size(32)));

static void gemm_micro(int64_t kc, const float *ap, const float *bp, float *c, int64_t ldc,
                       int64_t mr, int64_t nr) {
    v8f acc[GEMM_MR][2];
    for (int r = 0; r < GEMM_MR; ++r) {
        acc[r][0] = (v8f){0, 0, 0, 0, 0, 0, 0, 0};
        acc[r][1] = acc[r][0];
    }
    for (int64_t p = 0; p < kc; ++p) {
        v8f b0, b1;
        memcpy(&b0, bp + p * GEMM_NR, 32);
        memcpy(&b1, bp + p * GEMM_NR + 8, 32);
        const float *a = ap + p * GEMM_MR;
        for (int r = 0; r < GEMM_MR; ++r) {
            const v8f av = (v8f){a[r], a[r], a[r], a[r], a[r], a[r], a[r], a[r]};
            acc[r][0] += av * b0;
            acc[r][1] += av * b1;
        }
    }
    for (int64_t r = 0; r < mr; ++r) {
        float tmp[16];
        memcpy(tmp, &acc[r][0], 32);
        memcpy(tmp + 8, &acc[r][1], 32);
        for (int64_t j = 0; j < nr; ++j) c[r * ldc + j] += tmp[j];
    }
}

void or_sgemm(const float *a, const float *b, float *c, int64_t m, int64_t n, int64_t k,
              int32_t accumulate) {
    if (!accumulate) memset(c, 0, sizeof(float) * (size_t)(m * n));
    if (m == 0 || n == 0 || k == 0) return;
    const int64_t nc_max = GEMM_NC;
    float *bpack = (float *)aligned_alloc(64, sizeof(float) * (size_t)(GEMM_KC * nc_max));
#pragma omp parallel
    {
        float *apack = (float *)aligned_alloc(64, sizeof(float) * (size_t)(GEMM_MC * GEMM_KC));
        for (int64_t jc = 0; jc < n; jc += nc_max) {
            const int64_t nc = (n - jc < nc_max) ? n - jc : nc_max;
            const int64_t nstrips = (nc + GEMM_NR - 1) / GEMM_NR;
            for (int64_t pc = 0; pc < k; pc += GEMM_KC) {
                const int64_t kc = (k - pc < GEMM_KC) ? k - pc : GEMM_KC;
#pragma omp for schedule(static)
                for (int64_t s = 0; s < nstrips; ++s) {
                    float *dst = bpack + s * GEMM_NR * kc;
                    const int64_t j0 = jc + s * GEMM_NR;
                    const int64_t w = (nc - s * GEMM_NR < GEMM_NR) ? nc - s * GEMM_NR : GEMM_NR;
                    for (int64_t p = 0; p < kc; ++p) {
                        const float *src = b + (pc + p) * n + j0;
                        int64_t j = 0;
                        for (; j < w; ++j) dst[p * GEMM_NR + j] = src[j];
                        for (; j < GEMM_NR; ++j) dst[p * GEMM_NR + j] = 0.0f;
                    }
                }
#pragma omp for schedule(dynamic, 1)
                for (int64_t ic = 0; ic < m; ic += GEMM_MC) {
                    const int64_t mc = (m - ic < GEMM_MC) ? m - ic : GEMM_MC;
                    const int64_t mstrips = (mc + GEMM_MR - 1) / GEMM_MR;
                    for (int64_t s = 0; s < mstrips; ++s) {
                        float *dst = apack + s * GEMM_MR * kc;
                        const int64_t i0 = ic + s * GEMM_MR;
                        const int64_t h = (mc - s * GEMM_MR < GEMM_MR) ? mc - s * GEMM_MR : GEMM_MR;
                        for (int64_t p = 0; p < kc; ++p) {
                            int64_t r = 0;
                            for (; r < h; ++r) dst[p * GEMM_MR + r] = a[(i0 + r) * k + pc + p];
                            for (; r < GEMM_MR; ++r) dst[p * GEMM_MR + r] = 0.0f;
                        }
                    }
                    for (int64_t sn = 0; sn < nstrips; ++sn) {
                        const int64_t j0 = jc + sn * GEMM_NR;
                        const int64_t w = (nc - sn * GEMM_NR < GEMM_NR) ? nc - sn * GEMM_NR : GEMM_NR;
                        for (int64_t sm = 0; sm < mstrips; ++sm) {
                            const int64_t i0 = ic + sm * GEMM_MR;
                            const int64_t h = (mc - sm * GEMM_MR < GEMM_MR) ? mc - sm * GEMM_MR : GEMM_MR;
                            gemm_micro(kc, apack + sm * GEMM_MR * kc, bpack + sn * GEMM_NR * kc,
                                       c + i0 * n + j0, n, h, w);
                        }
                    }
                }
                /* the implicit barrier of `omp for` keeps bpack stable until every row block
                 * has consumed it */
            }
        }
        free(apack);
    }
    free(bpack);
}

/* conv1d_gemm_whole's CPU route, crates/tts-nn/src/lib.rs:818-860 (via causal_conv1d_gemm /
 * centered_conv1d_gemm, lib.rs:704-767): per lane, the tap-major im2col [k*cin, len], then
 * w_tap [cout, k*cin] @ cols, then + bias. Chunking (lib.rs:787-816) is exact by the
 * reference's own argument and is not restated. */
void or_conv1d_ncl_gemm_f32(const float *x, const float *w_tm, const float *bias, float *y,
                            int64_t lanes, int64_t cin, int64_t cout, int64_t len, int64_t k,
                            int64_t dil, int64_t pad_left) {
    float *cols = (float *)malloc(sizeof(float) * (size_t)(k * cin * len));
    for (int64_t b = 0; b < lanes; ++b) {
        or_im2col_tap_major_f32(x + b * cin * len, cols, cin, len, k, dil, pad_left);
        float *yb = y + b * cout * len;
        or_sgemm(w_tm, cols, yb, cout, len, k * cin, 0);
        if (bias)
            for (int64_t co = 0; co < cout; ++co)
                for (int64_t l = 0; l < len; ++l) yb[co * len + l] += bias[co];
    }
    free(cols);
}

/* nlc::causal_conv1d's CPU route, crates/tts-nn/src/nlc.rs:102-131, one lane: pad the length
 * axis by (k-1)*dil, concatenate the k shifted views on the channel axis into [len, k*cin],
 * one GEMM against w [k*cin, cout], then broadcast-add the bias. */
void or_conv1d_nlc_cat_gemm_f32(const float *x, const float *w_tap, const float *bias,
                                float *y, int64_t len, int64_t cin, int64_t cout, int64_t k,
                                int64_t dil) {
    const int64_t pad = (k - 1) * dil;
    if (k == 1) {
        or_sgemm(x, w_tap, y, len, cout, cin, 0);
    } else {
        float *wide = (float *)malloc(sizeof(float) * (size_t)(len * k * cin));
#pragma omp parallel for schedule(static)
        for (int64_t l = 0; l < len; ++l)
            for (int64_t t = 0; t < k; ++t) {
                const int64_t s = l + t * dil - pad;
                float *dst = wide + l * k * cin + t * cin;
                if (s < 0) memset(dst, 0, sizeof(float) * (size_t)cin);
                else memcpy(dst, x + s * cin, sizeof(float) * (size_t)cin);
            }
        or_sgemm(wide, w_tap, y, len, cout, k * cin, 0);
        free(wide);
    }
    if (bias) {
#pragma omp parallel for schedule(static)
        for (int64_t l = 0; l < len; ++l)
            for (int64_t co = 0; co < cout; ++co) y[l * cout + co] += bias[co];
    }
}

/* ------------------------------------------------------------------ a8 RMSNorm */

/* candle_nn::ops::rms_norm (called at crates/tts-nn/src/lib.rs:1002), believed CPU semantics
 * (candle-nn 0.10.2 is not vendored): f32 sum of squares in index order,
 * m = sqrt(sum/dim + eps), y = (x / m) * gamma. Pinned by f64 and closed-form tests
 * (tests/test_oracle_norm_rope.py); candle's own rounding points are unpinned. */
void or_rms_norm_f32(const float *x, const float *gamma, float *y, int64_t rows, int64_t dim,
                     float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * dim;
        float ss = 0.0f;
        for (int64_t i = 0; i < dim; ++i) ss += xr[i] * xr[i];
        const float m = sqrtf(ss / (float)dim + eps);
        for (int64_t i = 0; i < dim; ++i) y[r * dim + i] = (xr[i] / m) * gamma[i];
    }
}

/* The same for f16 storage: m is converted to f16 and both the divide and the gamma multiply
 * round to f16 (half's arithmetic: widen, operate in f32, round). */
void or_rms_norm_f16(const uint16_t *x, const uint16_t *gamma, uint16_t *y, int64_t rows,
                     int64_t dim, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t *xr = x + r * dim;
        float ss = 0.0f;
        for (int64_t i = 0; i < dim; ++i) {
            const float v = or_f16_to_f32(xr[i]);
            ss += v * v;
        }
        const float m = or_f16_to_f32(or_f32_to_f16(sqrtf(ss / (float)dim + eps)));
        for (int64_t i = 0; i < dim; ++i) {
            const float q = or_f16_to_f32(or_f32_to_f16(or_f16_to_f32(xr[i]) / m));
            y[r * dim + i] = or_f32_to_f16(q * or_f16_to_f32(gamma[i]));
        }
    }
}

void or_rms_norm_f64(const double *x, const double *gamma, double *y, int64_t rows, int64_t dim,
                     double eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const double *xr = x + r * dim;
        double ss = 0.0;
        for (int64_t i = 0; i < dim; ++i) ss += xr[i] * xr[i];
        const double m = sqrt(ss / (double)dim + eps);
        for (int64_t i = 0; i < dim; ++i) y[r * dim + i] = xr[i] / m * gamma[i];
    }
}

/* ------------------------------------------------------------------ a9 RoPE */

/* rope_pairs / rope_table_f32, crates/tts-nn/src/lib.rs:1178-1205: freq_i = 1/base^(2i/D),
 * phase = t*freq_i in f64, cos/sin rounded to f32; [len, D/2]. */
void or_rope_table_f32(int64_t len, int64_t head_dim, double base, float *cos_out,
                       float *sin_out) {
    const int64_t half = head_dim / 2;
    for (int64_t t = 0; t < len; ++t)
        for (int64_t i = 0; i < half; ++i) {
            const double freq = 1.0 / pow(base, 2.0 * (double)i / (double)head_dim);
            const double phase = (double)t * freq;
            cos_out[t * half + i] = (float)cos(phase);
            sin_out[t * half + i] = (float)sin(phase);
        }
}

/* candle_nn::rotary_emb::rope (half-split; called at crates/qwen3tts/src/qwen3.rs:384-387), one
 * position per row: o_i = x_i c - x_{i+D/2} s, o_{i+D/2} = x_{i+D/2} c + x_i s. x is
 * [rows, heads, D] and row r sits at position pos[r] (the reference passes one `start` per
 * batch; a position per lane is the 48-lane generalisation). */
static inline void rope_row(const float *x, const float *c, const float *s, float *o,
                            int64_t half) {
    for (int64_t i = 0; i < half; ++i) {
        const float x1 = x[i], x2 = x[i + half];
        const float a = x1 * c[i], b = x2 * s[i];
        const float e = x2 * c[i], f = x1 * s[i];
        o[i] = a - b;
        o[i + half] = e + f;
    }
}

void or_rope_halfsplit_f32(const float *x, const float *cos_t, const float *sin_t,
                           const int32_t *pos, float *y, int64_t rows, int64_t heads,
                           int64_t head_dim) {
    const int64_t half = head_dim / 2;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t h = 0; h < heads; ++h) {
            const int64_t o = (r * heads + h) * head_dim;
            rope_row(x + o, cos_t + (int64_t)pos[r] * half, sin_t + (int64_t)pos[r] * half,
                     y + o, half);
        }
}

/* f16 storage: widened, rotated in f32, rounded once. */
void or_rope_halfsplit_f16(const uint16_t *x, const float *cos_t, const float *sin_t,
                           const int32_t *pos, uint16_t *y, int64_t rows, int64_t heads,
                           int64_t head_dim) {
    const int64_t half = head_dim / 2;
    float xf[1024], of[1024];
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t h = 0; h < heads; ++h) {
            const int64_t o = (r * heads + h) * head_dim;
            for (int64_t i = 0; i < head_dim; ++i) xf[i] = or_f16_to_f32(x[o + i]);
            rope_row(xf, cos_t + (int64_t)pos[r] * half, sin_t + (int64_t)pos[r] * half, of,
                     half);
            for (int64_t i = 0; i < head_dim; ++i) y[o + i] = or_f32_to_f16(of[i]);
        }
}

/* ------------------------------------------------------------------ a10/a11 */

/* The composed fallback of crates/qwen3tts/src/qwen3.rs:358-394 (what qk_rope_f32 replaces,
 * tested that way at crates/tts-nn/src/qkrope.rs:211-244), one decode position per lane:
 * q and k heads RMS-normed over head_dim with norms[0] / norms[1], half-split RoPE at pos[b],
 * k (roped) and v written to the f16 caches [b, n_kv, cap, D] at pos[b] with RNE
 * (`to_dtype(F16)` then `slice_set`). qkv is [b, (heads + 2*n_kv) * D]; q_out [b, heads, D];
 * k_out [b, n_kv, D] is the f32 k before the cast. */
void or_qk_norm_rope_append_f32(const float *qkv, const float *norms, const float *cos_t,
                                const float *sin_t, const int32_t *pos, float *q_out,
                                float *k_out, uint16_t *kcache, uint16_t *vcache, int64_t b,
                                int64_t heads, int64_t n_kv, int64_t head_dim, int64_t cap,
                                float eps) {
    const int64_t width = (heads + 2 * n_kv) * head_dim;
    const int64_t half = head_dim / 2;
    float nrm[1024];
    for (int64_t bi = 0; bi < b; ++bi) {
        const float *row = qkv + bi * width;
        const float *c = cos_t + (int64_t)pos[bi] * half;
        const float *s = sin_t + (int64_t)pos[bi] * half;
        for (int64_t h = 0; h < heads + n_kv; ++h) {
            const int is_q = h < heads;
            or_rms_norm_f32(row + h * head_dim, norms + (is_q ? 0 : head_dim), nrm, 1, head_dim,
                            eps);
            if (is_q) {
                rope_row(nrm, c, s, q_out + (bi * heads + h) * head_dim, half);
            } else {
                const int64_t kh = h - heads;
                float *ko = k_out + (bi * n_kv + kh) * head_dim;
                rope_row(nrm, c, s, ko, half);
                const float *vs = row + (heads + n_kv + kh) * head_dim;
                const int64_t dst = ((bi * n_kv + kh) * cap + pos[bi]) * head_dim;
                for (int64_t d = 0; d < head_dim; ++d) {
                    kcache[dst + d] = or_f32_to_f16(ko[d]);
                    vcache[dst + d] = or_f32_to_f16(vs[d]);
                }
            }
        }
    }
}

/* cache.k.slice_set(&k.to_dtype(F16), 2, pos), crates/qwen3tts/src/qwen3.rs:389-392: k, v
 * [b, n_kv, D] written at [bi, h, pos[bi], :]; nothing else is touched. */
void or_kv_append_f32(const float *k, const float *v, const int32_t *pos, uint16_t *kcache,
                      uint16_t *vcache, int64_t b, int64_t n_kv, int64_t head_dim, int64_t cap) {
    for (int64_t bi = 0; bi < b; ++bi)
        for (int64_t h = 0; h < n_kv; ++h) {
            const int64_t src = (bi * n_kv + h) * head_dim;
            const int64_t dst = ((bi * n_kv + h) * cap + pos[bi]) * head_dim;
            for (int64_t d = 0; d < head_dim; ++d) {
                kcache[dst + d] = or_f32_to_f16(k[src + d]);
                vcache[dst + d] = or_f32_to_f16(v[src + d]);
            }
        }
}

void or_kv_append_f16(const uint16_t *k, const uint16_t *v, const int32_t *pos,
                      uint16_t *kcache, uint16_t *vcache, int64_t b, int64_t n_kv,
                      int64_t head_dim, int64_t cap) {
    for (int64_t bi = 0; bi < b; ++bi)
        for (int64_t h = 0; h < n_kv; ++h) {
            const int64_t src = (bi * n_kv + h) * head_dim;
            const int64_t dst = ((bi * n_kv + h) * cap + pos[bi]) * head_dim;
            memcpy(kcache + dst, k + src, 2 * (size_t)head_dim);
            memcpy(vcache + dst, v + src, 2 * (size_t)head_dim);
        }
}

/* ------------------------------------------------------------------ f-1 decode attention */

/* attn::decode_attention's CPU path (crates/tts-nn/src/attn.rs:18-73): Scores::cpu_fwd
 * (attn.rs:85-126: -inf outside [window_start, span), else the d-ordered f32 dot q.k with f16
 * cache values widened), candle_nn::ops::softmax_last_dim (called at attn.rs:62; candle-nn 0.10.2,
 * not vendored: max over the row, exp(x - max), their sum in order, each divided by the sum), and
 * Weighted::cpu_fwd (attn.rs:189-226: dst[d] += p * v[p][d] in position order over [0, span)).
 * q [b, n_kv, gqa, D]; caches [b, n_kv, cap, D] as f16 bits (kv_f16 = 1) or f32; span and
 * window start per lane. */
static float or_cache_at(const void *c, int kv_f16, int64_t i) {
    return kv_f16 ? or_f16_to_f32(((const uint16_t *)c)[i]) : ((const float *)c)[i];
}

void or_decode_attention_f32(const float *q, const void *kc, const void *vc, int kv_f16, float *out,
                             int64_t b, int64_t n_kv, int64_t gqa, int64_t hd, int64_t cap,
                             const int32_t *span, const int32_t *wstart) {
#pragma omp parallel for schedule(static)
    for (int64_t bh = 0; bh < b * n_kv; ++bh) {
        const int64_t bi = bh / n_kv;
        const int64_t sp = span[bi], ws = wstart ? wstart[bi] : 0;
        float *sc = (float *)malloc(sizeof(float) * (size_t)(sp > 0 ? sp : 1));
        for (int64_t g = 0; g < gqa; ++g) {
            const float *qr = q + (bh * gqa + g) * hd;
            for (int64_t p = 0; p < sp; ++p) {
                if (p < ws) {
                    sc[p] = -INFINITY;
                    continue;
                }
                float acc = 0.0f;
                for (int64_t d = 0; d < hd; ++d) acc += qr[d] * or_cache_at(kc, kv_f16, (bh * cap + p) * hd + d);
                sc[p] = acc;
            }
            float mx = -INFINITY;
            for (int64_t p = 0; p < sp; ++p) mx = sc[p] > mx ? sc[p] : mx;
            float sum = 0.0f;
            for (int64_t p = 0; p < sp; ++p) {
                sc[p] = expf(sc[p] - mx);
                sum += sc[p];
            }
            for (int64_t p = 0; p < sp; ++p) sc[p] /= sum;
            float *o = out + (bh * gqa + g) * hd;
            for (int64_t d = 0; d < hd; ++d) o[d] = 0.0f;
            for (int64_t p = 0; p < sp; ++p)
                for (int64_t d = 0; d < hd; ++d) o[d] += sc[p] * or_cache_at(vc, kv_f16, (bh * cap + p) * hd + d);
        }
        free(sc);
    }
}

/* ------------------------------------------------------------------ a12-a14 */

/* `[m,k] f16 x [k,n] f16 -> [m,n] f32` with f32 accumulation in k order: the arithmetic
 * gemm_skinny_f16 + sum_splits_f32 define (crates/tts-nn/src/mtl.rs:1078-1150), restated
 * without the split. */
void or_gemm_f16_f32acc(const uint16_t *a, const uint16_t *b_kn, float *c, int64_t m, int64_t k,
                        int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        float *cr = c + i * n;
        for (int64_t j = 0; j < n; ++j) cr[j] = 0.0f;
        for (int64_t p = 0; p < k; ++p) {
            const float av = or_f16_to_f32(a[i * k + p]);
            const uint16_t *br = b_kn + p * n;
            for (int64_t j = 0; j < n; ++j) cr[j] += av * or_f16_to_f32(br[j]);
        }
    }
}

void or_gemm_f16_f64(const uint16_t *a, const uint16_t *b_kn, double *c, int64_t m, int64_t k,
                     int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        double *cr = c + i * n;
        for (int64_t j = 0; j < n; ++j) cr[j] = 0.0;
        for (int64_t p = 0; p < k; ++p) {
            const double av = (double)or_f16_to_f32(a[i * k + p]);
            const uint16_t *br = b_kn + p * n;
            for (int64_t j = 0; j < n; ++j) cr[j] += av * (double)or_f16_to_f32(br[j]);
        }
    }
}

/* SwigluMul::cpu_fwd, crates/tts-nn/src/fused.rs:298-320: (x / (1 + exp(-x))) * u. */
void or_swiglu_mul_f32(const float *g, const float *u, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float x = g[i];
        const float e = expf(-x);
        const float den = 1.0f + e;
        y[i] = (x / den) * u[i];
    }
}

/* ------------------------------------------------------------------ a15 Q8_0 */

/* GGML block_q8_0 as candle stores it (the quantize_onto at crates/tts-nn/src/lib.rs:484-486):
 * per row, K/32 blocks of {f16 d; i8 qs[32]} = 34 bytes. Quantize (believed candle
 * BlockQ8_0::from_float, ggml's reference semantics): amax = max|x|, d = amax/127,
 * id = d != 0 ? 1/d : 0, qs = round-half-away(x*id), d stored as f16. */
void or_q8_0_quantize(const float *w, uint8_t *blocks, int64_t rows, int64_t k) {
    const int64_t nb = k / 32;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t bi = 0; bi < nb; ++bi) {
            const float *src = w + r * k + bi * 32;
            uint8_t *blk = blocks + (r * nb + bi) * 34;
            float amax = 0.0f;
            for (int j = 0; j < 32; ++j) {
                const float a = fabsf(src[j]);
                amax = a > amax ? a : amax;
            }
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const uint16_t dh = or_f32_to_f16(d);
            memcpy(blk, &dh, 2);
            for (int j = 0; j < 32; ++j) {
                const float q = roundf(src[j] * id);
                blk[2 + j] = (uint8_t)(int8_t)q;
            }
        }
}

/* w[n, k] = qs[n][k/32][k%32] * f32(d[n][k/32]). */
void or_q8_0_dequantize(const uint8_t *blocks, float *w, int64_t rows, int64_t k) {
    const int64_t nb = k / 32;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < k; ++c) {
            const uint8_t *blk = blocks + (r * nb + c / 32) * 34;
            uint16_t dh;
            memcpy(&dh, blk, 2);
            w[r * k + c] = (float)(int8_t)blk[2 + c % 32] * or_f16_to_f32(dh);
        }
}

/* Believed candle CPU QMatMul::forward for Q8_0 weights: activations quantized to Q8_0 per
 * 32-block (the vec-dot type), then per output the block dots as i32, each scaled
 * `sum_i as f32 * d_w * d_x` and summed in block order (BlockQ8_0::vec_dot's scalar form).
 * y [m, n] = x [m, k] . W[n, k]^T. Parity against candle itself is unpinned. */
void or_q8_0_matmul_w8a8(const float *x, const uint8_t *wblocks, float *y, int64_t m, int64_t k,
                         int64_t n) {
    const int64_t nb = k / 32;
    uint8_t *xq = (uint8_t *)malloc((size_t)(m * nb * 34));
    or_q8_0_quantize(x, xq, m, k);
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            float sumf = 0.0f;
            for (int64_t bi = 0; bi < nb; ++bi) {
                const uint8_t *wb = wblocks + (j * nb + bi) * 34;
                const uint8_t *xb = xq + (i * nb + bi) * 34;
                int32_t si = 0;
                for (int q = 0; q < 32; ++q)
                    si += (int32_t)(int8_t)wb[2 + q] * (int32_t)(int8_t)xb[2 + q];
                uint16_t dw, dx;
                memcpy(&dw, wb, 2);
                memcpy(&dx, xb, 2);
                const float t = ((float)si * or_f16_to_f32(dw)) * or_f16_to_f32(dx);
                sumf += t;
            }
            y[i * n + j] = sumf;
        }
    free(xq);
}

/* x . dequant(W)^T in double: the unquantized-activation target both GPU modes are held to. */
void or_q8_0_matmul_f64(const float *x, const uint8_t *wblocks, double *y, int64_t m, int64_t k,
                        int64_t n) {
    const int64_t nb = k / 32;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            double acc = 0.0;
            for (int64_t bi = 0; bi < nb; ++bi) {
                const uint8_t *wb = wblocks + (j * nb + bi) * 34;
                uint16_t dw;
                memcpy(&dw, wb, 2);
                const double d = (double)or_f16_to_f32(dw);
                for (int q = 0; q < 32; ++q)
                    acc += (double)x[i * k + bi * 32 + q] * ((double)(int8_t)wb[2 + q] * d);
            }
            y[i * n + j] = acc;
        }
}

/* ------------------------------------------------------------------ a17 */

/* abs_and_rel, crates/tts-nn/src/lib.rs:1239-1248: max|a-b| (in f32), and that over max|b|. */
void or_abs_and_rel(const float *a, const float *b, int64_t n, float *abs_out, float *rel_out) {
    float mx = 0.0f, sc = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        const float d = fabsf(a[i] - b[i]);
        if (d > mx || d != d) mx = (d != d) ? INFINITY : d;
        const float s = fabsf(b[i]);
        if (s > sc) sc = s;
    }
    *abs_out = mx;
    *rel_out = sc > 0.0f ? mx / sc : 0.0f;
}

/* ------------------------------------------------------------------ f-3 codec front half */

/* Rvq::decode's lookups (crates/qwen3tts/src/codec.rs:296-313): per row, the picked codebook rows
 * summed in codebook order (sum = q0; sum = sum + q1; ...) in f32, for books [0, n_first) and
 * [n_first, n_books) side by side, each rounded to f16. */
void or_rvq_lookup_sum_f16(const int32_t *codes, const float *books, int64_t n_books, int64_t n_first,
                           int64_t size, int64_t dim, uint16_t *out, int64_t rows) {
    for (int64_t r = 0; r < rows; ++r)
        for (int half = 0; half < 2; ++half) {
            const int64_t b0 = half ? n_first : 0, b1 = half ? n_books : n_first;
            for (int64_t d = 0; d < dim; ++d) {
                float s = 0.0f;
                for (int64_t b = b0; b < b1; ++b) {
                    const float v = books[(b * size + codes[r * n_books + b]) * dim + d];
                    s = b == b0 ? v : s + v;
                }
                out[r * 2 * dim + half * dim + d] = or_f32_to_f16(s);
            }
        }
}

/* ConvNext's depthwise conv and LayerNorm (codec.rs:186-188): nlc::depthwise (crates/tts-nn/src/
 * nlc.rs:236-256: left zero padding of k-1, taps accumulated oldest first, then the bias) and
 * layer_norm_plain (lib.rs:1030-1035: mean, centred, mean of squares, divide by sqrt(var + eps))
 * times the weight plus the bias (lib.rs:1020). f16 in and out, f32 inside. */
void or_depthwise_layernorm_f16(const uint16_t *x, const float *taps, const float *bias, const float *lnw,
                                const float *lnb, float eps, uint16_t *y, int64_t lanes, int64_t len,
                                int64_t C, int64_t K) {
    float *h = (float *)malloc(sizeof(float) * (size_t)C);
    for (int64_t b = 0; b < lanes; ++b)
        for (int64_t l = 0; l < len; ++l) {
            for (int64_t c = 0; c < C; ++c) {
                float acc = 0.0f;
                for (int64_t t = 0; t < K; ++t) {
                    const int64_t s = l - (K - 1) + t;
                    const float xv = s >= 0 ? or_f16_to_f32(x[(b * len + s) * C + c]) : 0.0f;
                    const float term = xv * taps[c * K + t];
                    acc = t == 0 ? term : acc + term;
                }
                h[c] = acc + bias[c];
            }
            float mean = 0.0f;
            for (int64_t c = 0; c < C; ++c) mean += h[c];
            mean /= (float)C;
            float var = 0.0f;
            for (int64_t c = 0; c < C; ++c) {
                h[c] = h[c] - mean;
                var += h[c] * h[c];
            }
            var /= (float)C;
            const float den = sqrtf(var + eps);
            for (int64_t c = 0; c < C; ++c) y[(b * len + l) * C + c] = or_f32_to_f16((h[c] / den) * lnw[c] + lnb[c]);
        }
    free(h);
}

/* Stack::forward's prefill attention (crates/qwen3tts/src/qwen3.rs:420-443) over one sequence
 * per lane with a sliding window, no QK-norm (the codec transformer's form, qwen3.rs:358-400):
 * q and k half-split-roped in f32 at their positions (candle_nn::rotary_emb::rope as called at
 * qwen3.rs:384-387), scores = (q . k) * scale (qwen3.rs:433-436), the mask of causal_window_mask
 * (lib.rs:1210-1224), softmax_last_dim (max, exp(s - max), in-order sum, divide), then probs . v.
 * Two f16 storage points the GPU adds (its matrix-core operands): the roped q and k, and
 * exp(s - max); the division by the sum of those rounded weights comes after the weighted sum,
 * which is softmax-then-product reassociated. qkv [lanes, T, (heads + 2 n_kv) D] f16 (q heads,
 * k heads, v heads); out [lanes, T, heads D] f16. */
void or_window_attention_prefill_f16(const uint16_t *qkv, const float *cos_t, const float *sin_t,
                                     uint16_t *out, int64_t lanes, int64_t T, int64_t heads, int64_t n_kv,
                                     int64_t D, int64_t window, float scale) {
    const int64_t width = (heads + 2 * n_kv) * D, half = D / 2, gqa = heads / n_kv;
    float *k = (float *)malloc(sizeof(float) * (size_t)(T * D));
    float *q = (float *)malloc(sizeof(float) * (size_t)D);
    float *xin = (float *)malloc(sizeof(float) * (size_t)D);
    float *p = (float *)malloc(sizeof(float) * (size_t)T);
    for (int64_t b = 0; b < lanes; ++b)
        for (int64_t h = 0; h < heads; ++h) {
            const int64_t kh = h / gqa;
            /* roped k, stored in f16 (the GPU's matrix-core operand) */
            for (int64_t j = 0; j < T; ++j) {
                const uint16_t *kr = qkv + (b * T + j) * width + (heads + kh) * D;
                for (int64_t d = 0; d < D; ++d) xin[d] = or_f16_to_f32(kr[d]);
                rope_row(xin, cos_t + j * half, sin_t + j * half, k + j * D, half);
                for (int64_t d = 0; d < D; ++d) k[j * D + d] = or_f16_to_f32(or_f32_to_f16(k[j * D + d]));
            }
            for (int64_t i = 0; i < T; ++i) {
                const uint16_t *qr = qkv + (b * T + i) * width + h * D;
                for (int64_t d = 0; d < D; ++d) xin[d] = or_f16_to_f32(qr[d]);
                rope_row(xin, cos_t + i * half, sin_t + i * half, q, half);
                for (int64_t d = 0; d < D; ++d) q[d] = or_f16_to_f32(or_f32_to_f16(q[d]));
                const int64_t lo = i + 1 > window ? i + 1 - window : 0;
                float mx = -INFINITY;
                for (int64_t j = lo; j <= i; ++j) {
                    float s = 0.0f;
                    for (int64_t d = 0; d < D; ++d) s += q[d] * k[j * D + d];
                    p[j] = s * scale;
                    mx = p[j] > mx ? p[j] : mx;
                }
                /* softmax's exp(s - max) in f16 (the weighted sum's operand), normalised after */
                float sum = 0.0f;
                for (int64_t j = lo; j <= i; ++j) {
                    p[j] = or_f16_to_f32(or_f32_to_f16(expf(p[j] - mx)));
                    sum += p[j];
                }
                for (int64_t d = 0; d < D; ++d) {
                    float o = 0.0f;
                    for (int64_t j = lo; j <= i; ++j)
                        o += p[j] * or_f16_to_f32(qkv[(b * T + j) * width + (heads + n_kv + kh) * D + d]);
                    out[(b * T + i) * heads * D + h * D + d] = or_f32_to_f16(o / sum);
                }
            }
        }
    free(k);
    free(q);
    free(xin);
    free(p);
}

/* rms_norm over f16 rows in f32 (lib.rs:1000-1003 on f32 activations), one rounding out. */
void or_rms_norm_rows_f16(const uint16_t *x, const float *gamma, uint16_t *y, int64_t rows, int64_t dim,
                          float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        float ss = 0.0f;
        for (int64_t i = 0; i < dim; ++i) {
            const float v = or_f16_to_f32(x[r * dim + i]);
            ss += v * v;
        }
        const float m = sqrtf(ss / (float)dim + eps);
        for (int64_t i = 0; i < dim; ++i) y[r * dim + i] = or_f32_to_f16((or_f16_to_f32(x[r * dim + i]) / m) * gamma[i]);
    }
}

/* silu(gate) * up (fused::swiglu_mul, crates/tts-nn/src/fused.rs:298-320) over f16 [rows, 2 ffn]. */
void or_swiglu_rows_f16(const uint16_t *gu, uint16_t *y, int64_t rows, int64_t ffn) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t j = 0; j < ffn; ++j) {
            const float g = or_f16_to_f32(gu[r * 2 * ffn + j]), u = or_f16_to_f32(gu[r * 2 * ffn + ffn + j]);
            y[r * ffn + j] = or_f32_to_f16((g / (1.0f + expf(-g))) * u);
        }
}
