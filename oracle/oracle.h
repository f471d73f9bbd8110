/*
 * CPU oracle for the tts-nn fused-op hot path. TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU arithmetic (drmhse/dream-tts, crates/tts-nn,
 * candle CPU path), used by tests/ as the parity checker and by bench.py's cpu_baseline leg as
 * the timed CPU baseline. The product (libdtts.so) never links, loads or calls anything here.
 * Each function cites the reference file:line it restates. Paths are relative to the reference
 * repository root.
 *
 * Conventions: row-major; NCL = [lanes, C, L], NLC = [lanes, L, C]; f16 values travel as
 * uint16_t bit patterns and are rounded to nearest-even (the `half` crate's from_f32).
 */
#ifndef DTTS_ORACLE_H
#define DTTS_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- f16 storage points (half 2.7.1 from_f32 / to_f32: IEEE binary16, RNE) ---- */
uint16_t or_f32_to_f16(float f);
float or_f16_to_f32(uint16_t h);
void or_f32_to_f16_array(const float *src, uint16_t *dst, int64_t n);
void or_f16_to_f32_array(const uint16_t *src, float *dst, int64_t n);

/* ---- a1/a2 snake ---- */
void or_snake_ncl_f32(const float *x, const float *alpha, const float *brecip, float *y,
                      int64_t lanes, int64_t chan, int64_t len);
void or_snake_nlc_f32(const float *x, const float *alpha, const float *brecip, float *y,
                      int64_t rows, int64_t chan);
void or_snake_nlc_f16(const uint16_t *x, const float *alpha, const float *brecip, uint16_t *y,
                      int64_t rows, int64_t chan);
void or_snake_ncl_f16(const uint16_t *x, const float *alpha, const float *brecip, uint16_t *y,
                      int64_t lanes, int64_t chan, int64_t len);
void or_snake_nlc_f64(const double *x, const double *alpha, const double *brecip, double *y,
                      int64_t rows, int64_t chan);
void or_snake_folded_f32(const float *x, float *y, int64_t n);
void or_snake_alpha_f32(const float *x, const float *alpha, float *y, int64_t lanes, int64_t chan,
                        int64_t len);

/* ---- a7 im2col gather (bit-exact) ---- */
void or_im2col_tap_major_f32(const float *x, float *cols, int64_t cin, int64_t len, int64_t k,
                             int64_t dil, int64_t pad_left);

/* ---- weight layouts ---- */
void or_tap_weight_f32(const float *w_oik, float *w_kio, int64_t cout, int64_t cin, int64_t k);
void or_tap_major_weight_f32(const float *w_oik, float *w_tm, int64_t cout, int64_t cin,
                             int64_t k);
void or_transpose_tap_weight_f32(const float *w_iok, float *w_tap, int64_t cin, int64_t cout,
                                 int64_t k, int64_t stride);
void or_transpose_bias_f32(const float *b, float *out, int64_t cout, int64_t stride);

/* ---- a3/a4 NLC causal-or-offset conv, direct ---- */
void or_conv1d_nlc_f32(const float *x, const float *w_tap, const float *bias, const float *alpha,
                       const float *brecip, const float *res, float *y, int64_t lanes,
                       int64_t len, int64_t cin, int64_t cout, int64_t k, int64_t dil,
                       int64_t pad_left);
void or_conv1d_nlc_f64(const double *x, const double *w_tap, const double *bias,
                       const double *alpha, const double *brecip, const double *res, double *y,
                       int64_t lanes, int64_t len, int64_t cin, int64_t cout, int64_t k,
                       int64_t dil, int64_t pad_left);
float or_gelu_erf(float x);
void or_conv1d_nlc_f16_ex(const uint16_t *x, const uint16_t *w_tap, const uint16_t *bias,
                          const float *alpha, const float *brecip, const uint16_t *res,
                          uint16_t *y, int64_t lanes, int64_t len, int64_t cin, int64_t cout,
                          int64_t k, int64_t dil, int64_t pad_left, int32_t act,
                          const float *scale);
void or_conv1d_nlc_f16(const uint16_t *x, const uint16_t *w_tap, const uint16_t *bias,
                       const float *alpha, const float *brecip, const uint16_t *res,
                       uint16_t *y, int64_t lanes, int64_t len, int64_t cin, int64_t cout,
                       int64_t k, int64_t dil, int64_t pad_left, int32_t act_tanh);

/* ---- a5 transposed conv, reference forms ---- */
void or_conv_transpose1d_causal_f64(const double *x, const double *w_iok, const double *bias,
                                    double *y, int64_t len, int64_t cin, int64_t cout,
                                    int64_t k, int64_t stride);

/* ---- a6 NCL conv through im2col + GEMM, and the NLC cat + GEMM route (CPU baseline) ---- */
void or_sgemm(const float *a, const float *b, float *c, int64_t m, int64_t n, int64_t k,
              int32_t accumulate);
void or_conv1d_ncl_gemm_f32(const float *x, const float *w_tm, const float *bias, float *y,
                            int64_t lanes, int64_t cin, int64_t cout, int64_t len, int64_t k,
                            int64_t dil, int64_t pad_left);
void or_conv1d_nlc_cat_gemm_f32(const float *x, const float *w_tap, const float *bias,
                                float *y, int64_t len, int64_t cin, int64_t cout, int64_t k,
                                int64_t dil);

/* ---- a8 RMSNorm ---- */
void or_rms_norm_f32(const float *x, const float *gamma, float *y, int64_t rows, int64_t dim,
                     float eps);
void or_rms_norm_f16(const uint16_t *x, const uint16_t *gamma, uint16_t *y, int64_t rows,
                     int64_t dim, float eps);
void or_rms_norm_f64(const double *x, const double *gamma, double *y, int64_t rows, int64_t dim,
                     double eps);

/* ---- a9 RoPE ---- */
void or_rope_table_f32(int64_t len, int64_t head_dim, double base, float *cos_out,
                       float *sin_out);
void or_rope_halfsplit_f32(const float *x, const float *cos_t, const float *sin_t,
                           const int32_t *pos, float *y, int64_t rows, int64_t heads,
                           int64_t head_dim);
void or_rope_halfsplit_f16(const uint16_t *x, const float *cos_t, const float *sin_t,
                           const int32_t *pos, uint16_t *y, int64_t rows, int64_t heads,
                           int64_t head_dim);

/* ---- a10/a11 QK-norm + RoPE + KV append, and the plain append ---- */
void or_qk_norm_rope_append_f32(const float *qkv, const float *norms, const float *cos_t,
                                const float *sin_t, const int32_t *pos, float *q_out,
                                float *k_out, uint16_t *kcache, uint16_t *vcache, int64_t b,
                                int64_t heads, int64_t n_kv, int64_t head_dim, int64_t cap,
                                float eps);
void or_kv_append_f32(const float *k, const float *v, const int32_t *pos, uint16_t *kcache,
                      uint16_t *vcache, int64_t b, int64_t n_kv, int64_t head_dim, int64_t cap);
void or_kv_append_f16(const uint16_t *k, const uint16_t *v, const int32_t *pos,
                      uint16_t *kcache, uint16_t *vcache, int64_t b, int64_t n_kv,
                      int64_t head_dim, int64_t cap);

/* ---- f-1 decode attention over the KV cache ---- */
void or_decode_attention_f32(const float *q, const void *kc, const void *vc, int kv_f16, float *out,
                             int64_t b, int64_t n_kv, int64_t gqa, int64_t hd, int64_t cap,
                             const int32_t *span, const int32_t *wstart);

/* ---- a12-a14 f16 projections ---- */
void or_gemm_f16_f32acc(const uint16_t *a, const uint16_t *b_kn, float *c, int64_t m, int64_t k,
                        int64_t n);
void or_gemm_f16_f64(const uint16_t *a, const uint16_t *b_kn, double *c, int64_t m, int64_t k,
                     int64_t n);
void or_swiglu_mul_f32(const float *g, const float *u, float *y, int64_t n);

/* ---- a15 Q8_0 ---- */
void or_q8_0_quantize(const float *w, uint8_t *blocks, int64_t rows, int64_t k);
void or_q8_0_dequantize(const uint8_t *blocks, float *w, int64_t rows, int64_t k);
void or_q8_0_matmul_w8a8(const float *x, const uint8_t *wblocks, float *y, int64_t m, int64_t k,
                         int64_t n);
void or_q8_0_matmul_f64(const float *x, const uint8_t *wblocks, double *y, int64_t m, int64_t k,
                        int64_t n);

/* ---- a17 parity metric ---- */
void or_abs_and_rel(const float *a, const float *b, int64_t n, float *abs_out, float *rel_out);

#ifdef __cplusplus
}
#endif
void or_rvq_lookup_sum_f16(const int32_t *codes, const float *books, int64_t n_books, int64_t n_first,
                           int64_t size, int64_t dim, uint16_t *out, int64_t rows);
void or_depthwise_layernorm_f16(const uint16_t *x, const float *taps, const float *bias, const float *lnw,
                                const float *lnb, float eps, uint16_t *y, int64_t lanes, int64_t len,
                                int64_t C, int64_t K);

void or_window_attention_prefill_f16(const uint16_t *qkv, const float *cos_t, const float *sin_t,
                                     uint16_t *out, int64_t lanes, int64_t T, int64_t heads, int64_t n_kv,
                                     int64_t D, int64_t window, float scale);
void or_rms_norm_rows_f16(const uint16_t *x, const float *gamma, uint16_t *y, int64_t rows, int64_t dim,
                          float eps);
void or_swiglu_rows_f16(const uint16_t *gu, uint16_t *y, int64_t rows, int64_t ffn);

#endif
