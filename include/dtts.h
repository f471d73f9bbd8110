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

/* The folded snakes, f32 (x, y any layout / [lanes, chan, len]; x == y allowed; full-precision
 * sine, as the SnakeBeta f32 forms):
 *   dtts_snake_folded_f32: y = x + sin^2(x) over n elements, for inputs whose alpha is folded into
 *     the preceding conv's output weights. Replaces fused::snake_folded / SnakeFolded
 *     (crates/tts-nn/src/fused.rs:17-91, 501-508; kernel snake_folded_f32, mtl.rs:128-143).
 *   dtts_snake_alpha_f32: u = alpha[c] * x, y = u + sin^2(u), the half-folded snake whose 1/alpha
 *     lives in the next conv's input weights. Replaces fused::snake_alpha / SnakeAlpha
 *     (fused.rs:93-184, 510-522; kernel snake_alpha_f32, mtl.rs:145-166) and tts_nn::snake
 *     (lib.rs:1075-1083); the reference takes lanes == 1, any lane count here. */
int dtts_snake_folded_f32(const float *x, float *y, int64_t n, hipStream_t stream);
int dtts_snake_alpha_f32(const float *x, const float *alpha, float *y, int64_t lanes, int64_t chan, int64_t len,
                         hipStream_t stream);

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
 * alignments take a direct (slow, exact-semantics) kernel. act: 0 none, 1 tanh, 2 GELU
 * (erf form, gelu_exact, crates/tts-nn/src/lib.rs:1129-1131), 3 clamp to [-1, 1] (Codec::forward's
 * clamp, crates/qwen3tts/src/codec.rs:433-436). With out_scale the sum is
 *   s[l, n] = residual[l, n] + out_scale[n] * (bias[n] + sum ...), the scaled term rounded in
 * f32 before the add. */
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
    const float *out_scale; /* [cout] factor on (sum + bias) before the residual is added, or NULL:
                               y = residual + scale * (bias + sum), ConvNeXt's gamma and LayerScale */
} dtts_conv_desc;

int dtts_conv1d_nlc_f16_ex(const dtts_conv_desc *desc, hipStream_t stream);

/* The same conv at NlcConv's own precision: every operand f32 (x, w, bias, residual, y_pre, y),
 * f32 accumulation -- NlcConv::cpu_fwd / nlc_conv_f32 (crates/tts-nn/src/nlcconv.rs:33-73,
 * mtl.rs:937-1065; the reference's op is f32-only, nlcconv.rs:185-198) with any lane count.
 * act: 0, 1 (tanh) or 3 (clamp). Matrix cores when cin % 16 == 0, cout % 32 == 0, k <= 7,
 * (k-1)*dilation <= 64 and x, w are 16-byte aligned; a direct kernel otherwise. */
int dtts_conv1d_nlc_f32_ex(const dtts_conv_desc *desc, hipStream_t stream);

/* The same f32 conv at f32 accuracy on the f16 matrix cores (NlcConv, crates/tts-nn/src/
 * nlcconv.rs:15-198; the route the f32 codec takes). The weight is split once at load:
 * dtts_conv_split_weight scales the tap-major f32 weight [cout, k*cin] by a power of two 2^s (its
 * largest magnitude then in [2^14, 2^15)) and writes [cout, k*3*cin] f16, per tap [hi | hi | lo]
 * of the scaled values, and w_inv = 2^-s; it synchronises `stream` once (to read the weight's
 * largest magnitude). Each dtts_conv1d_nlc_f32_split call then splits x (and the residual) into
 * f16 hi/lo pairs in the workspace, computes sum(xh wh + xl wh + xh wl) in f32 (the dropped xl wl
 * is ~2^-22 of a term), adds bias and residual in f32, applies the epilogue SnakeBeta at f32
 * accuracy, and writes f32 y (and y_pre). desc->w is the split weight; every other operand is
 * f32 as dtts_conv1d_nlc_f32_ex takes it. Taken for cin and cout multiples of 32, k <= 7 with
 * (k-1)*dilation <= 64 (cout a multiple of 96 for k > 2), len * cout * 4 < 2^31, no prologue
 * SnakeBeta, act 0 and no out_scale; anything else returns DTTS_ERR_UNSUPPORTED. Every operand is 16-byte aligned, and
 * w_inv is the power of two dtts_conv_split_weight returned (DTTS_ERR_INVALID otherwise). */
size_t dtts_conv_split_weight_bytes(int64_t cout, int64_t k, int64_t cin);
int dtts_conv_split_weight(const float *w_tm, int64_t cout, int64_t k, int64_t cin, void *w_split,
                           float *w_inv, hipStream_t stream);
size_t dtts_conv1d_nlc_f32_split_workspace_bytes(const dtts_conv_desc *desc);
int dtts_conv1d_nlc_f32_split(const dtts_conv_desc *desc, float w_inv, void *workspace,
                              size_t workspace_bytes, hipStream_t stream);

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

/* The codec's residual unit in one launch (ResidualUnit::forward, crates/qwen3tts/src/codec.rs:
 * 215-229; nlc::snake_conv_residual, crates/tts-nn/src/nlc.rs:40-68, fuses its second half):
 *
 *   h  = f16(conv_k(SnakeBeta1(x)) + b1)     causal, pad (k-1)*dilation
 *   h2 = f16(SnakeBeta2(h))
 *   y_pre = f16(conv_1(h2) + b2 + x)
 *   y  = f16(SnakeBeta_out(y_pre))           (y_pre itself when out_alpha == NULL)
 *
 * x, y, y_pre [lanes, len, channels] f16; w1 [C, k*C] and w2 [C, C] tap-major f16; b1, b2 f16;
 * SnakeBeta parameters f32. h and h2 stay on chip: two activation passes instead of five. Taken
 * for channels 96 and 192, k <= 7, (k-1)*dilation <= 64, 16-byte aligned x/y/y_pre/w1/w2/b2;
 * anything else returns DTTS_ERR_UNSUPPORTED (compose two dtts_conv1d_nlc_f16_ex calls). */
typedef struct dtts_ru_desc {
    int64_t lanes, len, channels, k, dilation;
    const void *x;
    const float *act1_alpha, *act1_brecip;
    const void *w1, *b1;
    const float *act2_alpha, *act2_brecip;
    const void *w2, *b2;
    void *y_pre;
    const float *out_alpha, *out_brecip;
    void *y;
} dtts_ru_desc;

int dtts_residual_unit_nlc_f16(const dtts_ru_desc *desc, hipStream_t stream);

/* 1 when dtts_residual_unit_nlc_f16 takes this descriptor, else 0 (no device work). */
int dtts_residual_unit_supported(const dtts_ru_desc *desc);

/* ------------------------------------------------------------------ a6/a7 channel-major f32 conv */

/* The channel-major conv in f32: the same fused form as dtts_conv1d_nlc_f16_ex, with x
 * [lanes, cin, len], residual / y_pre / y [lanes, cout, len], f32 everywhere (bias, weights
 * [cout, k*cin] tap-major, snake parameters), SnakeBeta with full-precision sine, and no rounding
 * between the fused steps. Replaces centered_conv1d_gemm / causal_conv1d_gemm /
 * conv1d_gemm_whole (crates/tts-nn/src/lib.rs:704-860: im2col gather, w_tap @ cols, + bias),
 * chunking included (it is exact there and needless here). pad_left = (k-1)*dilation is causal,
 * (k-1)*dilation/2 the centred form. Tiled on the f32 matrix cores when cin % 16 == 0,
 * cout % 64 == 0, k <= 7 and (k-1)*dilation <= 64; a direct kernel otherwise. */
int dtts_conv1d_ncl_f32_ex(const dtts_conv_desc *desc, hipStream_t stream);

/* im2col::im2col_tap_major / im2col_centered (crates/tts-nn/src/im2col.rs:47-166) for one lane:
 * cols[(t*cin + c)*len + l] = x[c*len + l + t*dilation - pad_left], 0 outside [0, len). Bit-exact.
 * The conv kernels never build this matrix; it is exported for parity and for callers that
 * want it. */
int dtts_im2col_tap_major_f32(const float *x, float *cols, int64_t cin, int64_t len, int64_t k,
                              int64_t dilation, int64_t pad_left, hipStream_t stream);

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

/* ------------------------------------------------------------------ a8-a11 norm, RoPE, KV cache */

/* RMSNorm over the last dim (rows x dim): y = (x / sqrt(mean(x^2) + eps)) * gamma, the sum of
 * squares in f32. Replaces rms_norm -> candle_nn::ops::rms_norm (crates/tts-nn/src/lib.rs:
 * 1000-1003). The f16 form keeps candle's f16 rounding points: m = sqrt(..) rounded to f16, then
 * x/m and *gamma each rounded to f16. */
int dtts_rms_norm_f32(const float *x, const float *gamma, float *y, int64_t rows, int64_t dim,
                      float eps, hipStream_t stream);
int dtts_rms_norm_f16(const dtts_f16 *x, const dtts_f16 *gamma, dtts_f16 *y, int64_t rows,
                      int64_t dim, float eps, hipStream_t stream);

/* rope_table_f32 / rope_pairs (crates/tts-nn/src/lib.rs:1178-1205), host: cos/sin [len, D/2],
 * phase t / base^(2i/D) in f64, rounded to f32. */
int dtts_rope_table_f32(int64_t len, int64_t head_dim, double base, float *cos_out,
                        float *sin_out);

/* Half-split RoPE (candle_nn::rotary_emb::rope as called at crates/qwen3tts/src/qwen3.rs:384-387;
 * not the interleaved rope_i): x, y [rows, heads, D]; row r is at position pos[r] (a HOST array
 * of `rows` int32, each in [0, table_len)); o_i = x_i c - x_{i+D/2} s, o_{i+D/2} = x_{i+D/2} c +
 * x_i s with each product rounded (no FMA). The reference passes one start per batch; a position
 * per lane is the batched-decode generalisation. rows <= 256. */
int dtts_rope_halfsplit_f32(const float *x, const float *cos_t, const float *sin_t,
                            const int32_t *pos, float *y, int64_t rows, int64_t heads,
                            int64_t head_dim, int64_t table_len, hipStream_t stream);
int dtts_rope_halfsplit_f16(const dtts_f16 *x, const float *cos_t, const float *sin_t,
                            const int32_t *pos, dtts_f16 *y, int64_t rows, int64_t heads,
                            int64_t head_dim, int64_t table_len, hipStream_t stream);

/* QK-norm, RoPE and the KV-cache write of one decode position per lane, in one launch: replaces
 * qkrope::apply / QkRope (crates/tts-nn/src/qkrope.rs:26-182, kernel qk_rope_f32 at mtl.rs:
 * 773-838) for t = 1, with a position per lane. qkv [b, (heads + 2*n_kv) * D] (q heads, then k,
 * then v); norms [2, D] f32 (q's weight, then k's); cos/sin [table_len, D/2]; pos a HOST int32[b]
 * (each < min(cap, table_len), checked before anything is enqueued, as qkrope.rs:40-44 checks
 * start + t <= capacity). Outputs: q_out [b, heads, D]; k_out [b, n_kv, D] f32 (optional, the
 * roped k before its f16 cast: the reference's f32_kv side output); kcache, vcache
 * [b, n_kv, cap, D] f16 written in place at [bi, h, pos[bi], :] (k roped, v as given, RNE) and
 * nothing else. D even and <= 128, b <= 256. */
int dtts_qk_norm_rope_kv_append_f32(const float *qkv, const float *norms, const float *cos_t,
                                    const float *sin_t, const int32_t *pos, float *q_out,
                                    float *k_out, dtts_f16 *kcache, dtts_f16 *vcache, int64_t b,
                                    int64_t heads, int64_t n_kv, int64_t head_dim, int64_t cap,
                                    int64_t table_len, float eps, hipStream_t stream);
int dtts_qk_norm_rope_kv_append_f16(const dtts_f16 *qkv, const float *norms, const float *cos_t,
                                    const float *sin_t, const int32_t *pos, dtts_f16 *q_out,
                                    float *k_out, dtts_f16 *kcache, dtts_f16 *vcache, int64_t b,
                                    int64_t heads, int64_t n_kv, int64_t head_dim, int64_t cap,
                                    int64_t table_len, float eps, hipStream_t stream);

/* qkrope::apply (crates/tts-nn/src/qkrope.rs:19-69; kernel qk_rope_f32, mtl.rs:773-838) with its
 * own signature: qkv [b, t, (heads + 2*n_kv) * D] f32 (q heads, then k, then v); norms [2, D] f32
 * (q's weight, then k's); cos/sin [table_len, D/2]; the caches [b, n_kv, cap, D] f16 (a lane window
 * of a larger cache is a pointer into it) are written in place at positions start .. start + t - 1
 * (k normed and roped, v as given, RNE) and nowhere else. Out: q_out [b, heads, t, D] f32 and, with
 * f32_kv, k_f32 and v_f32 [b, n_kv, t, D] f32 (pass both or neither). start + t must not exceed cap
 * ("positions exceed", qkrope.rs:40-44) nor table_len; checked before anything is enqueued.
 * D even and <= 128. */
int dtts_qkrope_apply_f32(const float *qkv, const float *norms, const float *cos_t, const float *sin_t,
                          dtts_f16 *kcache, dtts_f16 *vcache, int64_t heads, int64_t start, float eps,
                          float *q_out, float *k_f32, float *v_f32, int64_t b, int64_t t, int64_t n_kv,
                          int64_t head_dim, int64_t cap, int64_t table_len, hipStream_t stream);

/* The KV append alone: cache.k.slice_set(&k.to_dtype(F16), 2, start) and the same for v
 * (crates/qwen3tts/src/qwen3.rs:389-392), one position per lane. k, v [b, n_kv, D]; caches
 * [b, n_kv, cap, D] f16 written at pos[bi] (HOST int32[b], each < cap), RNE, bit-exact. */
int dtts_kv_append_f32(const float *k, const float *v, const int32_t *pos, dtts_f16 *kcache,
                       dtts_f16 *vcache, int64_t b, int64_t n_kv, int64_t head_dim, int64_t cap,
                       hipStream_t stream);
int dtts_kv_append_f16(const dtts_f16 *k, const dtts_f16 *v, const int32_t *pos,
                       dtts_f16 *kcache, dtts_f16 *vcache, int64_t b, int64_t n_kv,
                       int64_t head_dim, int64_t cap, hipStream_t stream);

/* ------------------------------------------------------------------ f-1 decode attention */

/* Decode attention reading the KV cache in place: replaces attn::decode_attention
 * (crates/tts-nn/src/attn.rs:18-73), whose CPU path (Scores, softmax_last_dim, Weighted:
 * attn.rs:85-126, 62, 189-226) defines the result. q [b, n_kv, gqa, D] f32 with any scale already
 * folded in; caches [b, n_kv, cap, D] (f16, or f32 for the _f32 form); out [b, n_kv, gqa, D] f32,
 * caller-allocated: out[b, h, g, :] = sum_p softmax_p(q[b,h,g] . k[b,h,p]) v[b,h,p] over
 * p in [window_start[b], span[b]). span and window_start are HOST int32[b] arrays (window_start
 * may be NULL: 0); the reference's one span and window start per batch are the case of equal
 * entries. Checked before anything is enqueued: span <= cap (attn.rs:31), window_start < span.
 * D in {64, 128}, gqa in {1, 2, 4, 8}, b <= 256. The caches are only read.
 * workspace (device, 16-byte aligned) may be NULL; given at least
 * dtts_decode_attention_workspace_bytes(b, n_kv, gqa, D, max_b(span - window_start)) bytes, long
 * spans are split over several workgroups and merged by a second launch (the reference has no
 * such argument: its op allocates; a shim passes a cached buffer). Bytes needed are 0 when no
 * window exceeds 512 positions. */
size_t dtts_decode_attention_workspace_bytes(int64_t b, int64_t n_kv, int64_t gqa,
                                             int64_t head_dim, int64_t max_window);
int dtts_decode_attention_f16(const float *q, const dtts_f16 *kcache, const dtts_f16 *vcache,
                              float *out, int64_t b, int64_t n_kv, int64_t gqa, int64_t head_dim,
                              int64_t cap, const int32_t *span, const int32_t *window_start,
                              void *workspace, size_t ws_bytes, hipStream_t stream);
int dtts_decode_attention_f32(const float *q, const float *kcache, const float *vcache, float *out,
                              int64_t b, int64_t n_kv, int64_t gqa, int64_t head_dim, int64_t cap,
                              const int32_t *span, const int32_t *window_start, void *workspace,
                              size_t ws_bytes, hipStream_t stream);

/* ------------------------------------------------------------------ f-2 decoder stack step */

/* One decode step (t = 1) of a Qwen3 decoder stack over all its layers: replaces Stack::forward
 * (crates/qwen3tts/src/qwen3.rs:294-467) on its decode path with f16 weights (Proj::Half) and an
 * f16 KV cache: per layer rms_norm, the fused QKV projection, QK-norm + RoPE + cache append (or
 * RoPE and q * 1/sqrt(head_dim) without QK-norm), decode attention over the cache (the last
 * `window` positions when set), the output projection added to the residual stream (times
 * attn_scale with LayerScale), rms_norm, gate|up with SiLU*mul, the down projection added to
 * the residual stream (times mlp_scale); then the final rms_norm. Activations are f32 as in the
 * reference, each projection's input rounded to f16 as Proj::forward casts it
 * (crates/tts-nn/src/lib.rs:517). Geometries: the talker (dim 2048, 28 layers, 16/8 heads, D 128,
 * ffn 6144), the code predictor (dim 1024, 5 layers, ffn 3072) and the codec's windowed
 * transformer (dim 512, 8 layers, 16/16 heads, D 64, LayerScale, window 72) all fit. */
typedef struct dtts_stack_geometry {
    int64_t dim, layers, heads, n_kv, head_dim, ffn;
    float eps;
    double rope_base;
    int32_t qk_norm, layer_scale; /* Geometry's flags (qwen3.rs:16-28) */
    int64_t window;               /* sliding window in positions; 0 = none */
    int64_t capacity;             /* RoPE table length (Stack::load's capacity); caches may be shorter */
} dtts_stack_geometry;

/* The layers' weight kinds (Stack::load's `how`, crates/qwen3tts/src/qwen3.rs:228-250; Weight,
 * crates/tts-nn/src/lib.rs:403-430). Every kind but F16 keeps f32 caches, as Stack::load does. */
#define DTTS_WEIGHT_F16 0     /* Proj::Half: f16 [out, in] projections, f16 caches */
#define DTTS_WEIGHT_F32 1     /* Proj::Dense: f32 [out, in] projections, f32 caches */
#define DTTS_WEIGHT_Q8_0 2    /* Proj::Quant(Q8_0): dtts_q8_0_repack'd blocks of the [out, in] weight; the
                                 f32 activations quantized per 32-block (candle CPU's vec_dot); f32 caches */
#define DTTS_WEIGHT_Q8_0_A32 3 /* the same blocks with the f32 activations unquantized (the dequantized
                                  product a GPU QMatMul takes); f32 caches */

/* Device pointers, kept (not copied) by dtts_stack_create; norms and scales f32, projections in
 * the checkpoint's [out, in] layout (rows of the stack's weight kind: f16, f32, or Q8_0 blocks
 * repacked by dtts_q8_0_repack), 16-byte aligned. */
typedef struct dtts_stack_layer {
    const float *attn_norm, *ffn_norm; /* [dim] */
    const void *wqkv;                  /* [(heads + 2 n_kv) head_dim, dim]: q, k, v rows (Layer::load's cat) */
    const void *wo;                    /* [dim, heads head_dim] */
    const void *w_gateup;              /* [2 ffn, dim]: gate rows, then up rows */
    const void *wdown;                 /* [dim, ffn] */
    const float *qk_norms;             /* [2, head_dim]: q's weight times 1/sqrt(head_dim), then k's (qk_norm) */
    const float *attn_scale, *mlp_scale; /* [dim] (layer_scale) */
} dtts_stack_layer;

/* One layer's cache (State's Cache, qwen3.rs:122-126): k and v [lanes, n_kv, cap, head_dim], f16
 * for a DTTS_WEIGHT_F16 stack and f32 for the other kinds (Stack::load's kv dtype). */
typedef struct dtts_stack_cache {
    void *k, *v;
} dtts_stack_cache;

typedef struct dtts_stack dtts_stack;

/* Checks the geometry and weights, builds the RoPE table (rope_table_f32, crates/tts-nn/src/
 * lib.rs:1178-1205) on the current device. */
int dtts_stack_create(const dtts_stack_geometry *geo, const dtts_stack_layer *layers, const float *final_norm,
                      dtts_stack **out);
/* The same with the layers' weight kind (DTTS_WEIGHT_*): Stack::load(.., how, ..). dtts_stack_create
 * is DTTS_WEIGHT_F16. F32 layers take dim, heads*head_dim and ffn multiples of 64; Q8_0 layers
 * multiples of 256 (the packed layout), with the gate and up rows quantized and repacked as one
 * [2 ffn, dim] weight (each row's blocks are its own, so this is the two QMatMuls). The prefill
 * branch (dtts_stack_prefill) takes F16 stacks only. */
int dtts_stack_create_as(const dtts_stack_geometry *geo, const dtts_stack_layer *layers, const float *final_norm,
                         int32_t how, dtts_stack **out);
void dtts_stack_destroy(dtts_stack *stack);

/* Device scratch bytes for a step of `lanes` lanes over caches of capacity `cap`. */
size_t dtts_stack_workspace_bytes(const dtts_stack *stack, int64_t lanes, int64_t cap);

#define DTTS_STACK_GRAPH 1 /* capture the step's launches once into a HIP graph and replay it */

/* x [lanes, dim] f32 (the embedded tokens) -> out [lanes, dim] f32 (the normed hidden state);
 * caches[layers]: layer i's k and v, written at each lane's position and read over its window;
 * pos a HOST int32[lanes], each < cap (checked before anything is enqueued, as Stack::forward
 * refuses start + t > capacity). lanes <= 64. Projection outputs follow Proj::Half's routing by lane
 * count: f32 for 8, 16, .. 48 lanes (skinny::eligible), f16-rounded otherwise (one lane included),
 * as candle's f16 matmul gives them. The reference advances one position for the whole
 * batch; a position per lane is the batched-decode generalisation. With DTTS_STACK_GRAPH the
 * launches are captured on the first call and replayed while x, out, the caches, lanes, cap and
 * the workspace stay the same (any change captures again). Calls on one stack must be ordered
 * (one stream at a time), as the reference's device-global encoder is (crates/tts-nn/src/
 * lib.rs:76-83). */
int dtts_stack_decode(dtts_stack *stack, const float *x, float *out, const dtts_stack_cache *caches, int64_t lanes,
                      int64_t cap, const int32_t *pos, void *workspace, size_t ws_bytes, int32_t flags,
                      hipStream_t stream);

/* Stack::forward at t >= 2, the prefill branch (crates/qwen3tts/src/qwen3.rs:294-467, :415-444)
 * for lanes sharing one start (State::width): the code predictor's [talker_hidden, code0_embed]
 * per frame (talker.rs:417-420) and the talker's prompt. x [lanes, t, dim] f32 -> out
 * [lanes, t, dim] f32; caches written at start .. start + t - 1 (k roped, v as given, f16) and
 * read below start; the new positions attend over their own f32 k and v. Projections follow
 * Proj::Half's routing by row count (lanes * t): at most 48 rows and a multiple of 8, f32 outputs
 * (skinny::eligible, crates/tts-nn/src/skinny.rs:123-131); otherwise f16 outputs, as candle's f16
 * matmul gives (lib.rs:516-529). start + t <= cap <= capacity and <= 16000, lanes * t <= 2^20. */
size_t dtts_stack_prefill_workspace_bytes(const dtts_stack *stack, int64_t lanes, int64_t t);
int dtts_stack_prefill(dtts_stack *stack, const float *x, float *out, const dtts_stack_cache *caches, int64_t lanes,
                       int64_t t, int64_t start, int64_t cap, void *workspace, size_t workspace_bytes,
                       hipStream_t stream);

/* ------------------------------------------------------------------ f-3 codec front half */

/* Rvq::decode's lookups (crates/qwen3tts/src/codec.rs:296-313) for both quantizer stacks at
 * once: out[r] = [sum_{b < n_first} books[b][codes[r, b]] | sum_{b >= n_first} books[b][codes[r, b]]],
 * each sum in codebook order in f32, stored f16. codes [rows, n_books] int32 (device); books
 * [n_books, book_size, dim] f32, already divided by the clamped cluster usage as Rvq::load folds
 * them (codec.rs:275-282); out [rows, 2 * dim]. The two output projections are then one conv
 * (k = 1) over the concatenated width: Ws and Wa side by side along the input channels. Codes
 * outside [0, book_size) are clamped on the device (the reference's index_select refuses them;
 * callers with host codes check them first, as the front-half driver does). */
int dtts_rvq_lookup_sum_f16(const int32_t *codes, const float *codebooks, int64_t n_books, int64_t n_first,
                            int64_t book_size, int64_t dim, dtts_f16 *out, int64_t rows, hipStream_t stream);

/* ConvNext::forward's depthwise conv and LayerNorm (codec.rs:186-188): per lane and channel c,
 *   h[l, c] = sum_{t < k} x[l - (k-1) + t, c] * taps[c, t] + bias[c]   (zero before the start;
 *             nlc::depthwise, crates/tts-nn/src/nlc.rs:236-256)
 *   y[l, :] = (h - mean) / sqrt(var + eps) * ln_weight + ln_bias       (layer_norm, lib.rs:1006-1035)
 * x, y [lanes, len, channels] f16 (not in place), taps [channels, k] f32 (the [C, 1, k] weight),
 * bias, ln_weight, ln_bias [channels] f32. channels % 8 == 0, <= 2048; k <= 64. */
int dtts_depthwise_layernorm_nlc_f16(const dtts_f16 *x, const float *taps, const float *bias,
                                     const float *ln_weight, const float *ln_bias, float eps, dtts_f16 *y,
                                     int64_t lanes, int64_t len, int64_t channels, int64_t k, hipStream_t stream);

/* RMSNorm over f16 rows with f32 arithmetic and one rounding out (rms_norm, crates/tts-nn/src/
 * lib.rs:1000-1003, on the f32 activations the codec transformer runs in); gamma f32 [dim]. */
int dtts_rms_norm_rows_f16(const dtts_f16 *x, const float *gamma, dtts_f16 *y, int64_t rows, int64_t dim,
                           float eps, hipStream_t stream);

/* y[r, j] = silu(gu[r, j]) * gu[r, ffn + j] (fused::swiglu_mul, crates/tts-nn/src/fused.rs:298-320,
 * on a gate|up projection's [rows, 2 ffn] output), f16 in and out, f32 inside. ffn % 8 == 0. */
int dtts_swiglu_rows_f16(const dtts_f16 *gate_up, dtts_f16 *y, int64_t rows, int64_t ffn, hipStream_t stream);

/* Stack::forward's prefill attention (crates/qwen3tts/src/qwen3.rs:420-443) over whole
 * sequences with a sliding window and no QK-norm (the codec transformer, codec.rs:337-349):
 * q and k half-split-roped at their positions 0..len-1 (cos/sin [table_len, D/2], rope_table_f32),
 * scores (q . k) * scale, key j visible to query i when i - window < j <= i (causal_window_mask,
 * lib.rs:1210-1224), softmax, weighted v. qkv [lanes, len, (heads + 2 n_kv) D] f16 (q heads, k
 * heads, v heads); out [lanes, len, heads D] f16. D = 64, 1 <= window <= 192, len <= table_len. */
int dtts_window_attention_prefill_f16(const dtts_f16 *qkv, const float *cos_t, const float *sin_t, int64_t table_len,
                                      dtts_f16 *out, int64_t lanes, int64_t len, int64_t heads, int64_t n_kv,
                                      int64_t head_dim, int64_t window, float scale, hipStream_t stream);

/* The codec's front half (Codec::forward up to the waveform stack, crates/qwen3tts/src/codec.rs:
 * 401-424): codes -> RVQ lookups and output projections (Rvq::decode, codec.rs:296-313) -> causal
 * pre_conv -> input projection -> the sliding-window transformer (Stack::forward's prefill over
 * the chunk, with LayerScale) -> output projection -> per upsampling ratio, a transposed conv
 * (kernel = stride) and a ConvNeXt block (codec.rs:160-196). Output: the latent the waveform
 * stack (dtts_codec_decode) takes, [lanes, frames * prod(up_ratios), latent_dim] f16. Every
 * activation is f16 in HBM with f32 arithmetic inside each kernel (the reference runs this half
 * in f32); projections are channels-last convs with k = 1. */
#define DTTS_FRONT_MAX_LAYERS 16
#define DTTS_FRONT_MAX_UP 4

typedef struct dtts_codec_front_geometry {
    int64_t n_books, n_first, book_size, book_dim; /* 16, 1, 2048, 256 (cfg.rs codec: QUANTIZERS...) */
    int64_t codebook_dim;                         /* 512: the width the two stacks are summed at */
    int64_t latent_dim, pre_kernel;               /* 1024, 3 */
    int64_t tf_dim, tf_layers, tf_heads, tf_n_kv, tf_head_dim, tf_ffn, tf_window; /* 512, 8, 16, 16, 64, 1024, 72 */
    float tf_eps;                                 /* 1e-5 */
    double tf_rope_base;                          /* 1e4 */
    int64_t n_up, up_ratios[DTTS_FRONT_MAX_UP];   /* 2, {2, 2} */
    int64_t dw_kernel;                            /* 7 */
    float ln_eps;                                 /* 1e-6 */
    int64_t max_frames;                           /* RoPE table length: frames per call at most */
} dtts_codec_front_geometry;

/* Device pointers, kept by dtts_codec_front_create. Projections are f16 [out, in]; norms and
 * scales f32. */
typedef struct dtts_codec_front_layer {
    const float *attn_norm, *attn_scale, *ffn_norm, *mlp_scale; /* [tf_dim] */
    const dtts_f16 *wqkv;     /* [(heads + 2 n_kv) D, tf_dim]: q, k, v rows */
    const dtts_f16 *wo;       /* [tf_dim, heads D] */
    const dtts_f16 *w_gateup; /* [2 ffn, tf_dim]: gate rows, then up rows */
    const dtts_f16 *wdown;    /* [tf_dim, ffn] */
} dtts_codec_front_layer;

typedef struct dtts_codec_front_up {
    const dtts_f16 *up_w, *up_b; /* the transposed conv: dtts_transpose_tap_major_weight's layout for
                                    kernel = stride = r ([r C, C]), bias repeated r times */
    const float *dw_taps, *dw_bias, *ln_weight, *ln_bias; /* [C, dw_kernel], [C] x 3 */
    const dtts_f16 *pw1_w, *pw1_b, *pw2_w, *pw2_b;        /* [4C, C], [4C], [C, 4C], [C] */
    const float *gamma;                                   /* [C] */
} dtts_codec_front_up;

typedef struct dtts_codec_front_weights {
    const float *codebooks;        /* [n_books, book_size, book_dim] f32, embedding_sum / clamp(usage) */
    const dtts_f16 *out_proj;      /* [codebook_dim, 2 book_dim]: semantic then acoustic output_proj */
    const dtts_f16 *pre_w, *pre_b; /* [latent, pre_kernel codebook_dim] tap-major, [latent] */
    const dtts_f16 *in_w, *in_b;   /* [tf_dim, latent], [tf_dim] */
    dtts_codec_front_layer layers[DTTS_FRONT_MAX_LAYERS];
    const float *tf_norm;          /* [tf_dim] */
    const dtts_f16 *out_w, *out_b; /* [latent, tf_dim], [latent] */
    dtts_codec_front_up up[DTTS_FRONT_MAX_UP];
} dtts_codec_front_weights;

typedef struct dtts_codec_front dtts_codec_front;

int dtts_codec_front_create(const dtts_codec_front_geometry *geo, const dtts_codec_front_weights *weights,
                            dtts_codec_front **out);
void dtts_codec_front_destroy(dtts_codec_front *front);
size_t dtts_codec_front_workspace_bytes(const dtts_codec_front *front, int64_t lanes, int64_t frames);

/* codes [lanes, frames, n_books] int32 on the HOST (Codec::forward's frames; checked against
 * book_size before anything is enqueued, then staged into the workspace) -> latent f16. */
int dtts_codec_front_decode(const dtts_codec_front *front, const int32_t *codes, dtts_f16 *latent, int64_t lanes,
                            int64_t frames, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------ a12-a14 f16 projections */

/* Decode-shape f16 GEMM, f32 accumulation and output: C[m, n] = A[m, k] . B. Replaces
 * skinny::matmul / gemm_skinny_f16 + sum_splits_f32 (crates/tts-nn/src/skinny.rs:155-165,
 * mtl.rs:1078-1150), which takes m <= 48, m % 8 == 0, k % 32 == 0, n % 64 == 0; the matrix-core
 * kernel here takes m <= 64 (any), k % 64 == 0, n % 16 == 0, 16-byte aligned operands, and any
 * other shape runs a direct kernel. Split-k partials are summed in a fixed order (deterministic).
 *   dtts_gemm_f16_skinny: B = b_kn [k, n], the reference's own operand (Proj::Half's W_t,
 *     crates/tts-nn/src/lib.rs:516-529);
 *   dtts_gemm_f16_nt: B = w_nk^T with w_nk [n, k], the checkpoint's [out, in] layout, so no
 *     load-time transpose is needed; the faster of the two. Its workspace (device, 16-byte
 *     aligned; NULL allowed) lets a projection with few output columns split k over
 *     workgroups as well, the splits' partials summed in split order by a second launch: give
 *     at least dtts_gemm_f16_workspace_bytes(m, k, n, 0) bytes (0 when no split is needed). */
int dtts_gemm_f16_skinny(const dtts_f16 *a, const dtts_f16 *b_kn, float *c, int64_t m, int64_t k,
                         int64_t n, hipStream_t stream);
size_t dtts_gemm_f16_workspace_bytes(int64_t m, int64_t k, int64_t n, int32_t gateup);
int dtts_gemm_f16_nt(const dtts_f16 *a, const dtts_f16 *w_nk, float *c, int64_t m, int64_t k,
                     int64_t n, void *workspace, size_t ws_bytes, hipStream_t stream);

/* dtts_gemm_f16_nt without a workspace argument and without allocating: no counterpart in the
 * reference. It is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The k-range partials live in a
 * library-owned device array of 16 MiB per GPU, held until the process ends; shapes whose
 * dtts_gemm_f16_workspace_bytes(m, k, n, 0) exceeds it are refused (DTTS_ERR_INVALID) before
 * anything is enqueued. Results are bit-identical to dtts_gemm_f16_nt given that workspace. Every
 * call on one GPU shares that array: calls that overlap on one GPU (other streams, other threads)
 * race, so order them. */
int dtts_gemm_f16_nt_noalloc(const dtts_f16 *a, const dtts_f16 *w_nk, float *c, int64_t m, int64_t k,
                             int64_t n, hipStream_t stream);

/* gate|up projection with SwiGLU fused: y[m, j] = silu(g) * u, g = A . Wg^T, u = A . Wu^T, where
 * w_gu [2*ffn, k] holds gate's rows then up's (f16, [out, in]). Replaces
 * swiglu_mul(gate.forward(x), up.forward(x)) at crates/qwen3tts/src/qwen3.rs:454-457. y f32.
 * Workspace as for dtts_gemm_f16_nt, sized by dtts_gemm_f16_workspace_bytes(m, k, ffn, 1). */
int dtts_gemm_f16_gateup_silu(const dtts_f16 *a, const dtts_f16 *w_gu, float *y, int64_t m,
                              int64_t k, int64_t ffn, void *workspace, size_t ws_bytes,
                              hipStream_t stream);

/* Proj::Dense's forward (matmul_2d of f32 activations by an f32 weight, crates/tts-nn/src/
 * lib.rs:438-459, 527) on the checkpoint's [out, in] layout: y[m, n] = x[m, k] . w[n, k]^T, f32
 * throughout, on the f32 matrix cores. m <= 64, k % 32 == 0, n % 64 == 0, x and w 16-byte
 * aligned. k is split into ranges over workgroups when that fills the GPU; the ranges' partials
 * then go to the workspace (dtts_gemm_f32_nt_workspace_bytes, 16-byte aligned; required when
 * nonzero) and a second launch sums them in range order. */
size_t dtts_gemm_f32_nt_workspace_bytes(int64_t m, int64_t k, int64_t n);
int dtts_gemm_f32_nt(const float *x, const float *w, float *y, int64_t m, int64_t k, int64_t n, void *workspace,
                     size_t workspace_bytes, hipStream_t stream);

/* fused::swiglu_mul / SwigluMul (crates/tts-nn/src/fused.rs:289-385): y = (g / (1 + exp(-g))) * u,
 * f32, n elements. */
int dtts_swiglu_mul_f32(const float *g, const float *u, float *y, int64_t n, hipStream_t stream);

/* ------------------------------------------------------------------ a15 Q8_0 */

/* GGML block_q8_0 as candle stores a quantized [out, in] weight (QTensor::quantize_onto,
 * crates/tts-nn/src/lib.rs:480-486): row n is k/32 consecutive 34-byte blocks {f16 d;
 * int8 qs[32]}; w[n, c] = qs[n][c/32][c%32] * d[n][c/32]. */
#define DTTS_Q8_W8A16 0 /* f16 activations times the exact int8 weights, scaled per block */
#define DTTS_Q8_W8A8 1  /* activations quantized to Q8_0 per 32-block first (candle CPU's vec_dot) */
#define DTTS_Q8_W8A32 2 /* f32 activations times the exact int8 weights, scaled per block, at f32
                           precision (the unquantized-activation product); f32 entry points only */

/* Host: quantize f32 [rows, k] (k % 32 == 0) into blocks: d = amax/127, qs = round-half-away(x/d)
 * with the f32 reciprocal, d stored as f16 (BlockQ8_0::from_float). blocks holds rows*k/32*34
 * bytes. */
int dtts_q8_0_quantize(const float *w, void *blocks, int64_t rows, int64_t k);

/* Device: blocks -> f32 [rows, k] (the dequant index math, bit-exact). */
int dtts_q8_0_dequantize_f32(const void *blocks, float *w, int64_t rows, int64_t k,
                             hipStream_t stream);

/* y[m, n] = x[m, k] . dequant(W)^T for the Q8_0 weight W [n, k]: replaces Proj::Quant's
 * QMatMul::forward (crates/tts-nn/src/lib.rs:531). x f16 (16-byte aligned), y f32, m <= 64,
 * n % 16 == 0, k % 32 == 0. mode: DTTS_Q8_W8A16 or DTTS_Q8_W8A8. */
int dtts_gemm_q8_0(const dtts_f16 *x, const void *blocks, float *y, int64_t m, int64_t k,
                   int64_t n, int32_t mode, hipStream_t stream);

/* The same product (QMatMul::forward, lib.rs:531) with an optional device workspace (16-byte
 * aligned, at least dtts_gemm_q8_0_workspace_bytes(m, k, n) bytes; 0 means none is needed): when
 * m > 16, n % 64 == 0 and k % 256 == 0, workgroups of 64 columns share the activation slab in LDS
 * (W8A8: quantised once per workgroup) and k is split into ranges merged in order by a second
 * launch. Without room (or for other shapes) it is dtts_gemm_q8_0. */
size_t dtts_gemm_q8_0_workspace_bytes(int64_t m, int64_t k, int64_t n);
int dtts_gemm_q8_0_ws(const dtts_f16 *x, const void *blocks, float *y, int64_t m, int64_t k, int64_t n,
                      int32_t mode, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Load-time repack of GGML blocks [rows, k/32] into a layout the matrix cores read with 16-byte
 * loads (same bytes, dtts_q8_0_packed_bytes of them, 16-byte aligned): per row, the quantised
 * weights lane-group major (weights 8g .. 8g + 7 of block b at g * (k/32) * 8 + b * 8), then the
 * k/32 f16 scales. k % 256 == 0. */
size_t dtts_q8_0_packed_bytes(int64_t rows, int64_t k);
int dtts_q8_0_repack(const void *blocks, void *packed, int64_t rows, int64_t k, hipStream_t stream);
/* QMatMul::forward (lib.rs:531) on the packed layout, by the A-sharing kernel at every m (bit for
 * bit dtts_gemm_q8_0_ws's result where that kernel runs there). n % 64 == 0, k % 256 == 0,
 * m <= 64; the workspace (dtts_gemm_q8_0_workspace_bytes) is required when nonzero. */
int dtts_gemm_q8_0_packed(const dtts_f16 *x, const void *packed, float *y, int64_t m, int64_t k, int64_t n,
                          int32_t mode, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* The f32-activation forms of the three above, with Proj::forward's own interface: it hands
 * QMatMul::forward the f32 hidden state and takes f32 back for every weight kind
 * (crates/tts-nn/src/lib.rs:509-531, `Proj::Quant(q) => q.forward(x)`). x is f32 [m, k], 16-byte
 * aligned; shapes, workspace and routing as the f16 forms. mode DTTS_Q8_W8A8 quantizes the f32
 * activations per 32-block directly (no f16 rounding first), as candle's CPU QMatMul receives
 * them; DTTS_Q8_W8A32 is the unquantized f32 product. DTTS_Q8_W8A16 is refused here (it names an
 * f16 operand). */
int dtts_gemm_q8_0_f32(const float *x, const void *blocks, float *y, int64_t m, int64_t k, int64_t n,
                       int32_t mode, hipStream_t stream);
int dtts_gemm_q8_0_ws_f32(const float *x, const void *blocks, float *y, int64_t m, int64_t k, int64_t n,
                          int32_t mode, void *workspace, size_t workspace_bytes, hipStream_t stream);
int dtts_gemm_q8_0_packed_f32(const float *x, const void *packed, float *y, int64_t m, int64_t k, int64_t n,
                              int32_t mode, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------ codec decoder stack */

/* The qwen3tts codec's waveform stack on f16 channels-last activations, all lanes at once:
 * Codec::forward's tail (crates/qwen3tts/src/codec.rs:426-436), i.e. head_conv, the
 * DecoderBlocks (codec.rs:252-258: SnakeBeta, TransConv, ResidualUnits), then SnakeBeta,
 * the output conv and tanh. The reference runs this batch-1 in f32 (codec.rs:33-43); every
 * tensor here is f16 in HBM with f32 arithmetic inside each kernel, and each SnakeBeta runs in
 * the epilogue of the conv that produces its input (or the prologue of its consumer).
 *
 * Geometry: a causal head conv latent_dim -> channels[0] (head_kernel); n_blocks blocks, block
 * i upsampling by rates[i] (ConvTranspose1d kernel 2*rates[i]) from channels[i] to
 * channels[i+1] and then 3 residual units (SnakeBeta, causal conv ru_kernel at
 * ru_dilations[j], SnakeBeta, conv k=1, + input); a final SnakeBeta and a causal out conv
 * channels[n_blocks] -> 1 (out_kernel), tanh. */
#define DTTS_CODEC_MAX_BLOCKS 8

typedef struct dtts_codec_geometry {
    int64_t latent_dim, head_kernel, n_blocks;
    int64_t channels[DTTS_CODEC_MAX_BLOCKS + 1];
    int64_t rates[DTTS_CODEC_MAX_BLOCKS];
    int64_t ru_kernel, ru_dilations[3], out_kernel;
    int64_t out_clamp; /* 0: tanh after the output conv (the benchmark's form); 1: clamp to [-1, 1]
                          (Codec::forward, crates/qwen3tts/src/codec.rs:433-436) */
} dtts_codec_geometry;

/* Device pointers. Conv weights are f16 in the layouts dtts_tap_major_weight /
 * dtts_transpose_tap_major_weight produce (the transposed conv's bias repeated by
 * dtts_transpose_bias); SnakeBeta parameters are f32 alpha = exp(alpha_log) and
 * brecip = 1/(exp(beta_log) + 1e-9), as SnakeBeta::load folds them (codec.rs:60-68). */
typedef struct dtts_codec_unit {
    const float *act1_alpha, *act1_brecip;
    const void *conv1_w, *conv1_b;
    const float *act2_alpha, *act2_brecip;
    const void *conv2_w, *conv2_b;
} dtts_codec_unit;

typedef struct dtts_codec_block {
    const float *act_alpha, *act_brecip;
    const void *up_w, *up_b;
    dtts_codec_unit units[3];
} dtts_codec_block;

typedef struct dtts_codec_weights {
    const void *head_w, *head_b;
    dtts_codec_block blocks[DTTS_CODEC_MAX_BLOCKS];
    const float *out_alpha, *out_brecip;
    const void *out_w, *out_b;
} dtts_codec_weights;

typedef struct dtts_codec dtts_codec;

/* Validates the geometry, keeps the weight pointers (the caller keeps the memory alive) and
 * builds the small per-phase parameter tables the fused transposed convs need (device memory,
 * freed by dtts_codec_destroy). Uses the current HIP device. */
int dtts_codec_create(const dtts_codec_geometry *geo, const dtts_codec_weights *weights,
                      dtts_codec **out);
/* The same stack at the reference's own precision: every conv weight and bias is f32 in the same
 * layouts, and the codec decodes f32 activations with dtts_codec_decode_f32 only. The reference
 * keeps its waveform stack f32 because f16 storage "missed the fixtures by 6x"
 * (crates/qwen3tts/src/codec.rs:33-43, WAV_DTYPE = F32). Every conv runs at f32 accuracy on the
 * f16 matrix cores (the split route of dtts_conv1d_nlc_f32_split: activations stored as f16 hi/lo
 * pairs, weights split once here), every residual unit is its two convs, and the output conv
 * reads the split activations directly. Create synchronises the null stream once per conv weight
 * (its largest magnitude picks the split's scale). */
int dtts_codec_create_f32(const dtts_codec_geometry *geo, const dtts_codec_weights *weights,
                          dtts_codec **out);
void dtts_codec_destroy(dtts_codec *codec);

/* Audio samples per latent frame (the product of the rates). */
int64_t dtts_codec_hop(const dtts_codec *codec);

/* Scratch bytes dtts_codec_decode (or _f32) needs for `lanes` x `frames` (four ping-pong
 * activation buffers at the widest stage, in the codec's element type). */
size_t dtts_codec_workspace_bytes(const dtts_codec *codec, int64_t lanes, int64_t frames);

/* latent [lanes, frames, latent_dim] f16 -> audio [lanes, frames * hop] f16 in [-1, 1].
 * Enqueues ~35 kernels per half of the lanes: the first half on `stream`, the second on a stream
 * the codec owns, forked from and joined back into `stream` with events, so the call is ordered
 * on `stream` like any other work (the two halves overlap each other's ramps and tails). The
 * workspace must hold dtts_codec_workspace_bytes bytes. Calls on one codec share its side stream
 * and events under a lock the codec holds from the fork to the join, so several host threads may
 * decode through one codec (each with its own workspace); their second halves then run one after
 * another on the side stream. */
int dtts_codec_decode(const dtts_codec *codec, const dtts_f16 *latent, dtts_f16 *audio,
                      int64_t lanes, int64_t frames, void *workspace, size_t workspace_bytes,
                      hipStream_t stream);
/* latent [lanes, frames, latent_dim] f32 -> audio [lanes, frames * hop] f32, for a codec made by
 * dtts_codec_create_f32 (the other kind is refused, and vice versa). */
int dtts_codec_decode_f32(const dtts_codec *codec, const float *latent, float *audio,
                          int64_t lanes, int64_t frames, void *workspace, size_t workspace_bytes,
                          hipStream_t stream);

/* One launch of the decode, as dtts_codec_profile reports it. flops and bytes are algorithmic
 * (2*MACs; each input, output and weight moved once); ms is the launch's own duration between
 * HIP events recorded on the stream around it. */
typedef struct dtts_codec_stage {
    char name[32];    /* e.g. "block2.unit1.conv1" */
    char kernel[96];  /* the HIP kernel that ran, as a profiler names it */
    int64_t lanes, len, cin, cout, k, dilation;
    double flops, bytes;
    float ms;
} dtts_codec_stage;

/* dtts_codec_decode (or _f32, by the codec's kind; latent and audio in its element type) with a
 * HIP event around every launch; synchronises the stream and fills stages[0 .. *n_stages). The
 * per-stage timing Codec::profile does (crates/qwen3tts/src/codec.rs:465-542), at kernel
 * granularity. */
int dtts_codec_profile(const dtts_codec *codec, const void *latent, void *audio,
                       int64_t lanes, int64_t frames, void *workspace, size_t workspace_bytes,
                       hipStream_t stream, dtts_codec_stage *stages, int max_stages,
                       int *n_stages);

/* Codec::decode (crates/qwen3tts/src/codec.rs:562-604) for one document of n code frames: windows
 * of chunk + context frames starting every `chunk` frames (the first without context), each padded
 * on the right to the full span by repeating its last frame when n >= span; every window through
 * the front half and the waveform stack, then the audio of each window's own chunk, without its
 * context, concatenated. The windows are independent forwards, so all of them run at once as
 * lanes of one length (for n < span: n, the later windows padded like the rest, which leaves the
 * kept audio of a causal decoder unchanged). codes [n, n_books] int32 on the HOST;
 * audio [n * samples_per_frame] f32 on the device, samples_per_frame = prod(up_ratios) *
 * dtts_codec_hop(codec). A codec made by dtts_codec_create_f32 runs the waveform stack at f32 (the
 * reference's WAV_DTYPE) on the front half's latent widened exactly from f16. */
size_t dtts_codec_document_workspace_bytes(const dtts_codec_front *front, const dtts_codec *codec, int64_t n,
                                           int64_t chunk, int64_t context);
int dtts_codec_decode_document(const dtts_codec_front *front, const dtts_codec *codec, const int32_t *codes,
                               int64_t n, int64_t chunk, int64_t context, float *audio, void *workspace,
                               size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------ f-4 checkpoints and weight formats
 *
 * What a loader must produce for the kernels (crates/tts-nn/src/lib.rs:143-360 Weights,
 * 1252-1298 host_layout; crates/tts-nn/src/nlc.rs:30-183 the conv layouts). A safetensors file
 * is memory-mapped and indexed by its header; tensors are read from the mapping in their
 * on-disk dtype. The rearrangements run on the GPU from the raw tensor uploaded once: casts to
 * f16/f32, the tap-major and polyphase conv layouts, the [out, in] -> [in, out] transpose,
 * SnakeBeta's and the codebooks' folds and Q8_0 quantisation. */
#define DTTS_DT_F32 0
#define DTTS_DT_F16 1
#define DTTS_DT_BF16 2
#define DTTS_DT_F64 3
#define DTTS_DT_I64 4
#define DTTS_DT_I32 5
#define DTTS_DT_I16 6
#define DTTS_DT_I8 7
#define DTTS_DT_U8 8
#define DTTS_DT_BOOL 9
#define DTTS_DT_OTHER 10 /* any other safetensors dtype (U16/U32/U64/F8_*): listed, not converted */
#define DTTS_TENSOR_MAX_DIMS 8

typedef struct dtts_checkpoint dtts_checkpoint;

typedef struct dtts_tensor_info {
    const char *name;   /* owned by the checkpoint */
    int32_t dtype;      /* DTTS_DT_* */
    int32_t ndim;
    int64_t shape[DTTS_TENSOR_MAX_DIMS];
    const void *data;   /* host pointer into the mapping */
    size_t bytes;
} dtts_tensor_info;

/* Weights::load (lib.rs:161-173): maps the file and parses its header; the header's offsets and
 * sizes are checked against the file and the dtypes' widths. */
int dtts_checkpoint_open(const char *path, dtts_checkpoint **out);
void dtts_checkpoint_close(dtts_checkpoint *ck);
/* Weights::len (lib.rs:339-341); tensors in the header's order. */
int64_t dtts_checkpoint_count(const dtts_checkpoint *ck);
int dtts_checkpoint_at(const dtts_checkpoint *ck, int64_t index, dtts_tensor_info *out);
/* Weights::cpu / file_shape (lib.rs:257-264, 349-351): "missing tensor <name>" when absent. */
int dtts_checkpoint_get(const dtts_checkpoint *ck, const char *name, dtts_tensor_info *out);

/* Device conversions: src is a raw tensor of dtype F32, F16, BF16 or F64 on the device; f16
 * results are rounded to nearest even once from the exact value. */
/* to_dtype (f16 / f32), n elements. */
int dtts_convert_f16(const void *src, int32_t dtype, dtts_f16 *dst, int64_t n, hipStream_t stream);
int dtts_convert_f32(const void *src, int32_t dtype, float *dst, int64_t n, hipStream_t stream);
/* f32 times a scale, one rounding: Layer::load's q_norm * 1/sqrt(head_dim) (qwen3.rs:78-84). */
int dtts_convert_f32_scaled(const void *src, int32_t dtype, float *dst, int64_t n, float scale, hipStream_t stream);
/* A [rows, cols] source into columns [col0, col0 + cols) of a [rows, ld] f16 destination: how
 * tensors are concatenated along the last dimension (the codec's two RVQ output projections). */
int dtts_convert_f16_cols(const void *src, int32_t dtype, dtts_f16 *dst, int64_t rows, int64_t cols, int64_t ld,
                          int64_t col0, hipStream_t stream);
/* host_layout (lib.rs:1252-1269): [rows, cols] -> [cols, rows] f16. */
int dtts_convert_transpose_f16(const void *src, int32_t dtype, dtts_f16 *dst, int64_t rows, int64_t cols,
                               hipStream_t stream);
/* dtts_tap_major_weight's layout: torch Conv1d [cout, cin, k] -> [cout, k*cin] f16. */
int dtts_convert_tap_major_f16(const void *w_oik, int32_t dtype, dtts_f16 *dst, int64_t cout, int64_t cin,
                               int64_t k, hipStream_t stream);
/* dtts_transpose_tap_major_weight's layout: ConvTranspose1d [cin, cout, kernel] ->
 * [stride*cout, (kernel/stride)*cin] f16, taps reversed per phase. */
int dtts_convert_transpose_tap_major_f16(const void *w_iok, int32_t dtype, dtts_f16 *dst, int64_t cin, int64_t cout,
                                         int64_t kernel, int64_t stride, hipStream_t stream);
/* nlc::transpose_bias (nlc.rs:177-183): [n] repeated `times` times, f16. */
int dtts_convert_repeat_f16(const void *src, int32_t dtype, dtts_f16 *dst, int64_t n, int64_t times,
                            hipStream_t stream);
/* SnakeBeta::load (crates/qwen3tts/src/codec.rs:60-68): alpha = exp(alpha_log),
 * brecip = 1 / (exp(beta_log) + 1e-9), in f32 (exp correctly rounded to f32). */
int dtts_convert_snake_fold(const void *alpha_log, const void *beta_log, int32_t dtype, float *alpha, float *brecip,
                            int64_t n, hipStream_t stream);
/* Rvq::load (codec.rs:275-282): embedding_sum [size, dim] / clamp(cluster_usage [size], eps). */
int dtts_convert_codebook_fold(const void *embedding_sum, const void *cluster_usage, int32_t dtype, float eps,
                               float *dst, int64_t size, int64_t dim, hipStream_t stream);
/* QTensor::quantize_onto for an [rows, k] weight into GGML block_q8_0 (the same rule as the host
 * dtts_q8_0_quantize, bit for bit): blocks holds rows*k/32*34 bytes, 2-byte aligned. */
int dtts_convert_q8_0(const void *w, int32_t dtype, void *blocks, int64_t rows, int64_t k, hipStream_t stream);

/* Codec::load (crates/qwen3tts/src/codec.rs:347-399) from a checkpoint in the reference's naming
 * ("decoder.quantizer.rvq_first.*", "decoder.pre_transformer.layers.<i>.*",
 * "decoder.upsample.<i>.*", "decoder.decoder.<i>.*"): every tensor's presence and shape is
 * checked against the two geometries before anything is allocated; then one device arena is
 * allocated and filled by the conversions above (the raw tensors pass through a device staging
 * buffer freed before return), and the front half and waveform stack are created on it. The
 * call synchronises `stream`. */
typedef struct dtts_codec_model dtts_codec_model;
int dtts_codec_model_load(const dtts_checkpoint *ck, const dtts_codec_front_geometry *front,
                          const dtts_codec_geometry *wave, hipStream_t stream, dtts_codec_model **out);
void dtts_codec_model_destroy(dtts_codec_model *model);
const dtts_codec_front *dtts_codec_model_front(const dtts_codec_model *model);
const dtts_codec *dtts_codec_model_wave(const dtts_codec_model *model);
size_t dtts_codec_model_bytes(const dtts_codec_model *model); /* the arena's size */

/* Stack::load (crates/qwen3tts/src/qwen3.rs:61-119, 226-250) from a checkpoint: "<prefix>layers.<i>."
 * input_layernorm / post_attention_layernorm, self_attn.{q,k,v,o}_proj, mlp.{gate,up,down}_proj,
 * with QK-norm self_attn.{q,k}_norm (q's folded with 1/sqrt(head_dim)), with LayerScale
 * self_attn_layer_scale.scale / mlp_layer_scale.scale, and "<prefix>norm.weight"; prefix e.g.
 * "talker.model." (talker.rs:597) or "talker.code_predictor.model." (talker.rs:292). Checked,
 * then converted into one arena (projections f16 [out, in], q|k|v and gate|up rows joined) on
 * which the stack is created. The call synchronises `stream`. */
typedef struct dtts_stack_model dtts_stack_model;
int dtts_stack_model_load(const dtts_checkpoint *ck, const char *prefix, const dtts_stack_geometry *geo,
                          hipStream_t stream, dtts_stack_model **out);
/* Stack::load with its `how` (DTTS_WEIGHT_*; dtts_stack_model_load is DTTS_WEIGHT_F16): projections
 * converted to f32, or quantized on the device to Q8_0 as QTensor::quantize_onto does
 * (crates/tts-nn/src/lib.rs:480-486; bit for bit the host quantizer) and repacked; the stack is
 * created with that kind (f32 caches for all but F16). */
int dtts_stack_model_load_as(const dtts_checkpoint *ck, const char *prefix, const dtts_stack_geometry *geo,
                             int32_t how, hipStream_t stream, dtts_stack_model **out);
void dtts_stack_model_destroy(dtts_stack_model *model);
dtts_stack *dtts_stack_model_stack(const dtts_stack_model *model);
size_t dtts_stack_model_bytes(const dtts_stack_model *model);

#ifdef __cplusplus
}
#endif
#endif /* DTTS_H */
