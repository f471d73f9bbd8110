// The codec's front half, kernels of their own (the projections and convs between them run on
// the channels-last conv kernel):
//
//   RVQ lookup-sum  Rvq::decode (crates/qwen3tts/src/codec.rs:296-313): per frame, the rows the
//                   codes pick from each codebook, summed in codebook order, for the semantic
//                   stack (the first n_first books) and the acoustic stack (the rest) side by side.
//                   The two output projections then run as one GEMM over the concatenated width,
//                   which is the reference's q_sem + q_ac (codec.rs:403-408).
//   depthwise+LN    ConvNext::forward's first two ops (codec.rs:186-188): the causal depthwise
//                   conv (nlc::depthwise, crates/tts-nn/src/nlc.rs:236-256: taps accumulated
//                   oldest first, then the bias) and LayerNorm over the channels (two passes:
//                   mean, then the variance of the centred values; lib.rs:1006-1035), one wave
//                   per position.
//
//   RMSNorm rows   rms_norm over channels-last rows for the windowed transformer: f16 in, f32
//                   arithmetic, one rounding out (the reference runs it in f32).
//   SwiGLU rows    silu(gate) * up from a [rows, 2 * ffn] gate|up projection, f16 out.
//   window attn    Stack::forward's prefill branch (crates/qwen3tts/src/qwen3.rs:420-443) for a
//                   sliding window: RoPE on q and k as they are loaded (the roped values are the
//                   MFMA's f16 operands), scores = q.k * scale, the causal window mask of
//                   causal_window_mask (lib.rs:1210-1224: key j is visible to query i when
//                   i - window < j <= i), softmax, weighted v.
//
// The lookup, depthwise+LN, the norm and SwiGLU are HBM-bound passes: the lookup reads n_books
// rows of `dim` f32 per frame and writes 2 * dim f16; depthwise+LN reads its k input rows (the
// earlier k-1 mostly from cache, as neighbouring positions share them) and writes one row.
#include "norm_rope.hpp"

namespace dtts {
namespace {

__device__ __forceinline__ float wave_sum64(float v) { return wave_sum(v); }

// Thread per (row, 4 output dims). codes [rows, n_books] int32 (clamped into the codebook; the
// entry point checks them on the host when it is given host codes); books [n_books, size, dim]
// f32; out [rows, 2 * dim] f16 = [semantic sum | acoustic sum].
__global__ __launch_bounds__(256) void rvq_gather_kernel(const int32_t *codes, const float *books, half_t *out,
                                                         int64_t rows, int n_books, int n_first, int size, int dim) {
    const int q4 = dim / 4;
    const int64_t total = rows * 2 * q4;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t row = e / (2 * q4);
        const int w = static_cast<int>(e - row * 2 * q4);
        const int half_sel = w / q4;  // 0 semantic, 1 acoustic
        const int d = (w - half_sel * q4) * 4;
        const int b0 = half_sel ? n_first : 0, b1 = half_sel ? n_books : n_first;
        const int32_t *cr = codes + row * n_books;
        float4_t s = float4_t{0.f, 0.f, 0.f, 0.f};
        for (int b = b0; b < b1; ++b) {
            int c = cr[b];
            c = c < 0 ? 0 : (c >= size ? size - 1 : c);
            const float4_t v = *reinterpret_cast<const float4_t *>(books + (static_cast<int64_t>(b) * size + c) * dim + d);
            s = b == b0 ? v : s + v;
        }
        half4_t h;
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = static_cast<half_t>(s[j]);
        *reinterpret_cast<half4_t *>(out + row * 2 * dim + half_sel * dim + d) = h;
    }
}

// One wave per position; lane j holds channel groups g = j, j + 64, ... of 8 channels (NG of
// them). x, y [lanes, len, C] f16; taps [C, K] f32 (tap 0 multiplies position l - (K - 1));
// bias, ln_w, ln_b [C] f32.
template <int NG>
__global__ __launch_bounds__(256) void depthwise_ln_kernel(const half_t *x, const float *taps, const float *bias,
                                                           const float *ln_w, const float *ln_b, half_t *y,
                                                           int64_t rows, int len, int C, int K, float eps) {
#pragma clang fp contract(off)
    const int64_t row = blockIdx.x * int64_t(4) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int l = static_cast<int>(row % len);
    const int groups = C / 8;
    float h[NG][8];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int g = lane + 64 * i;
        if (g >= groups) continue;
        float acc[8];
        for (int t = 0; t < K; ++t) {
            const int src = l - (K - 1) + t;
            half8_t v = half8_t{};
            if (src >= 0) v = *reinterpret_cast<const half8_t *>(x + (row - l + src) * C + g * 8);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float term = static_cast<float>(v[q]) * taps[(g * 8 + q) * K + t];
                acc[q] = t == 0 ? term : acc[q] + term;
            }
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            h[i][q] = acc[q] + bias[g * 8 + q];
            s += h[i][q];
        }
    }
    const float mean = wave_sum64(s) / static_cast<float>(C);
    float v2 = 0.0f;
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int g = lane + 64 * i;
        if (g >= groups) continue;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            h[i][q] = h[i][q] - mean;
            v2 += h[i][q] * h[i][q];
        }
    }
    const float den = sqrtf(wave_sum64(v2) / static_cast<float>(C) + eps);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int g = lane + 64 * i;
        if (g >= groups) continue;
        half8_t o;
#pragma unroll
        for (int q = 0; q < 8; ++q) o[q] = static_cast<half_t>((h[i][q] / den) * ln_w[g * 8 + q] + ln_b[g * 8 + q]);
        *reinterpret_cast<half8_t *>(y + row * C + g * 8) = o;
    }
}

// The same op with the taps fixed at compile time, a workgroup per strip of P positions of one
// lane: thread g owns channels [8g, 8g + 8) for the whole strip (taps, bias and LayerNorm
// parameters loaded once into registers), loads the strip's P + K - 1 input rows once (16 bytes
// per thread per row, a row coalesced across the workgroup), computes the P depthwise outputs in
// registers and reduces the P row sums, then the P centred sums of squares, across the workgroup
// in two LDS rounds (one barrier each). Threads = C/8 rounded up to a wave (C <= 2048).
template <int K, int P>
__global__ __launch_bounds__(256) void depthwise_ln_strip_kernel(const half_t *x, const float *taps, const float *bias,
                                                                 const float *ln_w, const float *ln_b, half_t *y,
                                                                 int len, int C, float eps) {
#pragma clang fp contract(off)
    __shared__ float red[4][P];
    const int g = threadIdx.x, wave = threadIdx.x >> 6;
    const int nw = (blockDim.x + 63) >> 6;
    const bool on = g < C / 8;
    const int l0 = blockIdx.x * P;
    const half_t *xl = x + static_cast<int64_t>(blockIdx.y) * len * C + g * 8;
    half_t *yl = y + static_cast<int64_t>(blockIdx.y) * len * C + g * 8;
    float h[P][8];
    if (on) {
        float w[K][8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
            for (int t = 0; t < K; ++t) w[t][q] = taps[(g * 8 + q) * K + t];
        half8_t win[P + K - 1];
#pragma unroll
        for (int r = 0; r < P + K - 1; ++r) {
            const int src = l0 - (K - 1) + r;
            win[r] = (src >= 0 && src < len) ? *reinterpret_cast<const half8_t *>(xl + static_cast<int64_t>(src) * C)
                                             : half8_t{};
        }
        const float4_t b0 = *reinterpret_cast<const float4_t *>(bias + g * 8);
        const float4_t b1 = *reinterpret_cast<const float4_t *>(bias + g * 8 + 4);
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                float acc = static_cast<float>(win[p][q]) * w[0][q];
#pragma unroll
                for (int t = 1; t < K; ++t) acc = acc + static_cast<float>(win[p + t][q]) * w[t][q];
                h[p][q] = acc + (q < 4 ? b0[q] : b1[q - 4]);
            }
    } else {
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
            for (int q = 0; q < 8; ++q) h[p][q] = 0.0f;
    }
    // mean per position
    float mean[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q) s += h[p][q];
        s = wave_sum64(s);
        if ((threadIdx.x & 63) == 0) red[wave][p] = s;
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < P; ++p) {
        float s = red[0][p];
        for (int i = 1; i < nw; ++i) s += red[i][p];
        mean[p] = s / static_cast<float>(C);
    }
    __syncthreads();  // red is reused
#pragma unroll
    for (int p = 0; p < P; ++p) {
        float v2 = 0.0f;
        if (on) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                h[p][q] = h[p][q] - mean[p];
                v2 += h[p][q] * h[p][q];
            }
        }
        v2 = wave_sum64(v2);
        if ((threadIdx.x & 63) == 0) red[wave][p] = v2;
    }
    __syncthreads();
    if (!on) return;
    const float4_t w0 = *reinterpret_cast<const float4_t *>(ln_w + g * 8);
    const float4_t w1 = *reinterpret_cast<const float4_t *>(ln_w + g * 8 + 4);
    const float4_t c0 = *reinterpret_cast<const float4_t *>(ln_b + g * 8);
    const float4_t c1 = *reinterpret_cast<const float4_t *>(ln_b + g * 8 + 4);
#pragma unroll
    for (int p = 0; p < P; ++p) {
        if (l0 + p >= len) break;
        float v2 = red[0][p];
        for (int i = 1; i < nw; ++i) v2 += red[i][p];
        const float den = sqrtf(v2 / static_cast<float>(C) + eps);
        half8_t o;
#pragma unroll
        for (int q = 0; q < 8; ++q)
            o[q] = static_cast<half_t>((h[p][q] / den) * (q < 4 ? w0[q] : w1[q - 4]) + (q < 4 ? c0[q] : c1[q - 4]));
        *reinterpret_cast<half8_t *>(yl + static_cast<int64_t>(l0 + p) * C) = o;
    }
}

// One wave per row: x f16 [rows, C] -> y f16, y = (x / sqrt(mean(x^2) + eps)) * gamma in f32.
__global__ __launch_bounds__(256) void rms_rows_kernel(const half_t *x, const float *gamma, half_t *y, int64_t rows,
                                                       int C, float eps) {
#pragma clang fp contract(off)
    const int64_t row = blockIdx.x * int64_t(4) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const half_t *xr = x + row * C;
    float ss = 0.0f;
    for (int c = lane * 8; c < C; c += 512) {
        const half8_t v = *reinterpret_cast<const half8_t *>(xr + c);
#pragma unroll
        for (int q = 0; q < 8; ++q) ss += static_cast<float>(v[q]) * static_cast<float>(v[q]);
    }
    const float m = sqrtf(wave_sum(ss) / static_cast<float>(C) + eps);
    for (int c = lane * 8; c < C; c += 512) {
        const half8_t v = *reinterpret_cast<const half8_t *>(xr + c);
        half8_t o;
#pragma unroll
        for (int q = 0; q < 8; ++q) o[q] = static_cast<half_t>((static_cast<float>(v[q]) / m) * gamma[c + q]);
        *reinterpret_cast<half8_t *>(y + row * C + c) = o;
    }
}

// gu [rows, 2 * ffn] f16 (gate columns, then up columns) -> t [rows, ffn] f16 = silu(g) * u.
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const half_t *gu, half_t *t, int64_t rows, int ffn) {
    const int q8 = ffn / 8;
    const int64_t total = rows * q8;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t row = e / q8;
        const int c = static_cast<int>(e - row * q8) * 8;
        const half8_t g = *reinterpret_cast<const half8_t *>(gu + row * 2 * ffn + c);
        const half8_t u = *reinterpret_cast<const half8_t *>(gu + row * 2 * ffn + ffn + c);
        half8_t o;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float gv = static_cast<float>(g[q]);
            o[q] = static_cast<half_t>((gv / (1.0f + expf(-gv))) * static_cast<float>(u[q]));
        }
        *reinterpret_cast<half8_t *>(t + row * ffn + c) = o;
    }
}

// Windowed causal attention over a sequence, D = 64, on v_mfma_f32_16x16x32_f16. Workgroup =
// (64-query block, query head, lane), one wave per 16 queries. The block's keys, from the first
// query - window + 1 on, 16 (NT + 3) rows, are staged in LDS once: k roped in f32 and stored in
// f16 (row-major, the scores' A operand), v transposed to [dim][key] (the weighted sum's A
// operand); keys before 0 or past the sequence are zero rows. A wave's queries see NT 16-key
// tiles starting at its first query - window + 1 (16 NT >= window + 15).
//   scores^T = K . Q^T      two MFMAs per tile; a lane ends with one query (lane % 16) and four
//                           keys per tile, so a query's max and sum are a lane's own values
//                           plus two shuffles (xor 16, 32). Scaled after the dot product, as the
//                           prefill branch scales the scores; keys outside (q - window, q]
//                           masked to -inf.
//   p = exp(s - max)        rounded to f16 (the MFMA operand); sum over the rounded p in f32.
//   out^T = V^T . P^T       two tiles of p per MFMA: a lane's own p values are the B operand as
//                           they stand, with V^T's k slots permuted to the same keys (exact: the
//                           sum over keys is order-free). out = acc / sum, one f16 rounding.
constexpr int kWinMax = 192;
constexpr int kQBlock = 64;

template <int NT>
__global__ __launch_bounds__(256) void window_attn_kernel(const half_t *qkv, const float *cos_t, const float *sin_t,
                                                          half_t *out, int T, int heads, int n_kv, int window,
                                                          float scale) {
#pragma clang fp contract(off)
    constexpr int D = 64, HALF = 32, ROWS = 16 * (NT + 3);
    constexpr int KP = D + 8;     // K row pitch, halves (144 bytes: 16-byte aligned rows)
    constexpr int VP = ROWS + 8;  // V^T row pitch, halves
    __shared__ __attribute__((aligned(16))) half_t Ks[ROWS * KP];
    __shared__ __attribute__((aligned(16))) half_t Vt[D * VP];
    const int l0 = blockIdx.x * kQBlock;
    const int h = blockIdx.y;
    const int lane_idx = blockIdx.z;
    const int kh = h / (heads / n_kv);
    const int width = (heads + 2 * n_kv) * D;
    const half_t *base = qkv + static_cast<int64_t>(lane_idx) * T * width;
    const int j0 = l0 - window + 1;  // key of staged row 0
    // stage: 4 threads per row; thread g takes dims [8g, 8g + 8) and their RoPE partners + 32
    for (int e = threadIdx.x; e < ROWS * 4; e += 256) {
        const int r = e >> 2, g = e & 3;
        const int j = j0 + r;
        half8_t k1 = {}, k2 = {}, v1 = {}, v2 = {};
        if (j >= 0 && j < T) {
            const half_t *kr = base + static_cast<int64_t>(j) * width + (heads + kh) * D + 8 * g;
            const half8_t a = *reinterpret_cast<const half8_t *>(kr);
            const half8_t b = *reinterpret_cast<const half8_t *>(kr + HALF);
            const float *cr = cos_t + static_cast<int64_t>(j) * HALF + 8 * g;
            const float *sr = sin_t + static_cast<int64_t>(j) * HALF + 8 * g;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                float o1, o2;
                rope_pair(static_cast<float>(a[u]), static_cast<float>(b[u]), cr[u], sr[u], o1, o2);
                k1[u] = static_cast<half_t>(o1);
                k2[u] = static_cast<half_t>(o2);
            }
            const half_t *vr = base + static_cast<int64_t>(j) * width + (heads + n_kv + kh) * D + 8 * g;
            v1 = *reinterpret_cast<const half8_t *>(vr);
            v2 = *reinterpret_cast<const half8_t *>(vr + HALF);
        }
        *reinterpret_cast<half8_t *>(Ks + r * KP + 8 * g) = k1;
        *reinterpret_cast<half8_t *>(Ks + r * KP + HALF + 8 * g) = k2;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            Vt[(8 * g + u) * VP + r] = v1[u];
            Vt[(HALF + 8 * g + u) * VP + r] = v2[u];
        }
    }
    // this lane's query (lane % 16 of the wave's 16) and its k slots [8g, 8g + 8) of each half
    const int w = threadIdx.x >> 6, ln = threadIdx.x & 63;
    const int col = ln & 15, g = ln >> 4;
    const int q = l0 + 16 * w + col;
    half8_t qa = {}, qb = {};
    if (q < T) {
        const half_t *qr = base + static_cast<int64_t>(q) * width + h * D + 8 * g;
        const half8_t a = *reinterpret_cast<const half8_t *>(qr);
        const half8_t b = *reinterpret_cast<const half8_t *>(qr + HALF);
        const float *cr = cos_t + static_cast<int64_t>(q) * HALF + 8 * g;
        const float *sr = sin_t + static_cast<int64_t>(q) * HALF + 8 * g;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            float o1, o2;
            rope_pair(static_cast<float>(a[u]), static_cast<float>(b[u]), cr[u], sr[u], o1, o2);
            qa[u] = static_cast<half_t>(o1);
            qb[u] = static_cast<half_t>(o2);
        }
    }
    __syncthreads();
    if (l0 + 16 * w >= T) return;  // the whole wave is past the sequence (no barrier follows)
    // scores^T per tile: rows = keys 16 (w + t) + 4g + r of the staging, column = this query
    float s[NT][4];
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const half_t *kr = Ks + (16 * (w + t) + col) * KP + 8 * g;
        const half8_t ka = *reinterpret_cast<const half8_t *>(kr);
        const half8_t kb = *reinterpret_cast<const half8_t *>(kr + HALF);
        float4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qa, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb, qb, c, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int j = j0 + 16 * (w + t) + 4 * g + r;
            const bool seen = j >= 0 && j <= q && j > q - window;
            s[t][r] = seen ? c[r] * scale : -INFINITY;
            mx = fmaxf(mx, s[t][r]);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (mx == -INFINITY) mx = 0.0f;  // a query past the sequence (not stored)
    half_t p[NT][4];
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p[t][r] = static_cast<half_t>(__builtin_expf(s[t][r] - mx));
            sum += static_cast<float>(p[t][r]);
        }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    float4_t o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < NT / 2; ++c) {
        const half8_t pb = {p[2 * c][0], p[2 * c][1], p[2 * c][2], p[2 * c][3],
                            p[2 * c + 1][0], p[2 * c + 1][1], p[2 * c + 1][2], p[2 * c + 1][3]};
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const half_t *vr = Vt + (16 * dt + col) * VP + 16 * (w + 2 * c) + 4 * g;
            const half4_t a0 = *reinterpret_cast<const half4_t *>(vr);
            const half4_t a1 = *reinterpret_cast<const half4_t *>(vr + 16);
            const half8_t va = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, o[dt], 0, 0, 0);
        }
    }
    if (q >= T) return;
    // out^T tile dt: this lane holds dims 16 dt + 4g + r of its query
    half_t *dst = out + (static_cast<int64_t>(lane_idx) * T + q) * heads * D + h * D + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
        half4_t v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = static_cast<half_t>(o[dt][r] / sum);
        *reinterpret_cast<half4_t *>(dst + 16 * dt) = v;
    }
}

}  // namespace
}  // namespace dtts

using dtts::half_t;

extern "C" int dtts_rvq_lookup_sum_f16(const int32_t *codes, const float *codebooks, int64_t n_books,
                                       int64_t n_first, int64_t book_size, int64_t dim, dtts_f16 *out, int64_t rows,
                                       hipStream_t stream) {
    const char *name = "dtts_rvq_lookup_sum_f16";
    DTTS_REQUIRE(rows >= 0 && n_books > 0 && n_first > 0 && n_first < n_books && book_size > 0 && dim > 0 &&
                     dim % 4 == 0,
                 "%s: bad shape (rows %lld, books %lld, first %lld, size %lld, dim %lld)", name, (long long)rows,
                 (long long)n_books, (long long)n_first, (long long)book_size, (long long)dim);
    if (rows == 0) return DTTS_OK;
    DTTS_REQUIRE(codes && codebooks && out, "%s: null pointer", name);
    DTTS_REQUIRE(dtts::aligned(codebooks, 16) && dtts::aligned(out, 8), "%s: misaligned operand", name);
    DTTS_REQUIRE(n_books * book_size * dim < (int64_t(1) << 40) && n_books < (1 << 20) && book_size < (1 << 30) &&
                     dim < (1 << 20),
                 "%s: shape too large", name);
    const int64_t total = rows * 2 * (dim / 4);
    dtts::rvq_gather_kernel<<<dtts::grid_for(total, 256), 256, 0, stream>>>(
        codes, codebooks, reinterpret_cast<half_t *>(out), rows, static_cast<int>(n_books), static_cast<int>(n_first),
        static_cast<int>(book_size), static_cast<int>(dim));
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_depthwise_layernorm_nlc_f16(const dtts_f16 *x, const float *taps, const float *bias,
                                                const float *ln_weight, const float *ln_bias, float eps, dtts_f16 *y,
                                                int64_t lanes, int64_t len, int64_t channels, int64_t k,
                                                hipStream_t stream) {
    const char *name = "dtts_depthwise_layernorm_nlc_f16";
    DTTS_REQUIRE(lanes >= 0 && len >= 0 && channels > 0 && channels % 8 == 0 && channels <= 2048 && k > 0 && k <= 64,
                 "%s: bad shape (lanes %lld, len %lld, channels %lld, k %lld): channels a multiple of 8 up to 2048",
                 name, (long long)lanes, (long long)len, (long long)channels, (long long)k);
    if (lanes == 0 || len == 0) return DTTS_OK;
    DTTS_REQUIRE(x && taps && bias && ln_weight && ln_bias && y, "%s: null pointer", name);
    DTTS_REQUIRE(x != y, "%s: in place is not supported (rows read their predecessors)", name);
    DTTS_REQUIRE(dtts::aligned(x, 16) && dtts::aligned(y, 16), "%s: x and y must be 16-byte aligned", name);
    DTTS_REQUIRE(lanes * len < (int64_t(1) << 40) && len < (int64_t(1) << 30), "%s: shape too large", name);
    const int64_t rows = lanes * len;
    const unsigned grid = static_cast<unsigned>((rows + 3) / 4);
    const int ng = static_cast<int>((channels / 8 + 63) / 64);
    const half_t *xh = reinterpret_cast<const half_t *>(x);
    half_t *yh = reinterpret_cast<half_t *>(y);
    const int L = static_cast<int>(len), C = static_cast<int>(channels), K = static_cast<int>(k);
    if (K == 7 && lanes < 65536 && dtts::aligned(taps, 16) && dtts::aligned(bias, 16) && dtts::aligned(ln_weight, 16) &&
        dtts::aligned(ln_bias, 16)) {
        constexpr int P = 8;
        const dim3 sgrid(static_cast<unsigned>((len + P - 1) / P), static_cast<unsigned>(lanes));
        const int threads = (C / 8 + 63) / 64 * 64;
        dtts::depthwise_ln_strip_kernel<7, P><<<sgrid, threads, 0, stream>>>(xh, taps, bias, ln_weight, ln_bias, yh, L, C,
                                                                            eps);
        DTTS_LAUNCH_CHECK(name);
        return DTTS_OK;
    }
    if (ng <= 1)
        dtts::depthwise_ln_kernel<1><<<grid, 256, 0, stream>>>(xh, taps, bias, ln_weight, ln_bias, yh, rows, L, C, K, eps);
    else if (ng <= 2)
        dtts::depthwise_ln_kernel<2><<<grid, 256, 0, stream>>>(xh, taps, bias, ln_weight, ln_bias, yh, rows, L, C, K, eps);
    else
        dtts::depthwise_ln_kernel<4><<<grid, 256, 0, stream>>>(xh, taps, bias, ln_weight, ln_bias, yh, rows, L, C, K, eps);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_rms_norm_rows_f16(const dtts_f16 *x, const float *gamma, dtts_f16 *y, int64_t rows, int64_t dim,
                                      float eps, hipStream_t stream) {
    const char *name = "dtts_rms_norm_rows_f16";
    DTTS_REQUIRE(rows >= 0 && dim > 0 && dim % 8 == 0 && dim < (1 << 24), "%s: bad shape (%lld, %lld): dim a multiple of 8",
                 name, (long long)rows, (long long)dim);
    if (rows == 0) return DTTS_OK;
    DTTS_REQUIRE(x && gamma && y, "%s: null pointer", name);
    DTTS_REQUIRE(dtts::aligned(x, 16) && dtts::aligned(y, 16), "%s: x and y must be 16-byte aligned", name);
    DTTS_REQUIRE(rows < (int64_t(1) << 40), "%s: too many rows", name);
    dtts::rms_rows_kernel<<<static_cast<unsigned>((rows + 3) / 4), 256, 0, stream>>>(
        reinterpret_cast<const half_t *>(x), gamma, reinterpret_cast<half_t *>(y), rows, static_cast<int>(dim), eps);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_swiglu_rows_f16(const dtts_f16 *gate_up, dtts_f16 *y, int64_t rows, int64_t ffn, hipStream_t stream) {
    const char *name = "dtts_swiglu_rows_f16";
    DTTS_REQUIRE(rows >= 0 && ffn > 0 && ffn % 8 == 0 && ffn < (1 << 24), "%s: bad shape (%lld, %lld)", name,
                 (long long)rows, (long long)ffn);
    if (rows == 0) return DTTS_OK;
    DTTS_REQUIRE(gate_up && y, "%s: null pointer", name);
    DTTS_REQUIRE(dtts::aligned(gate_up, 16) && dtts::aligned(y, 16), "%s: misaligned operand", name);
    dtts::swiglu_rows_kernel<<<dtts::grid_for(rows * (ffn / 8), 256), 256, 0, stream>>>(
        reinterpret_cast<const half_t *>(gate_up), reinterpret_cast<half_t *>(y), rows, static_cast<int>(ffn));
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_window_attention_prefill_f16(const dtts_f16 *qkv, const float *cos_t, const float *sin_t,
                                                 int64_t table_len, dtts_f16 *out, int64_t lanes, int64_t len,
                                                 int64_t heads, int64_t n_kv, int64_t head_dim, int64_t window,
                                                 float scale, hipStream_t stream) {
    const char *name = "dtts_window_attention_prefill_f16";
    DTTS_REQUIRE(lanes >= 0 && len >= 0 && heads > 0 && n_kv > 0 && heads % n_kv == 0,
                 "%s: bad shape (lanes %lld, len %lld, heads %lld, n_kv %lld)", name, (long long)lanes, (long long)len,
                 (long long)heads, (long long)n_kv);
    DTTS_REQUIRE(head_dim == 64, "%s: head_dim %lld (64 supported)", name, (long long)head_dim);
    DTTS_REQUIRE(window >= 1 && window <= dtts::kWinMax, "%s: window %lld (1 to %d)", name, (long long)window,
                 dtts::kWinMax);
    if (lanes == 0 || len == 0) return DTTS_OK;
    DTTS_REQUIRE(qkv && cos_t && sin_t && out, "%s: null pointer", name);
    DTTS_REQUIRE(len <= table_len, "%s: %lld positions exceed the RoPE table (%lld)", name, (long long)len,
                 (long long)table_len);
    DTTS_REQUIRE(dtts::aligned(qkv, 16) && dtts::aligned(out, 16), "%s: misaligned operand", name);
    DTTS_REQUIRE(lanes < 65536 && heads < 65536 && len < (int64_t(1) << 30) &&
                     lanes * len * (heads + 2 * n_kv) * head_dim < (int64_t(1) << 40),
                 "%s: shape too large", name);
    const dim3 grid(static_cast<unsigned>((len + dtts::kQBlock - 1) / dtts::kQBlock), static_cast<unsigned>(heads),
                    static_cast<unsigned>(lanes));
    const half_t *x = reinterpret_cast<const half_t *>(qkv);
    half_t *y = reinterpret_cast<half_t *>(out);
    const int T = static_cast<int>(len), H = static_cast<int>(heads), KV = static_cast<int>(n_kv);
    const int W = static_cast<int>(window);
    switch (2 * ((W + 15 + 31) / 32)) {  // key tiles per wave: 16 NT >= window + 15
#define WIN_CASE(NT)                                                                                   \
    case NT:                                                                                           \
        dtts::window_attn_kernel<NT><<<grid, 256, 0, stream>>>(x, cos_t, sin_t, y, T, H, KV, W, scale); \
        break;
        WIN_CASE(2)
        WIN_CASE(4)
        WIN_CASE(6)
        WIN_CASE(8)
        WIN_CASE(10)
        WIN_CASE(12)
        WIN_CASE(14)
#undef WIN_CASE
        default:
            DTTS_REQUIRE(false, "%s: window %d has no tile count", name, W);
    }
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}
