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
// Both are HBM-bound gathers: the lookup reads n_books rows of `dim` f32 per frame and writes
// 2 * dim f16; depthwise+LN reads its k input rows (the earlier k-1 mostly from cache, as
// neighbouring positions share them) and writes one row.
#include "common.hpp"

namespace dtts {
namespace {

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

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
    if (ng <= 1)
        dtts::depthwise_ln_kernel<1><<<grid, 256, 0, stream>>>(xh, taps, bias, ln_weight, ln_bias, yh, rows, L, C, K, eps);
    else if (ng <= 2)
        dtts::depthwise_ln_kernel<2><<<grid, 256, 0, stream>>>(xh, taps, bias, ln_weight, ln_bias, yh, rows, L, C, K, eps);
    else
        dtts::depthwise_ln_kernel<4><<<grid, 256, 0, stream>>>(xh, taps, bias, ln_weight, ln_bias, yh, rows, L, C, K, eps);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}
