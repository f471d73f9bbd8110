// Q8_0 projections in candle's GGML block layout: weight row n holds k/32 consecutive blocks
// {f16 d; i8 qs[32]} (34 bytes), w[n, k] = qs[n][k/32][k%32] * d[n][k/32].
//
// y[m, n] = sum over blocks b of d_w[n,b] * (block dot), m <= 64 lanes:
//   W8A16: the block dot of f16 activations against the exact f16 images of the int8 weights
//          (v_mfma_f32_16x16x32_f16: one MFMA is one block), scaled by d_w in f32;
//   W8A8:  activations quantized per 32-block in registers exactly as Q8_0 quantizes
//          (amax/127, round half away from zero, f16 scale), the block dot exact in i32
//          (v_mfma_i32_16x16x32_i8), then ((float)dot * d_w) * d_x summed in block order -- the
//          vec_dot arithmetic candle's CPU QMatMul is believed to perform.
// Blocks start at 2-byte alignment, so the weights are read as 16-bit units. Like the f16
// skinny GEMM, a wave owns 16 columns, waves of a workgroup split k, and the partials are summed
// through LDS in slab order.
#include <cmath>
#include <cstring>

#include "common.hpp"

#pragma clang fp contract(off)

namespace dtts {
namespace {

typedef float float4v __attribute__((ext_vector_type(4)));
typedef int int4v __attribute__((ext_vector_type(4)));

struct Q8Params {
    const half_t *x;       // [m, k]
    const uint8_t *w;      // [n][k/32] blocks of 34 bytes
    float *y;              // [m, n]
    int m, k, n, ks, slab_blocks;
};

__device__ __forceinline__ uint16_t ld16(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }

// The lane's 8 quantized weights (k-group g of block blk of row n) and the block's scale.
__device__ __forceinline__ void load_wblock(const uint8_t *blk, int g, uint64_t &q8, float &d) {
    const uint8_t *qs = blk + 2 + g * 8;
    q8 = static_cast<uint64_t>(ld16(qs)) | (static_cast<uint64_t>(ld16(qs + 2)) << 16) |
         (static_cast<uint64_t>(ld16(qs + 4)) << 32) | (static_cast<uint64_t>(ld16(qs + 6)) << 48);
    const uint16_t dh = ld16(blk);
    half_t h;
    __builtin_memcpy(&h, &dh, 2);
    d = static_cast<float>(h);
}

template <int MB, bool A8>
__global__ __launch_bounds__(1024) void gemm_q8_0(Q8Params p) {
    extern __shared__ __attribute__((aligned(16))) float red[];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int kslab = wave;
    const int g = lane >> 4;
    const int r = lane & 15;
    const int nblocks = p.k / 32;
    const int col = blockIdx.x * 16 + r;
    const uint8_t *wrow = p.w + static_cast<int64_t>(col) * nblocks * 34;
    const int b0 = kslab * p.slab_blocks;
    float4v acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = float4v{0.f, 0.f, 0.f, 0.f};
    const half_t *xr[MB];
    bool xrow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int row = mb * 16 + r;
        xrow[mb] = row < p.m;
        xr[mb] = p.x + static_cast<int64_t>(xrow[mb] ? row : 0) * p.k + g * 8;
    }
    for (int b = b0; b < b0 + p.slab_blocks; ++b) {
        uint64_t q8;
        float dw;
        load_wblock(wrow + static_cast<int64_t>(b) * 34, g, q8, dw);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            half8_t xv = *reinterpret_cast<const half8_t *>(xr[mb] + b * 32);
            if (!xrow[mb]) xv = half8_t{};
            if constexpr (A8) {
                // Q8_0 quantization of this row's block: amax over the 4 lanes holding it
                float v[8], amax = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    v[j] = static_cast<float>(xv[j]);
                    amax = fmaxf(amax, fabsf(v[j]));
                }
                amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
                amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
                const float d = amax / 127.0f;
                const float id = d != 0.0f ? 1.0f / d : 0.0f;
                uint64_t qa = 0;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int q = static_cast<int>(roundf(v[j] * id));
                    qa |= static_cast<uint64_t>(static_cast<uint8_t>(static_cast<int8_t>(q))) << (8 * j);
                }
                const float dx = static_cast<float>(static_cast<half_t>(d));
                const int4v dot = __builtin_amdgcn_mfma_i32_16x16x32_i8(static_cast<long>(qa), static_cast<long>(q8),
                                                                         int4v{0, 0, 0, 0}, 0, 0, 0);
                // the C fragment holds rows 4g + i; their scales live in lanes 4g + i
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float dxi = __shfl(dx, g * 4 + i, 64);
                    const float t = (static_cast<float>(dot[i]) * dw) * dxi;
                    acc[mb][i] += t;
                }
            } else {
                half8_t wv;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    wv[j] = static_cast<half_t>(static_cast<float>(static_cast<int8_t>((q8 >> (8 * j)) & 0xff)));
                const float4v part = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, wv, float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mb][i] += part[i] * dw;
            }
        }
    }
    float *mine = red + static_cast<int64_t>(kslab) * MB * 256;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) *reinterpret_cast<float4v *>(mine + mb * 256 + lane * 4) = acc[mb];
    __syncthreads();
    if (kslab != 0) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        float4v s = float4v{0.f, 0.f, 0.f, 0.f};
        for (int sl = 0; sl < p.ks; ++sl) s += *reinterpret_cast<const float4v *>(red + (sl * MB + mb) * 256 + lane * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mb * 16 + g * 4 + i;
            if (row < p.m) p.y[static_cast<int64_t>(row) * p.n + col] = s[i];
        }
    }
}

__global__ __launch_bounds__(256) void dequant_q8_0(const uint8_t *blocks, float *w, int64_t rows, int64_t k) {
    const int64_t total = rows * k;
    const int64_t nb = k / 32;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t r = e / k;
        const int64_t c = e - r * k;
        const uint8_t *blk = blocks + (r * nb + c / 32) * 34;
        const uint16_t dh = ld16(blk);
        half_t h;
        __builtin_memcpy(&h, &dh, 2);
        w[e] = static_cast<float>(static_cast<int8_t>(blk[2 + c % 32])) * static_cast<float>(h);
    }
}

int pick_ks_blocks(int64_t groups, int64_t nblocks) {
    int ks = 1;
    while (ks * 2 <= 16 && nblocks % (ks * 2) == 0 && nblocks / (ks * 2) >= 4 && groups * ks < 1024) ks *= 2;
    return ks;
}

}  // namespace
}  // namespace dtts

using dtts::half_t;

extern "C" int dtts_q8_0_quantize(const float *w, void *blocks, int64_t rows, int64_t k) {
    DTTS_REQUIRE(rows >= 0 && k > 0 && k % 32 == 0, "dtts_q8_0_quantize: k = %lld is not a multiple of 32",
                 (long long)k);
    DTTS_REQUIRE(rows == 0 || (w && blocks), "dtts_q8_0_quantize: null pointer");
    uint8_t *out = static_cast<uint8_t *>(blocks);
    const int64_t nb = k / 32;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const float *src = w + r * k + b * 32;
            uint8_t *blk = out + (r * nb + b) * 34;
            float amax = 0.0f;
            for (int j = 0; j < 32; ++j) amax = std::fmax(amax, std::fabs(src[j]));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const _Float16 dh = static_cast<_Float16>(d);
            std::memcpy(blk, &dh, 2);
            for (int j = 0; j < 32; ++j) blk[2 + j] = static_cast<uint8_t>(static_cast<int8_t>(std::round(src[j] * id)));
        }
    return DTTS_OK;
}

extern "C" int dtts_q8_0_dequantize_f32(const void *blocks, float *w, int64_t rows, int64_t k, hipStream_t stream) {
    DTTS_REQUIRE(rows >= 0 && k > 0 && k % 32 == 0, "dtts_q8_0_dequantize_f32: bad shape");
    if (rows == 0) return DTTS_OK;
    DTTS_REQUIRE(blocks && w, "dtts_q8_0_dequantize_f32: null pointer");
    DTTS_REQUIRE(dtts::aligned(blocks, 2), "dtts_q8_0_dequantize_f32: blocks must be 2-byte aligned");
    dtts::dequant_q8_0<<<dtts::grid_for(rows * k, 256), 256, 0, stream>>>(static_cast<const uint8_t *>(blocks), w, rows, k);
    DTTS_LAUNCH_CHECK("dtts_q8_0_dequantize_f32");
    return DTTS_OK;
}

extern "C" int dtts_gemm_q8_0(const dtts_f16 *x, const void *blocks, float *y, int64_t m, int64_t k, int64_t n,
                              int32_t mode, hipStream_t stream) {
    const char *name = "dtts_gemm_q8_0";
    DTTS_REQUIRE(m >= 0 && k > 0 && n > 0 && k % 32 == 0, "%s: bad shape (%lld, %lld, %lld)", name, (long long)m,
                 (long long)k, (long long)n);
    DTTS_REQUIRE(mode == DTTS_Q8_W8A16 || mode == DTTS_Q8_W8A8, "%s: mode %d unknown", name, mode);
    if (m == 0) return DTTS_OK;
    DTTS_REQUIRE(x && blocks && y, "%s: null pointer", name);
    DTTS_REQUIRE(m <= 64, "%s: m = %lld > 64 (decode shapes only)", name, (long long)m);
    DTTS_REQUIRE(n % 16 == 0, "%s: n = %lld not a multiple of 16", name, (long long)n);
    DTTS_REQUIRE(dtts::aligned(x, 16) && dtts::aligned(blocks, 2), "%s: x must be 16-byte aligned", name);
    DTTS_REQUIRE(k < (int64_t(1) << 30) && n < (int64_t(1) << 30), "%s: shape too large", name);
    dtts::Q8Params p{};
    p.x = reinterpret_cast<const half_t *>(x);
    p.w = static_cast<const uint8_t *>(blocks);
    p.y = y;
    p.m = static_cast<int>(m);
    p.k = static_cast<int>(k);
    p.n = static_cast<int>(n);
    const int64_t groups = n / 16;
    p.ks = dtts::pick_ks_blocks(groups, k / 32);
    p.slab_blocks = static_cast<int>(k / 32 / p.ks);
    const int mb = static_cast<int>((m + 15) / 16);
    const unsigned threads = static_cast<unsigned>(64 * p.ks);
    const size_t lds = static_cast<size_t>(p.ks) * mb * 256 * 4;
    const unsigned grid = static_cast<unsigned>(groups);
    const bool a8 = mode == DTTS_Q8_W8A8;
#define DTTS_Q8_LAUNCH(MB)                                                                                            \
    if (a8)                                                                                                           \
        dtts::gemm_q8_0<MB, true><<<grid, threads, lds, stream>>>(p);                                                 \
    else                                                                                                              \
        dtts::gemm_q8_0<MB, false><<<grid, threads, lds, stream>>>(p);
    switch (mb) {
        case 1: DTTS_Q8_LAUNCH(1) break;
        case 2: DTTS_Q8_LAUNCH(2) break;
        case 3: DTTS_Q8_LAUNCH(3) break;
        default: DTTS_Q8_LAUNCH(4) break;
    }
#undef DTTS_Q8_LAUNCH
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}
