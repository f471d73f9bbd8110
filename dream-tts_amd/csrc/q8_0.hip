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

// The A-sharing form (with a workspace): a workgroup of 4 waves owns 64 columns (16 per wave)
// and a k range of NB blocks. The activation slab A[0:m, range] is read once per workgroup into
// LDS, where the four waves read their fragments; each lane's NB weight blocks are all requested
// before the slab is staged. For W8A8 the slab is quantised once while it is staged (int8 values
// and f16-rounded scales in LDS) instead of once per 16-column wave. The block arithmetic is
// gemm_q8_0's; with several ranges each
// workgroup writes its partial [m, 64] tile to part[range] and q8_merge sums the ranges in order.
// PACKED: the weights are in dtts_q8_0_repack's layout, where a lane's 8 quantised weights of
// consecutive blocks are contiguous (NB/2 16-byte loads) and the row's scales follow (NB/8
// loads), instead of 5 two-byte loads per 34-byte block.
template <int MB, int NB, bool A8, bool PACKED = false>
__global__ __launch_bounds__(256) void gemm_q8_lds(Q8Params p, float *part) {
    constexpr int KR = NB * 32;       // elements of a slab row
    constexpr int PITCH = KR + 8;     // f16 slab: 16 bytes of padding spread the fragment reads over banks
    constexpr int PITCH8 = KR + 16;   // int8 slab (W8A8), likewise
    constexpr int SEGS = KR / 8;      // 8-element segments per slab row
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    half_t *as = reinterpret_cast<half_t *>(smem);
    float *scale = reinterpret_cast<float *>(smem + MB * 16 * PITCH8);  // W8A8: [NB][MB * 16] f16-rounded scales
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, r = lane & 15;
    const int nblocks = p.k / 32;
    const int col = blockIdx.x * 64 + wave * 16 + r;
    const int b0 = blockIdx.y * NB;
    uint64_t q8[NB];
    float dw[NB];
    if constexpr (PACKED) {
        static_assert(NB % 8 == 0, "whole 16-byte loads of scales");
        const uint8_t *row = p.w + static_cast<int64_t>(col) * (p.k + 2 * nblocks);
        const uint8_t *qs = row + (static_cast<int64_t>(g) * nblocks + b0) * 8;
#pragma unroll
        for (int b = 0; b < NB; b += 2) {
            const uint4 v = *reinterpret_cast<const uint4 *>(qs + b * 8);
            q8[b] = static_cast<uint64_t>(v.x) | (static_cast<uint64_t>(v.y) << 32);
            q8[b + 1] = static_cast<uint64_t>(v.z) | (static_cast<uint64_t>(v.w) << 32);
        }
        const half_t *ds = reinterpret_cast<const half_t *>(row + p.k) + b0;
#pragma unroll
        for (int b = 0; b < NB; b += 8) {
            const half8_t v = *reinterpret_cast<const half8_t *>(ds + b);
#pragma unroll
            for (int j = 0; j < 8; ++j) dw[b + j] = static_cast<float>(v[j]);
        }
    } else {
        const uint8_t *wrow = p.w + (static_cast<int64_t>(col) * nblocks + b0) * 34;
#pragma unroll
        for (int b = 0; b < NB; ++b) load_wblock(wrow + b * 34, g, q8[b], dw[b]);
    }
    // MB * 16 * SEGS is a multiple of 256: every thread runs every staging iteration, so the
    // quad shuffles below see all four lanes of a block.
    for (int e = tid; e < MB * 16 * SEGS; e += 256) {
        const int row = e / SEGS, sg = e - (e / SEGS) * SEGS;
        half8_t v = half8_t{};
        if (row < p.m) v = *reinterpret_cast<const half8_t *>(p.x + static_cast<int64_t>(row) * p.k + b0 * 32 + sg * 8);
        if constexpr (A8) {
            // the row's block quantised once per workgroup (4 consecutive threads hold it)
            float f[8], amax = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                f[j] = static_cast<float>(v[j]);
                amax = fmaxf(amax, fabsf(f[j]));
            }
            amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint64_t qa = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int q = static_cast<int>(roundf(f[j] * id));
                qa |= static_cast<uint64_t>(static_cast<uint8_t>(static_cast<int8_t>(q))) << (8 * j);
            }
            *reinterpret_cast<uint64_t *>(smem + row * PITCH8 + sg * 8) = qa;
            if ((sg & 3) == 0) scale[(sg >> 2) * (MB * 16) + row] = static_cast<float>(static_cast<half_t>(d));
        } else {
            *reinterpret_cast<half8_t *>(as + row * PITCH + sg * 8) = v;
        }
    }
    __syncthreads();
    float4v acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            if constexpr (A8) {
                const uint64_t qa = *reinterpret_cast<const uint64_t *>(smem + (mb * 16 + r) * PITCH8 + b * 32 + g * 8);
                const int4v dot = __builtin_amdgcn_mfma_i32_16x16x32_i8(static_cast<long>(qa), static_cast<long>(q8[b]),
                                                                         int4v{0, 0, 0, 0}, 0, 0, 0);
                // the C fragment holds rows 4g + i
                const float4v dx = *reinterpret_cast<const float4v *>(scale + b * (MB * 16) + mb * 16 + g * 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float t = (static_cast<float>(dot[i]) * dw[b]) * dx[i];
                    acc[mb][i] += t;
                }
            } else {
                const half8_t xv = *reinterpret_cast<const half8_t *>(as + (mb * 16 + r) * PITCH + b * 32 + g * 8);
                half8_t wv;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    wv[j] = static_cast<half_t>(static_cast<float>(static_cast<int8_t>((q8[b] >> (8 * j)) & 0xff)));
                const float4v pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, wv, float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mb][i] += pr[i] * dw[b];
            }
        }
    }
    float *dst = part ? part + static_cast<int64_t>(blockIdx.y) * p.m * p.n : p.y;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mb * 16 + g * 4 + i;
            if (row < p.m) dst[static_cast<int64_t>(row) * p.n + col] = acc[mb][i];
        }
}

// y = the k ranges' partials summed in range order.
__global__ __launch_bounds__(256) void q8_merge(const float *part, float *y, int64_t mn, int ranges) {
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < mn; e += int64_t(gridDim.x) * 256) {
        float s = part[e];
        for (int q = 1; q < ranges; ++q) s += part[q * mn + e];
        y[e] = s;
    }
}

// Blocks per k range for the A-sharing kernel: the widest range that still gives >= 192
// workgroups and keeps the f16 slab within 64 KB of LDS (else the narrowest); 0 when the shape
// does not fit it.
int pick_q8_nb(int64_t m, int64_t k, int64_t n) {
    const int64_t nblocks = k / 32, tiles = n / 64, rows = (m + 15) / 16 * 16;
    if (m <= 0 || m > 64 || n % 64 != 0 || nblocks % 8 != 0 || tiles >= 65536) return 0;
    for (int nb : {32, 16})
        if (nblocks % nb == 0 && tiles * (nblocks / nb) >= 192 && rows * (nb * 32 + 8) * 2 <= 65536) return nb;
    return 8;
}

// GGML blocks -> the packed layout: row n is k bytes of quantised weights, lane-group major
// (group g's 8 weights of block b at g * nblocks * 8 + b * 8: weights 8g .. 8g + 7 of the block),
// then the nblocks f16 scales. One thread per (row, block).
__global__ __launch_bounds__(256) void repack_q8_0(const uint8_t *blocks, uint8_t *packed, int64_t rows, int nblocks) {
    const int64_t total = rows * nblocks;
    const int64_t stride = static_cast<int64_t>(nblocks) * 34;  // k + 2 * nblocks bytes per row
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t r = e / nblocks;
        const int b = static_cast<int>(e - r * nblocks);
        const uint8_t *blk = blocks + e * 34;
        uint8_t *row = packed + r * stride;
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int j = 0; j < 8; ++j) row[(static_cast<int64_t>(g) * nblocks + b) * 8 + j] = blk[2 + 8 * g + j];
        reinterpret_cast<uint16_t *>(row + static_cast<int64_t>(nblocks) * 32)[b] = ld16(blk);
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

extern "C" size_t dtts_gemm_q8_0_workspace_bytes(int64_t m, int64_t k, int64_t n) {
    if (m <= 0 || k <= 0 || n <= 0 || k % 32 != 0) return 0;
    const int nb = dtts::pick_q8_nb(m, k, n);
    const int64_t ranges = nb ? k / 32 / nb : 1;
    return ranges > 1 ? static_cast<size_t>(ranges * m * n) * sizeof(float) : 0;
}

namespace dtts {
namespace {

int q8_lds_launch(const char *name, const dtts_f16 *x, const void *w, float *y, int64_t m, int64_t k, int64_t n,
                  int32_t mode, int nb, void *workspace, bool packed, hipStream_t stream) {
    const int64_t ranges = k / 32 / nb;
    const size_t need = ranges > 1 ? static_cast<size_t>(ranges * m * n) * sizeof(float) : 0;
    DTTS_REQUIRE(k < (int64_t(1) << 30) && n < (int64_t(1) << 30), "%s: shape too large", name);
    Q8Params p{};
    p.x = reinterpret_cast<const half_t *>(x);
    p.w = static_cast<const uint8_t *>(w);
    p.y = y;
    p.m = static_cast<int>(m);
    p.k = static_cast<int>(k);
    p.n = static_cast<int>(n);
    float *part = need ? static_cast<float *>(workspace) : nullptr;
    const int mb = static_cast<int>((m + 15) / 16);
    const size_t lds = mode == DTTS_Q8_W8A8 ? static_cast<size_t>(mb) * 16 * (nb * 32 + 16) + nb * mb * 16 * 4
                                            : static_cast<size_t>(mb) * 16 * (nb * 32 + 8) * 2;
    const dim3 grid(static_cast<unsigned>(n / 64), static_cast<unsigned>(ranges));
    const bool a8 = mode == DTTS_Q8_W8A8;
#define DTTS_Q8L(MB, NB)                                                                              \
    if (packed) {                                                                                     \
        if (a8)                                                                                       \
            gemm_q8_lds<MB, NB, true, true><<<grid, 256, lds, stream>>>(p, part);                     \
        else                                                                                          \
            gemm_q8_lds<MB, NB, false, true><<<grid, 256, lds, stream>>>(p, part);                    \
    } else if (a8) {                                                                                  \
        gemm_q8_lds<MB, NB, true, false><<<grid, 256, lds, stream>>>(p, part);                        \
    } else {                                                                                          \
        gemm_q8_lds<MB, NB, false, false><<<grid, 256, lds, stream>>>(p, part);                       \
    }
#define DTTS_Q8L_NB(MB)         \
    if (nb == 32) {             \
        DTTS_Q8L(MB, 32)        \
    } else if (nb == 16) {      \
        DTTS_Q8L(MB, 16)        \
    } else {                    \
        DTTS_Q8L(MB, 8)         \
    }
    switch (mb) {
        case 1: DTTS_Q8L_NB(1) break;
        case 2: DTTS_Q8L_NB(2) break;
        case 3: DTTS_Q8L_NB(3) break;
        default: DTTS_Q8L_NB(4) break;
    }
#undef DTTS_Q8L_NB
#undef DTTS_Q8L
    DTTS_LAUNCH_CHECK(name);
    if (part) {
        q8_merge<<<grid_for(m * n, 256), 256, 0, stream>>>(part, y, m * n, static_cast<int>(ranges));
        DTTS_LAUNCH_CHECK(name);
    }
    return DTTS_OK;
}

}  // namespace
}  // namespace dtts

extern "C" int dtts_gemm_q8_0_ws(const dtts_f16 *x, const void *blocks, float *y, int64_t m, int64_t k, int64_t n,
                                 int32_t mode, void *workspace, size_t ws_bytes, hipStream_t stream) {
    const char *name = "dtts_gemm_q8_0_ws";
    DTTS_REQUIRE(m >= 0 && k > 0 && n > 0 && k % 32 == 0, "%s: bad shape (%lld, %lld, %lld)", name, (long long)m,
                 (long long)k, (long long)n);
    DTTS_REQUIRE(mode == DTTS_Q8_W8A16 || mode == DTTS_Q8_W8A8, "%s: mode %d unknown", name, mode);
    if (m == 0) return DTTS_OK;
    // On the GGML layout the A-sharing kernel pays for its 2-byte weight loads only once a slab
    // serves more than 16 rows (measured at m = 1, 8 and 48); below that, and without room for
    // the ranges, the workspace-free kernel runs.
    const int nb = m > 16 ? dtts::pick_q8_nb(m, k, n) : 0;
    const size_t need = dtts_gemm_q8_0_workspace_bytes(m, k, n);
    if (!nb || (need && (!workspace || ws_bytes < need)))
        return dtts_gemm_q8_0(x, blocks, y, m, k, n, mode, stream);
    DTTS_REQUIRE(x && blocks && y, "%s: null pointer", name);
    DTTS_REQUIRE(dtts::aligned(x, 16) && dtts::aligned(blocks, 2) && (!need || dtts::aligned(workspace, 16)),
                 "%s: x and the workspace must be 16-byte aligned", name);
    return dtts::q8_lds_launch(name, x, blocks, y, m, k, n, mode, nb, workspace, false, stream);
}

extern "C" size_t dtts_q8_0_packed_bytes(int64_t rows, int64_t k) {
    return rows > 0 && k > 0 && k % 32 == 0 ? static_cast<size_t>(rows) * (k / 32) * 34 : 0;
}

extern "C" int dtts_q8_0_repack(const void *blocks, void *packed, int64_t rows, int64_t k, hipStream_t stream) {
    const char *name = "dtts_q8_0_repack";
    DTTS_REQUIRE(rows >= 0 && k > 0 && k % 256 == 0, "%s: k = %lld is not a multiple of 256", name, (long long)k);
    if (rows == 0) return DTTS_OK;
    DTTS_REQUIRE(blocks && packed && blocks != packed, "%s: null or aliased pointers", name);
    DTTS_REQUIRE(dtts::aligned(blocks, 2) && dtts::aligned(packed, 16), "%s: packed must be 16-byte aligned", name);
    DTTS_REQUIRE(k < (int64_t(1) << 30) && rows < (int64_t(1) << 30), "%s: shape too large", name);
    dtts::repack_q8_0<<<dtts::grid_for(rows * (k / 32), 256), 256, 0, stream>>>(
        static_cast<const uint8_t *>(blocks), static_cast<uint8_t *>(packed), rows, static_cast<int>(k / 32));
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

extern "C" int dtts_gemm_q8_0_packed(const dtts_f16 *x, const void *packed, float *y, int64_t m, int64_t k, int64_t n,
                                     int32_t mode, void *workspace, size_t ws_bytes, hipStream_t stream) {
    const char *name = "dtts_gemm_q8_0_packed";
    DTTS_REQUIRE(m >= 0 && k > 0 && n > 0 && k % 256 == 0 && n % 64 == 0,
                 "%s: bad shape (%lld, %lld, %lld): k a multiple of 256, n of 64", name, (long long)m, (long long)k,
                 (long long)n);
    DTTS_REQUIRE(mode == DTTS_Q8_W8A16 || mode == DTTS_Q8_W8A8, "%s: mode %d unknown", name, mode);
    if (m == 0) return DTTS_OK;
    DTTS_REQUIRE(m <= 64, "%s: m = %lld > 64 (decode shapes only)", name, (long long)m);
    DTTS_REQUIRE(x && packed && y, "%s: null pointer", name);
    const int nb = dtts::pick_q8_nb(m, k, n);
    const size_t need = dtts_gemm_q8_0_workspace_bytes(m, k, n);
    DTTS_REQUIRE(nb > 0, "%s: shape not supported", name);
    DTTS_REQUIRE(!need || (workspace && ws_bytes >= need), "%s: workspace %zu bytes < %zu needed", name, ws_bytes, need);
    DTTS_REQUIRE(dtts::aligned(x, 16) && dtts::aligned(packed, 16) && (!need || dtts::aligned(workspace, 16)),
                 "%s: x, packed and the workspace must be 16-byte aligned", name);
    return dtts::q8_lds_launch(name, x, packed, y, m, k, n, mode, nb, workspace, true, stream);
}
