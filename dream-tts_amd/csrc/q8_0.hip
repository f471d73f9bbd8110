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
#include <type_traits>

#include "common.hpp"

#pragma clang fp contract(off)

namespace dtts {
namespace {

typedef float float4v __attribute__((ext_vector_type(4)));
typedef int int4v __attribute__((ext_vector_type(4)));

// Activation modes (the DTTS_Q8_* values).
constexpr int kA16 = DTTS_Q8_W8A16, kA8 = DTTS_Q8_W8A8, kA32 = DTTS_Q8_W8A32;

template <typename XT>
struct Q8Params {
    const XT *x;           // [m, k], f16 or f32
    const uint8_t *w;      // [n][k/32] blocks of 34 bytes (or the packed layout)
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

// 8 consecutive activations as f32 (f16 widens exactly), zero when the row is absent.
__device__ __forceinline__ void load_x8(const half_t *p, bool valid, float v[8]) {
    half8_t h = valid ? *reinterpret_cast<const half8_t *>(p) : half8_t{};
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = static_cast<float>(h[j]);
}
__device__ __forceinline__ void load_x8(const float *p, bool valid, float v[8]) {
    float4v a = float4v{0.f, 0.f, 0.f, 0.f}, b = a;
    if (valid) {
        a = *reinterpret_cast<const float4v *>(p);
        b = *reinterpret_cast<const float4v *>(p + 4);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[j] = a[j];
        v[4 + j] = b[j];
    }
}

// Q8_0 quantization of one 32-block of activations held 8 per lane by the four lanes XOR-ed
// together by X1 and X2 (amax/127, round half away from zero, the scale rounded to f16):
// exactly the weight quantizer's rule, applied to the values as given (f32 activations are
// quantized directly, with no f16 rounding first).
template <int X1, int X2>
__device__ __forceinline__ uint64_t quant_block8(const float v[8], float &dx) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, __shfl_xor(amax, X1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, X2, 64));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint64_t qa = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q = static_cast<int>(roundf(v[j] * id));
        qa |= static_cast<uint64_t>(static_cast<uint8_t>(static_cast<int8_t>(q))) << (8 * j);
    }
    dx = static_cast<float>(static_cast<half_t>(d));
    return qa;
}

// W8A32: one 32-block of f32 activations as two f16 terms for the f16 matrix cores. The block is
// scaled by 2^e so its amax lies in [2^14, 2^15) (f16 range, and lo = s - f16(s) kept normal for
// the block's large entries), then s = hi + lo with hi = f16(s) and lo = f16(s - hi); s - hi is
// exact in f32, so the pair carries s to 2^-22 of the block's amax. inv = 2^-e undoes the scale.
template <int X1, int X2>
__device__ __forceinline__ void split_block8(const float v[8], half8_t &hi, half8_t &lo, float &inv) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, __shfl_xor(amax, X1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, X2, 64));
    int e = 0;
    if (amax > 0.0f) {
        int ex;
        frexpf(amax, &ex);  // amax = f * 2^ex, f in [0.5, 1)
        e = min(max(15 - ex, -126), 126);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float s = ldexpf(v[j], e);
        const half_t h = static_cast<half_t>(s);
        hi[j] = h;
        lo[j] = static_cast<half_t>(s - static_cast<float>(h));
    }
    inv = ldexpf(1.0f, -e);
}

// The lane's 8 int8 weights as exact f16 values.
__device__ __forceinline__ half8_t widen_w8(uint64_t q8) {
    half8_t wv;
#pragma unroll
    for (int j = 0; j < 8; ++j) wv[j] = static_cast<half_t>(static_cast<float>(static_cast<int8_t>((q8 >> (8 * j)) & 0xff)));
    return wv;
}

template <int MB, int MODE, typename XT>
__global__ __launch_bounds__(1024) void gemm_q8_0(Q8Params<XT> p) {
    static_assert(MODE != kA16 || sizeof(XT) == 2, "W8A16 takes f16 activations");
    static_assert(MODE != kA32 || sizeof(XT) == 4, "W8A32 takes f32 activations");
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
    const XT *xr[MB];
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
            if constexpr (MODE == kA16) {
                half8_t xv = *reinterpret_cast<const half8_t *>(xr[mb] + b * 32);
                if (!xrow[mb]) xv = half8_t{};
                const float4v part = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, widen_w8(q8), float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mb][i] += part[i] * dw;
            } else {
                float v[8];
                load_x8(xr[mb] + b * 32, xrow[mb], v);
                if constexpr (MODE == kA8) {
                    // Q8_0 quantization of this row's block: amax over the 4 lanes holding it
                    float dx;
                    const uint64_t qa = quant_block8<16, 32>(v, dx);
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
                    half8_t hi, lo;
                    float inv;
                    split_block8<16, 32>(v, hi, lo, inv);
                    const half8_t wv = widen_w8(q8);
                    float4v part = __builtin_amdgcn_mfma_f32_16x16x32_f16(lo, wv, float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    part = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi, wv, part, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[mb][i] += (part[i] * dw) * __shfl(inv, g * 4 + i, 64);
                }
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

// One launch at short k (k * ceil(m/16) <= 3072, as the f16 projections): workgroup x owns 16
// columns and all of k, wave w (at most 8) the NBW blocks from w * NBW. Every lane requests its weights (the
// packed layout's contiguous 8-byte groups and scales, or the GGML blocks' 2-byte units) and its
// activations for all NBW blocks before the first MFMA -- gemm_q8_0 above walks its slab a block
// at a time, one memory round trip each. The block arithmetic is gemm_q8_0's; the waves' partials
// meet in LDS and are summed in wave order, with no workspace and no merge launch. W8A16 and
// W8A32 only (q8_row_wins).
template <int MB, int NBW, int MODE, bool PACKED, typename XT>
__global__ __launch_bounds__(512) void gemm_q8_row(Q8Params<XT> p) {
    static_assert((MODE == kA16 && sizeof(XT) == 2) || (MODE == kA32 && sizeof(XT) == 4),
                  "W8A16 on f16 activations or W8A32 on f32 ones (q8_row_wins)");
    static_assert(NBW % 2 == 0, "whole 16-byte weight loads and 4-byte scale loads");
    extern __shared__ __attribute__((aligned(16))) float4v qsum[];  // [waves][MB][64]
    const int nw = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g = lane >> 4, r = lane & 15;
    const int nblocks = p.k / 32;
    const int col = blockIdx.x * 16 + r;
    const int b0 = wave * NBW;
    uint64_t q8[NBW];
    float dw[NBW];
    if constexpr (PACKED) {
        const uint8_t *row = p.w + static_cast<int64_t>(col) * (p.k + 2 * nblocks);
        const uint8_t *qs = row + (static_cast<int64_t>(g) * nblocks + b0) * 8;
#pragma unroll
        for (int b = 0; b < NBW; b += 2) {
            const uint4 v = *reinterpret_cast<const uint4 *>(qs + b * 8);
            q8[b] = static_cast<uint64_t>(v.x) | (static_cast<uint64_t>(v.y) << 32);
            q8[b + 1] = static_cast<uint64_t>(v.z) | (static_cast<uint64_t>(v.w) << 32);
        }
        const uint32_t *ds = reinterpret_cast<const uint32_t *>(row + p.k + 2 * b0);
#pragma unroll
        for (int b = 0; b < NBW; b += 2) {
            const uint32_t v = ds[b / 2];
            half_t h0, h1;
            const uint16_t u0 = static_cast<uint16_t>(v & 0xffff), u1 = static_cast<uint16_t>(v >> 16);
            __builtin_memcpy(&h0, &u0, 2);
            __builtin_memcpy(&h1, &u1, 2);
            dw[b] = static_cast<float>(h0);
            dw[b + 1] = static_cast<float>(h1);
        }
    } else {
        const uint8_t *wrow = p.w + (static_cast<int64_t>(col) * nblocks + b0) * 34;
#pragma unroll
        for (int b = 0; b < NBW; ++b) load_wblock(wrow + b * 34, g, q8[b], dw[b]);
    }
    // the lane's activations: row mb * 16 + r, elements 8g .. 8g + 7 of each block
    typedef typename std::conditional<sizeof(XT) == 2, half8_t, float4v>::type XV;
    constexpr int XW = sizeof(XT) == 2 ? 1 : 2;  // vectors per 8 elements
    XV xv[MB][NBW][XW];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int row = mb * 16 + r;
        const XT *xr = p.x + static_cast<int64_t>(row < p.m ? row : 0) * p.k + b0 * 32 + g * 8;
#pragma unroll
        for (int b = 0; b < NBW; ++b)
#pragma unroll
            for (int j = 0; j < XW; ++j) xv[mb][b][j] = *reinterpret_cast<const XV *>(xr + b * 32 + j * 4);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is in flight before the first wait
    float4v acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NBW; ++b)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const bool live = mb * 16 + r < p.m;  // rows past m carry zeros
            if constexpr (MODE == kA16) {
                const half8_t x8 = live ? xv[mb][b][0] : half8_t{};
                const float4v pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(x8, widen_w8(q8[b]), float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mb][i] += pr[i] * dw[b];
            } else {
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = live ? xv[mb][b][j / 4][j % 4] : 0.0f;
                half8_t hi, lo;
                float inv;
                split_block8<16, 32>(v, hi, lo, inv);
                const half8_t wv = widen_w8(q8[b]);
                float4v pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(lo, wv, float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi, wv, pr, 0, 0, 0);
                // the C fragment holds rows 4g + i; their scales live in lanes 4g + i
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mb][i] += (pr[i] * dw[b]) * __shfl(inv, g * 4 + i, 64);
            }
        }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) qsum[(wave * MB + mb) * 64 + lane] = acc[mb];
    __syncthreads();
    // C layout of 16x16: lane l holds column l & 15, rows 4 * (l >> 4) + i
    for (int t = threadIdx.x; t < MB * 64; t += blockDim.x) {
        const int mb = t >> 6, l = t & 63;
        float4v s = qsum[mb * 64 + l];
        for (int q = 1; q < nw; ++q) s += qsum[(q * MB + mb) * 64 + l];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mb * 16 + (l >> 4) * 4 + i;
            if (row < p.m) p.y[static_cast<int64_t>(row) * p.n + blockIdx.x * 16 + (l & 15)] = s[i];
        }
    }
}

// The (row blocks, blocks per wave) pairs q8_row_launch instantiates: 4 blocks per wave at any
// row-block count, 6 up to two row blocks, 8 and 12 for one (a lane holds MB x NBW activation
// blocks in registers).
constexpr bool q8_row_instantiated(int64_t mb, int nbw) {
    return nbw == 4 || (nbw == 6 && mb <= 2) || ((nbw == 8 || nbw == 12) && mb == 1);
}

// Blocks per wave for gemm_q8_row (0: not applicable): the fewest of 4, 6, 8 and 12 that need at
// most 8 waves (two waves per SIMD, so a lane's activations for its blocks fit its registers) and
// are instantiated for the row-block count; m <= 64, k * ceil(m/16) <= 3072, n a multiple of 16.
int pick_q8_row(int64_t m, int64_t k, int64_t n) {
    if (m <= 0 || m > 64 || k % 32 != 0 || n % 16 != 0 || n / 16 >= 65536) return 0;
    const int64_t mb = (m + 15) / 16;
    if (k * mb > 3072) return 0;
    const int64_t nblocks = k / 32;
    for (int nbw : {4, 6, 8, 12})
        if (nblocks % nbw == 0 && nblocks / nbw <= 8 && q8_row_instantiated(mb, nbw)) return nbw;
    return 0;
}

// Where the one-launch kernel beats the A-sharing kernel and its merge (measured at config 4's
// shapes, m = 1, 8 and 48, graph-replayed): W8A16 on the packed layout everywhere it applies, and
// on GGML blocks (five 2-byte loads per block) up to 4 blocks per wave; W8A32 on the packed
// layout up to 4 blocks per wave at m <= 16. Not W8A8: every workgroup would quantize all of x
// again, where the A-sharing kernel quantizes its slab once per 64 columns.
bool q8_row_wins(int32_t mode, bool packed, int nbw, int64_t m) {
    if (nbw == 0) return false;
    if (mode == DTTS_Q8_W8A16) return packed || nbw == 4;
    if (mode == DTTS_Q8_W8A32) return packed && nbw == 4 && m <= 16;
    return false;
}

// LDS of the A-sharing kernel: the activation slab of MB*16 rows by NB blocks as f16 (W8A16),
// int8 codes plus f32 scales (W8A8), or f16 hi and lo slabs plus f32 inverse scales (W8A32).
constexpr int q8_pitch(int nb) { return nb * 32 + 8; }    // f16 slab row: 16 bytes of padding spread the fragment reads over banks
constexpr int q8_pitch8(int nb) { return nb * 32 + 16; }  // int8 slab row, likewise
constexpr size_t q8_lds_bytes(int mb, int nb, int mode) {
    return mode == kA16   ? static_cast<size_t>(mb) * 16 * q8_pitch(nb) * 2
           : mode == kA8 ? static_cast<size_t>(mb) * 16 * q8_pitch8(nb) + static_cast<size_t>(nb) * mb * 16 * 4
                          : static_cast<size_t>(mb) * 16 * q8_pitch(nb) * 2 * 2 + static_cast<size_t>(nb) * mb * 16 * 4;
}
constexpr size_t kQ8MaxLds = 160 * 1024;  // gfx950's LDS per workgroup

// The A-sharing form (with a workspace): a workgroup of 4 waves owns 64 columns (16 per wave)
// and a k range of NB blocks. The activation slab A[0:m, range] is read once per workgroup into
// LDS, where the four waves read their fragments; each lane's NB weight blocks are all requested
// before the slab is staged. For W8A8 the slab is quantised once while it is staged (int8 values
// and f16-rounded scales in LDS) instead of once per 16-column wave; for W8A32 it is split once
// into its scaled f16 hi and lo terms. The block arithmetic is gemm_q8_0's; with several ranges
// each workgroup writes its partial [m, 64] tile to part[range] and q8_merge sums the ranges in
// order.
// PACKED: the weights are in dtts_q8_0_repack's layout, where a lane's 8 quantised weights of
// consecutive blocks are contiguous (NB/2 16-byte loads) and the row's scales follow (NB/8
// loads), instead of 5 two-byte loads per 34-byte block.
template <int MB, int NB, int MODE, bool PACKED, typename XT>
__global__ __launch_bounds__(256) void gemm_q8_lds(Q8Params<XT> p, float *part) {
    static_assert(MODE != kA16 || sizeof(XT) == 2, "W8A16 takes f16 activations");
    static_assert(MODE != kA32 || sizeof(XT) == 4, "W8A32 takes f32 activations");
    constexpr int KR = NB * 32;       // elements of a slab row
    constexpr int PITCH = q8_pitch(NB);
    constexpr int PITCH8 = q8_pitch8(NB);
    constexpr int SEGS = KR / 8;      // 8-element segments per slab row
    constexpr size_t LDS = q8_lds_bytes(MB, NB, MODE);
    static_assert(LDS <= kQ8MaxLds, "slab exceeds the LDS");
    __shared__ __attribute__((aligned(16))) unsigned char smem[LDS];
    half_t *as = reinterpret_cast<half_t *>(smem);
    half_t *as_lo = as + MB * 16 * PITCH;  // W8A32: the lo slab follows the hi slab
    // [NB][MB * 16] per-row block scales: W8A8's f16-rounded d_x, W8A32's 2^-e
    float *scale = reinterpret_cast<float *>(smem + (MODE == kA8 ? MB * 16 * PITCH8 : MB * 16 * PITCH * 4));
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
        const XT *src = p.x + static_cast<int64_t>(row < p.m ? row : 0) * p.k + b0 * 32 + sg * 8;
        if constexpr (MODE == kA16) {
            half8_t v = half8_t{};
            if (row < p.m) v = *reinterpret_cast<const half8_t *>(src);
            *reinterpret_cast<half8_t *>(as + row * PITCH + sg * 8) = v;
        } else {
            float f[8];
            load_x8(src, row < p.m, f);
            if constexpr (MODE == kA8) {
                // the row's block quantised once per workgroup (4 consecutive threads hold it)
                float dx;
                const uint64_t qa = quant_block8<1, 2>(f, dx);
                *reinterpret_cast<uint64_t *>(smem + row * PITCH8 + sg * 8) = qa;
                if ((sg & 3) == 0) scale[(sg >> 2) * (MB * 16) + row] = dx;
            } else {
                half8_t hi, lo;
                float inv;
                split_block8<1, 2>(f, hi, lo, inv);
                *reinterpret_cast<half8_t *>(as + row * PITCH + sg * 8) = hi;
                *reinterpret_cast<half8_t *>(as_lo + row * PITCH + sg * 8) = lo;
                if ((sg & 3) == 0) scale[(sg >> 2) * (MB * 16) + row] = inv;
            }
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
            if constexpr (MODE == kA8) {
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
            } else if constexpr (MODE == kA16) {
                const half8_t xv = *reinterpret_cast<const half8_t *>(as + (mb * 16 + r) * PITCH + b * 32 + g * 8);
                const float4v pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, widen_w8(q8[b]), float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mb][i] += pr[i] * dw[b];
            } else {
                const half8_t xh = *reinterpret_cast<const half8_t *>(as + (mb * 16 + r) * PITCH + b * 32 + g * 8);
                const half8_t xl = *reinterpret_cast<const half8_t *>(as_lo + (mb * 16 + r) * PITCH + b * 32 + g * 8);
                const half8_t wv = widen_w8(q8[b]);
                float4v pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, wv, float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, wv, pr, 0, 0, 0);
                const float4v inv = *reinterpret_cast<const float4v *>(scale + b * (MB * 16) + mb * 16 + g * 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mb][i] += (pr[i] * dw[b]) * inv[i];
            }
        }
        if constexpr (MB >= 2) {
            // fold each block's products into the accumulators before the next block's MFMAs
            // issue: left to itself the compiler issues all NB * MB block products first and holds
            // their results (~480 registers at MB = 3, NB = 16: one wave per SIMD; 84 this way, and
            // the gate|up projection at the talker's shape 30.3 -> 21.4 us). At MB = 1 the
            // overlap is worth more than the occupancy.
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) asm volatile("" : "+v"(acc[mb]));
            __builtin_amdgcn_sched_barrier(0);
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
        // the first eight ranges' partials requested together, summed in range order
        float w[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
            if (q < ranges) w[q] = part[q * mn + e];
        float s = w[0];
#pragma unroll
        for (int q = 1; q < 8; ++q)
            if (q < ranges) s += w[q];
        for (int q = 8; q < ranges; ++q) s += part[q * mn + e];
        y[e] = s;
    }
}

// Blocks per k range for the A-sharing kernel: the widest range that still gives >= 192
// workgroups and keeps the f16 slab within 64 KB of LDS (else the narrowest); 0 when the shape
// does not fit it. W8A32 above 16 rows takes eight-block ranges: its two f16 slabs then leave room
// for three workgroups per CU (52 KB at 48 rows, against 103 KB and one at sixteen blocks; the
// gate|up projection at the talker's shape 41.6 -> 29.7 us), where the other modes measured
// faster with the wider ranges.
int pick_q8_nb(int64_t m, int64_t k, int64_t n, int32_t mode) {
    const int64_t nblocks = k / 32, tiles = n / 64, rows = (m + 15) / 16 * 16;
    if (m <= 0 || m > 64 || n % 64 != 0 || nblocks % 8 != 0 || tiles >= 65536) return 0;
    if (mode == DTTS_Q8_W8A32 && m > 16) return 8;
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

namespace dtts {
namespace {

const char *mode_name(int32_t mode) {
    return mode == DTTS_Q8_W8A16 ? "W8A16" : mode == DTTS_Q8_W8A8 ? "W8A8" : mode == DTTS_Q8_W8A32 ? "W8A32" : "?";
}

// The modes each activation type takes: f16 x runs W8A16 (its product is exact already) or W8A8;
// f32 x runs W8A8 (quantized from f32 directly) or W8A32.
template <typename XT>
bool mode_ok(int32_t mode) {
    if (sizeof(XT) == 2) return mode == DTTS_Q8_W8A16 || mode == DTTS_Q8_W8A8;
    return mode == DTTS_Q8_W8A8 || mode == DTTS_Q8_W8A32;
}

template <int MB, int NBW, int MODE, typename XT>
void q8_row_kernel(bool packed, unsigned grid, unsigned threads, size_t lds, hipStream_t stream, const Q8Params<XT> &p) {
    if (packed)
        gemm_q8_row<MB, NBW, MODE, true, XT><<<grid, threads, lds, stream>>>(p);
    else
        gemm_q8_row<MB, NBW, MODE, false, XT><<<grid, threads, lds, stream>>>(p);
}

// W8A16 for f16 activations, W8A32 for f32 ones: the modes q8_row_wins takes.
template <int MB, int NBW, typename XT>
void q8_row_modes(bool packed, unsigned grid, unsigned threads, size_t lds, hipStream_t stream, const Q8Params<XT> &p) {
    q8_row_kernel<MB, NBW, sizeof(XT) == 2 ? kA16 : kA32, XT>(packed, grid, threads, lds, stream, p);
}

// gemm_q8_row over (m, k, n) with pick_q8_row's nbw, in the mode q8_row_wins takes for XT (the
// caller checked shape, mode and pointers).
template <typename XT>
int q8_row_launch(const char *name, const XT *x, const void *w, float *y, int64_t m, int64_t k, int64_t n,
                  int nbw, bool packed, hipStream_t stream) {
    DTTS_REQUIRE(k < (int64_t(1) << 30) && n < (int64_t(1) << 30), "%s: shape too large", name);
    Q8Params<XT> p{};
    p.x = x;
    p.w = static_cast<const uint8_t *>(w);
    p.y = y;
    p.m = static_cast<int>(m);
    p.k = static_cast<int>(k);
    p.n = static_cast<int>(n);
    const int mb = static_cast<int>((m + 15) / 16);
    const int nw = static_cast<int>(k / 32 / nbw);
    const unsigned grid = static_cast<unsigned>(n / 16), threads = static_cast<unsigned>(64 * nw);
    const size_t lds = static_cast<size_t>(nw) * mb * 64 * sizeof(float4v);
    auto launch = [&](auto mbc) {
        constexpr int MB = decltype(mbc)::value;
        // the blocks per wave q8_row_instantiated lists for MB
        if constexpr (MB == 1) {
            if (nbw == 12) return q8_row_modes<MB, 12, XT>(packed, grid, threads, lds, stream, p);
            if (nbw == 8) return q8_row_modes<MB, 8, XT>(packed, grid, threads, lds, stream, p);
        }
        if constexpr (MB <= 2)
            if (nbw == 6) return q8_row_modes<MB, 6, XT>(packed, grid, threads, lds, stream, p);
        q8_row_modes<MB, 4, XT>(packed, grid, threads, lds, stream, p);
    };
    DTTS_REQUIRE(q8_row_instantiated(mb, nbw), "%s: no one-launch kernel for %d blocks per wave at %d row blocks", name,
                 nbw, mb);
    switch (mb) {
        case 1: launch(std::integral_constant<int, 1>{}); break;
        case 2: launch(std::integral_constant<int, 2>{}); break;
        case 3: launch(std::integral_constant<int, 3>{}); break;
        default: launch(std::integral_constant<int, 4>{}); break;
    }
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

template <typename XT>
int q8_plain(const char *name, const XT *x, const void *blocks, float *y, int64_t m, int64_t k, int64_t n,
             int32_t mode, hipStream_t stream) {
    DTTS_REQUIRE(m >= 0 && k > 0 && n > 0 && k % 32 == 0, "%s: bad shape (%lld, %lld, %lld)", name, (long long)m,
                 (long long)k, (long long)n);
    DTTS_REQUIRE(mode_ok<XT>(mode), "%s: mode %d (%s) not taken with %s activations", name, mode, mode_name(mode),
                 sizeof(XT) == 2 ? "f16" : "f32");
    if (m == 0) return DTTS_OK;
    DTTS_REQUIRE(x && blocks && y, "%s: null pointer", name);
    DTTS_REQUIRE(m <= 64, "%s: m = %lld > 64 (decode shapes only)", name, (long long)m);
    DTTS_REQUIRE(n % 16 == 0, "%s: n = %lld not a multiple of 16", name, (long long)n);
    DTTS_REQUIRE(aligned(x, 16) && aligned(blocks, 2), "%s: x must be 16-byte aligned", name);
    DTTS_REQUIRE(k < (int64_t(1) << 30) && n < (int64_t(1) << 30), "%s: shape too large", name);
    if (const int nbw = pick_q8_row(m, k, n); q8_row_wins(mode, false, nbw, m))
        return q8_row_launch(name, x, blocks, y, m, k, n, nbw, false, stream);
    Q8Params<XT> p{};
    p.x = x;
    p.w = static_cast<const uint8_t *>(blocks);
    p.y = y;
    p.m = static_cast<int>(m);
    p.k = static_cast<int>(k);
    p.n = static_cast<int>(n);
    const int64_t groups = n / 16;
    p.ks = pick_ks_blocks(groups, k / 32);
    p.slab_blocks = static_cast<int>(k / 32 / p.ks);
    const int mb = static_cast<int>((m + 15) / 16);
    const unsigned threads = static_cast<unsigned>(64 * p.ks);
    const size_t lds = static_cast<size_t>(p.ks) * mb * 256 * 4;
    const unsigned grid = static_cast<unsigned>(groups);
    auto launch = [&](auto mbc) {
        constexpr int MB = decltype(mbc)::value;
        if constexpr (sizeof(XT) == 2) {
            if (mode == DTTS_Q8_W8A8)
                gemm_q8_0<MB, kA8, XT><<<grid, threads, lds, stream>>>(p);
            else
                gemm_q8_0<MB, kA16, XT><<<grid, threads, lds, stream>>>(p);
        } else {
            if (mode == DTTS_Q8_W8A8)
                gemm_q8_0<MB, kA8, XT><<<grid, threads, lds, stream>>>(p);
            else
                gemm_q8_0<MB, kA32, XT><<<grid, threads, lds, stream>>>(p);
        }
    };
    switch (mb) {
        case 1: launch(std::integral_constant<int, 1>{}); break;
        case 2: launch(std::integral_constant<int, 2>{}); break;
        case 3: launch(std::integral_constant<int, 3>{}); break;
        default: launch(std::integral_constant<int, 4>{}); break;
    }
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

template <int MB, int NB, int MODE, typename XT>
void q8_lds_kernel(bool packed, dim3 grid, hipStream_t stream, const Q8Params<XT> &p, float *part) {
    // pick_q8_nb keeps the f16 slab within 64 KB: other (MB, NB) pairs are never launched
    if constexpr (q8_lds_bytes(MB, NB, MODE) <= kQ8MaxLds && q8_lds_bytes(MB, NB, kA16) <= 65536) {
        if (packed)
            gemm_q8_lds<MB, NB, MODE, true, XT><<<grid, 256, 0, stream>>>(p, part);
        else
            gemm_q8_lds<MB, NB, MODE, false, XT><<<grid, 256, 0, stream>>>(p, part);
    }
}

template <int MB, int NB, typename XT>
void q8_lds_modes(int32_t mode, bool packed, dim3 grid, hipStream_t stream, const Q8Params<XT> &p, float *part) {
    if (mode == DTTS_Q8_W8A8)
        q8_lds_kernel<MB, NB, kA8, XT>(packed, grid, stream, p, part);
    else if constexpr (sizeof(XT) == 2)
        q8_lds_kernel<MB, NB, kA16, XT>(packed, grid, stream, p, part);
    else
        q8_lds_kernel<MB, NB, kA32, XT>(packed, grid, stream, p, part);
}

template <int MB, typename XT>
void q8_lds_nb(int nb, int32_t mode, bool packed, dim3 grid, hipStream_t stream, const Q8Params<XT> &p, float *part) {
    if (nb == 32)
        q8_lds_modes<MB, 32, XT>(mode, packed, grid, stream, p, part);
    else if (nb == 16)
        q8_lds_modes<MB, 16, XT>(mode, packed, grid, stream, p, part);
    else
        q8_lds_modes<MB, 8, XT>(mode, packed, grid, stream, p, part);
}

// Whether the A-sharing kernel's slab fits the LDS for this (m, nb, mode): pick_q8_nb bounds the
// f16 slab by 64 KB, so W8A16 and W8A8 always fit and W8A32 (two f16 slabs) stays within 134 KB.
bool q8_lds_fits(int64_t m, int nb, int32_t mode) {
    const int mb = static_cast<int>((m + 15) / 16);
    return mb >= 1 && mb <= 4 && q8_lds_bytes(mb, nb, mode) <= kQ8MaxLds;
}

template <typename XT>
int q8_lds_launch(const char *name, const XT *x, const void *w, float *y, int64_t m, int64_t k, int64_t n,
                  int32_t mode, int nb, void *workspace, bool packed, hipStream_t stream, bool merge = true) {
    const int64_t ranges = k / 32 / nb;
    const size_t need = ranges > 1 ? static_cast<size_t>(ranges * m * n) * sizeof(float) : 0;
    DTTS_REQUIRE(k < (int64_t(1) << 30) && n < (int64_t(1) << 30), "%s: shape too large", name);
    DTTS_REQUIRE(q8_lds_fits(m, nb, mode), "%s: no slab layout for m = %lld", name, (long long)m);
    Q8Params<XT> p{};
    p.x = x;
    p.w = static_cast<const uint8_t *>(w);
    p.y = y;
    p.m = static_cast<int>(m);
    p.k = static_cast<int>(k);
    p.n = static_cast<int>(n);
    float *part = need ? static_cast<float *>(workspace) : nullptr;
    const int mb = static_cast<int>((m + 15) / 16);
    const dim3 grid(static_cast<unsigned>(n / 64), static_cast<unsigned>(ranges));
    switch (mb) {
        case 1: q8_lds_nb<1, XT>(nb, mode, packed, grid, stream, p, part); break;
        case 2: q8_lds_nb<2, XT>(nb, mode, packed, grid, stream, p, part); break;
        case 3: q8_lds_nb<3, XT>(nb, mode, packed, grid, stream, p, part); break;
        default: q8_lds_nb<4, XT>(nb, mode, packed, grid, stream, p, part); break;
    }
    DTTS_LAUNCH_CHECK(name);
    if (part && merge) {
        q8_merge<<<grid_for(m * n, 256), 256, 0, stream>>>(part, y, m * n, static_cast<int>(ranges));
        DTTS_LAUNCH_CHECK(name);
    }
    return DTTS_OK;
}

template <typename XT>
int q8_ws(const char *name, const XT *x, const void *blocks, float *y, int64_t m, int64_t k, int64_t n, int32_t mode,
          void *workspace, size_t ws_bytes, hipStream_t stream, const char *plain_name) {
    DTTS_REQUIRE(m >= 0 && k > 0 && n > 0 && k % 32 == 0, "%s: bad shape (%lld, %lld, %lld)", name, (long long)m,
                 (long long)k, (long long)n);
    DTTS_REQUIRE(mode_ok<XT>(mode), "%s: mode %d (%s) not taken with %s activations", name, mode, mode_name(mode),
                 sizeof(XT) == 2 ? "f16" : "f32");
    if (m == 0) return DTTS_OK;
    // Where the one-launch kernel wins, it runs (q8_plain takes it). Otherwise, on the GGML layout
    // the A-sharing kernel pays for its 2-byte weight loads only once a slab serves more than 16 rows
    // (measured at m = 1, 8 and 48); below that, and without room for the ranges, the
    // workspace-free kernel runs.
    const int nb = m > 16 && !q8_row_wins(mode, false, pick_q8_row(m, k, n), m) ? pick_q8_nb(m, k, n, mode) : 0;
    const size_t need = dtts_gemm_q8_0_workspace_bytes(m, k, n);
    if (!nb || (need && (!workspace || ws_bytes < need)))
        return q8_plain(plain_name, x, blocks, y, m, k, n, mode, stream);
    DTTS_REQUIRE(x && blocks && y, "%s: null pointer", name);
    DTTS_REQUIRE(aligned(x, 16) && aligned(blocks, 2) && (!need || aligned(workspace, 16)),
                 "%s: x and the workspace must be 16-byte aligned", name);
    return q8_lds_launch(name, x, blocks, y, m, k, n, mode, nb, workspace, false, stream);
}

template <typename XT>
int q8_packed(const char *name, const XT *x, const void *packed, float *y, int64_t m, int64_t k, int64_t n,
              int32_t mode, void *workspace, size_t ws_bytes, hipStream_t stream) {
    DTTS_REQUIRE(m >= 0 && k > 0 && n > 0 && k % 256 == 0 && n % 64 == 0,
                 "%s: bad shape (%lld, %lld, %lld): k a multiple of 256, n of 64", name, (long long)m, (long long)k,
                 (long long)n);
    DTTS_REQUIRE(mode_ok<XT>(mode), "%s: mode %d (%s) not taken with %s activations", name, mode, mode_name(mode),
                 sizeof(XT) == 2 ? "f16" : "f32");
    if (m == 0) return DTTS_OK;
    DTTS_REQUIRE(m <= 64, "%s: m = %lld > 64 (decode shapes only)", name, (long long)m);
    DTTS_REQUIRE(x && packed && y, "%s: null pointer", name);
    if (const int nbw = pick_q8_row(m, k, n); q8_row_wins(mode, true, nbw, m)) {
        DTTS_REQUIRE(aligned(x, 16) && aligned(packed, 16), "%s: x and packed must be 16-byte aligned", name);
        return q8_row_launch(name, x, packed, y, m, k, n, nbw, true, stream);
    }
    const int nb = pick_q8_nb(m, k, n, mode);
    const size_t need = dtts_gemm_q8_0_workspace_bytes(m, k, n);
    DTTS_REQUIRE(nb > 0, "%s: shape not supported", name);
    DTTS_REQUIRE(!need || (workspace && ws_bytes >= need), "%s: workspace %zu bytes < %zu needed", name, ws_bytes, need);
    DTTS_REQUIRE(aligned(x, 16) && aligned(packed, 16) && (!need || aligned(workspace, 16)),
                 "%s: x, packed and the workspace must be 16-byte aligned", name);
    return q8_lds_launch(name, x, packed, y, m, k, n, mode, nb, workspace, true, stream);
}

}  // namespace

int q8_stack_ranges(int64_t m, int64_t k, int64_t n, int32_t mode) {
    const int nb = pick_q8_nb(m, k, n, mode);
    return nb ? static_cast<int>(k / 32 / nb) : 0;
}

int q8_stack_gemm(const float *x, const void *packed, float *y, float *part, int64_t m, int64_t k, int64_t n,
                  int32_t mode, hipStream_t stream) {
    const char *name = "dtts_stack (Q8_0 projection)";
    const int nb = pick_q8_nb(m, k, n, mode);
    DTTS_REQUIRE(nb > 0 && k % 256 == 0 && m <= 64, "%s: shape (%lld, %lld, %lld) not supported", name, (long long)m,
                 (long long)k, (long long)n);
    DTTS_REQUIRE(k / 32 / nb == 1 || part, "%s: no room for the k ranges", name);
    return q8_lds_launch(name, x, packed, y, m, k, n, mode, nb, part, true, stream, false);
}

}  // namespace dtts

extern "C" int dtts_gemm_q8_0(const dtts_f16 *x, const void *blocks, float *y, int64_t m, int64_t k, int64_t n,
                              int32_t mode, hipStream_t stream) {
    return dtts::q8_plain("dtts_gemm_q8_0", reinterpret_cast<const half_t *>(x), blocks, y, m, k, n, mode, stream);
}

extern "C" int dtts_gemm_q8_0_f32(const float *x, const void *blocks, float *y, int64_t m, int64_t k, int64_t n,
                                  int32_t mode, hipStream_t stream) {
    return dtts::q8_plain("dtts_gemm_q8_0_f32", x, blocks, y, m, k, n, mode, stream);
}

extern "C" size_t dtts_gemm_q8_0_workspace_bytes(int64_t m, int64_t k, int64_t n) {
    if (m <= 0 || k <= 0 || n <= 0 || k % 32 != 0) return 0;
    const int nb = dtts::pick_q8_nb(m, k, n, DTTS_Q8_W8A32);  // the mode with the most ranges
    const int64_t ranges = nb ? k / 32 / nb : 1;
    return ranges > 1 ? static_cast<size_t>(ranges * m * n) * sizeof(float) : 0;
}

extern "C" int dtts_gemm_q8_0_ws(const dtts_f16 *x, const void *blocks, float *y, int64_t m, int64_t k, int64_t n,
                                 int32_t mode, void *workspace, size_t ws_bytes, hipStream_t stream) {
    return dtts::q8_ws("dtts_gemm_q8_0_ws", reinterpret_cast<const half_t *>(x), blocks, y, m, k, n, mode, workspace,
                       ws_bytes, stream, "dtts_gemm_q8_0");
}

extern "C" int dtts_gemm_q8_0_ws_f32(const float *x, const void *blocks, float *y, int64_t m, int64_t k, int64_t n,
                                     int32_t mode, void *workspace, size_t ws_bytes, hipStream_t stream) {
    return dtts::q8_ws("dtts_gemm_q8_0_ws_f32", x, blocks, y, m, k, n, mode, workspace, ws_bytes, stream,
                       "dtts_gemm_q8_0_f32");
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
    return dtts::q8_packed("dtts_gemm_q8_0_packed", reinterpret_cast<const half_t *>(x), packed, y, m, k, n, mode,
                           workspace, ws_bytes, stream);
}

extern "C" int dtts_gemm_q8_0_packed_f32(const float *x, const void *packed, float *y, int64_t m, int64_t k, int64_t n,
                                         int32_t mode, void *workspace, size_t ws_bytes, hipStream_t stream) {
    return dtts::q8_packed("dtts_gemm_q8_0_packed_f32", x, packed, y, m, k, n, mode, workspace, ws_bytes, stream);
}
