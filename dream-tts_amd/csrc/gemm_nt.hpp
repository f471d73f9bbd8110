// The decode-shape NT projection kernel, shared by the projection entry points and the
// decoder-stack step: C[m, n] = A[m, k] . W^T with m <= 64 lanes, W in the checkpoint layout
// [n, k], f16 operands, f32 accumulation.
//
// Weight streaming is the whole cost (A is 48 rows; W is megabytes), so the kernel is built
// around reading W exactly once with full cache lines and many bytes in flight:
//   * W stays in the checkpoint layout [n, k] (K contiguous), which is what the matrix cores
//     want for the B operand, so fragments load straight from HBM with no LDS staging.
//   * v_mfma_f32_16x16x32_f16: a wave owns 16 output columns and all ceil(m/16) row blocks.
//     Lane group g = lane/16 reads 16 consecutive k (32 bytes) of its row per 64-k chunk, so
//     the four lanes of a row cover a full 128-byte line. The 64 k of a chunk are split over the
//     two MFMAs as {g*16 .. g*16+7} and {g*16+8 .. g*16+15}; A uses the same split, and the
//     dot product is order-free over k, so the permutation is exact.
//   * K is split over the waves of a workgroup (KS slabs); the slab partials are summed through
//     LDS in slab order, so results are deterministic (the reference's ordered sum_splits,
//     crates/tts-nn/src/mtl.rs:1136-1150) and no partials reach HBM.
//   * The gate|up variant computes a gate block and its up block in one workgroup and writes
//     silu(g) * u (SwigluMul fused into the GEMM epilogue), in f32 or rounded to f16 for a
//     consumer that casts it (Proj::forward's x.to_dtype(F16), crates/tts-nn/src/lib.rs:517).
//   * The residual variant adds the product (times an optional per-column scale, LayerScale) to
//     C in place: h = h + attn and h = h + mlp of Stack::forward (crates/qwen3tts/src/qwen3.rs:
//     445-465), the product complete before the add.
#pragma once

#include "common.hpp"

namespace dtts {
namespace {

typedef float float4v __attribute__((ext_vector_type(4)));

struct GemmParams {
    const half_t *a;     // [m, k]
    const half_t *w;     // [n, k] (gate rows then up rows for the gate|up form)
    float *c;            // [m, n] (or [m, n/2] for gate|up); MODE 2 reads and rewrites it
    half_t *c16;         // MODE 1: when set, the [m, n/2] output in f16 instead of c
    const float *scale;  // MODE 2: per-column factor on the product, or null
    float *part;         // [ysplit][m][n] partial sums when k is split across workgroups, else null
    int m, k, n, ks, slab;
};

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// The output of one (row, column): s0 the column's sum (the gate's for MODE 1), s1 the up's.
template <int MODE>
__device__ __forceinline__ void gemm_store(const GemmParams &p, int64_t row, int col, float s0, float s1) {
#pragma clang fp contract(off)  // MODE 2 rounds the scaled product before the add, as the reference does
    if constexpr (MODE == 0) {
        p.c[row * p.n + col] = s0;
    } else if constexpr (MODE == 1) {
        const float y = silu_mul(s0, s1);
        const int64_t o = row * (p.n / 2) + col;
        if (p.c16)
            p.c16[o] = static_cast<half_t>(y);
        else
            p.c[o] = y;
    } else {
        float *d = p.c + row * p.n + col;
        *d = *d + (p.scale ? s0 * p.scale[col] : s0);
    }
}

// MODE 0: plain, NB = 1. MODE 1: gate|up + SiLU*mul, NB = 2 (block 0 gate, block 1 up).
// MODE 2: residual (C += product), NB = 1.
// Workgroup (blockIdx.x, blockIdx.y): column group x, k split y; wave (nb, kslab) reduces the
// slab of NC 64-k chunks starting at ((y * ks + kslab) * slab). All NC chunks of the wave's
// weights are requested before the first MFMA, so a CU has every wave's slab in flight at once
// (the whole matrix is a few MB: latency, not bandwidth per request, is what there is to hide).
template <int MB, int MODE, int NC>
__global__ __launch_bounds__(1024) void gemm_skinny_nt(GemmParams p) {
    extern __shared__ __attribute__((aligned(16))) float red[];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int kslab = wave % p.ks;
    const int nb = wave / p.ks;
    const int g = lane >> 4;
    const int r = lane & 15;
    const int k0 = (blockIdx.y * p.ks + kslab) * p.slab;
    int col;  // W row this lane streams
    if constexpr (MODE != 1) {
        col = blockIdx.x * 16 + r;
    } else {
        col = (nb == 0 ? 0 : p.n / 2) + blockIdx.x * 16 + r;
    }
    const half_t *wr = p.w + static_cast<int64_t>(col) * p.k + k0 + g * 16;
    half8_t b[NC][2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        b[c][0] = *reinterpret_cast<const half8_t *>(wr + c * 64);
        b[c][1] = *reinterpret_cast<const half8_t *>(wr + c * 64 + 8);
    }
    const half_t *ar[MB];
    bool arow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int row = mb * 16 + r;
        arow[mb] = row < p.m;
        ar[mb] = p.a + static_cast<int64_t>(arow[mb] ? row : 0) * p.k + k0 + g * 16;
    }
    // keep every weight load ahead of the first MFMA (the scheduler would otherwise sink them
    // next to their uses, leaving a few requests in flight per wave)
    __builtin_amdgcn_sched_barrier(0);
    float4v acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            half8_t a0 = *reinterpret_cast<const half8_t *>(ar[mb] + c * 64);
            half8_t a1 = *reinterpret_cast<const half8_t *>(ar[mb] + c * 64 + 8);
            if (!arow[mb]) {
                a0 = half8_t{};
                a1 = half8_t{};
            }
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b[c][0], acc[mb], 0, 0, 0);
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b[c][1], acc[mb], 0, 0, 0);
        }
    }

    // slab partials -> LDS [nb][kslab][mb][lane][4]
    float *mine = red + ((static_cast<int64_t>(nb) * p.ks + kslab) * MB) * 256;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
        *reinterpret_cast<float4v *>(mine + mb * 256 + lane * 4) = acc[mb];
    __syncthreads();
    if (kslab != 0 || nb != 0) return;
    // C layout of 16x16: lane holds column r, rows 4*g + i
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        float4v s0 = float4v{0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < p.ks; ++s) s0 += *reinterpret_cast<const float4v *>(red + ((0 * p.ks + s) * MB + mb) * 256 + lane * 4);
        float4v s1 = float4v{0.f, 0.f, 0.f, 0.f};
        if constexpr (MODE == 1)
            for (int s = 0; s < p.ks; ++s)
                s1 += *reinterpret_cast<const float4v *>(red + ((1 * p.ks + s) * MB + mb) * 256 + lane * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mb * 16 + g * 4 + i;
            if (row >= p.m) continue;
            if (p.part) {  // this k split's sums; the merge kernel finishes the output
                float *pr = p.part + (static_cast<int64_t>(blockIdx.y) * p.m + row) * p.n + blockIdx.x * 16 + r;
                pr[0] = s0[i];
                if constexpr (MODE == 1) pr[p.n / 2] = s1[i];
            } else {
                gemm_store<MODE>(p, row, blockIdx.x * 16 + r, s0[i], s1[i]);
            }
        }
    }
}

// Sums the k splits' partials in split order (deterministic), then the mode's store; four
// output columns per thread (every caller has output widths that are multiples of 16).
template <int MODE>
__global__ __launch_bounds__(256) void gemm_merge_splits(GemmParams p, int ysplit) {
    const int c4n = (MODE == 1 ? p.n / 2 : p.n) / 4;
    const int64_t total = static_cast<int64_t>(p.m) * c4n;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t row = e / c4n;
        const int col = static_cast<int>(e - row * c4n) * 4;
        const float *pr = p.part + row * p.n + col;
        const int64_t stride = static_cast<int64_t>(p.m) * p.n;
        const float4v s0 = ordered_sum4<8, true>(pr, ysplit, stride);
        float4v s1 = float4v{0.f, 0.f, 0.f, 0.f};
        if constexpr (MODE == 1) s1 = ordered_sum4<8, true>(pr + p.n / 2, ysplit, stride);
#pragma unroll
        for (int i = 0; i < 4; ++i) gemm_store<MODE>(p, row, col + i, s0[i], s1[i]);
    }
}

// How the NT kernel splits k: ks waves per workgroup (nb * ks <= 16) times ysplit workgroups per
// column group, each wave NC = k / 64 / (ks * ysplit) chunks (1..8). The aim is ~2048 waves
// (eight per CU) with as few workgroup splits as reach it; ysplit > 1 needs the partial buffer.
struct NtSplit {
    int ks, ysplit, nc;
};

NtSplit pick_nt_split(int64_t groups, int nb, int64_t k, bool can_split) {
    const int64_t chunks = k / 64;
    NtSplit most{0, 0, 0};
    int64_t most_waves = 0;
    for (int ysplit = 1; ysplit <= (can_split ? 8 : 1); ++ysplit)
        for (int ks = 1; ks * nb <= 16; ++ks) {
            if (chunks % (int64_t(ks) * ysplit) != 0) continue;
            const int64_t nc = chunks / (int64_t(ks) * ysplit);
            if (nc > 8) continue;
            const int64_t waves = groups * nb * ks * ysplit;
            if (waves >= 2048) return NtSplit{ks, ysplit, static_cast<int>(nc)};  // fewest splits that fill
            if (waves > most_waves) {
                most = NtSplit{ks, ysplit, static_cast<int>(nc)};
                most_waves = waves;
            }
        }
    return most;
}

// ---------------------------------------------------------------- one launch, k over the waves
//
// For the per-op entry points at short k (k * ceil(m/16) <= 3072): workgroup x owns 16 output
// columns (16 gate and the matching 16 up rows for gate|up) and all of k; wave w takes the slab
// [w * NCW * 64, (w + 1) * NCW * 64). Every lane requests its weight and A fragments for the
// whole slab before the first MFMA (the per-wave kernel above requests A inside its MFMA loop,
// where the compiler puts a wait before each use: one memory round trip per chunk). The slab
// partials meet in LDS and are summed in wave order, so the output is complete in one launch,
// with no workspace and no merge. Past that k the A fragments each workgroup reads (48 rows x k)
// outweigh the 16 weight rows it streams, and the A-sharing kernel with its range merge is the
// faster of the two (measured at the talker's and config 3's shapes, 8 and 48 rows).
template <int MB, int NCW, int MODE>
__global__ __launch_bounds__(1024) void gemm_row_nt(GemmParams p) {
    constexpr int NB = MODE == 1 ? 2 : 1;
    extern __shared__ __attribute__((aligned(16))) float4v rsum[];  // [NB][waves][MB][64]
    const int nw = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g = lane >> 4, r = lane & 15;
    const int k0 = wave * NCW * 64 + g * 16;
    const int col = blockIdx.x * 16 + r;
    half8_t b[NB][NCW][2];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const half_t *wr = p.w + static_cast<int64_t>(nb == 0 ? col : p.n / 2 + col) * p.k + k0;
#pragma unroll
        for (int c = 0; c < NCW; ++c) {
            b[nb][c][0] = *reinterpret_cast<const half8_t *>(wr + c * 64);
            b[nb][c][1] = *reinterpret_cast<const half8_t *>(wr + c * 64 + 8);
        }
    }
    half8_t av[MB][NCW][2];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int row = mb * 16 + r;
        const half_t *ar = p.a + static_cast<int64_t>(row < p.m ? row : 0) * p.k + k0;
#pragma unroll
        for (int c = 0; c < NCW; ++c) {
            av[mb][c][0] = *reinterpret_cast<const half8_t *>(ar + c * 64);
            av[mb][c][1] = *reinterpret_cast<const half8_t *>(ar + c * 64 + 8);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is in flight before the first wait
    float4v acc[NB][MB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[nb][mb] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NCW; ++c)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const bool live = mb * 16 + r < p.m;  // rows past m multiply zeros
            const half8_t a0 = live ? av[mb][c][0] : half8_t{};
            const half8_t a1 = live ? av[mb][c][1] : half8_t{};
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b[nb][c][0], acc[nb][mb], 0, 0, 0);
                acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b[nb][c][1], acc[nb][mb], 0, 0, 0);
            }
        }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) rsum[((nb * nw + wave) * MB + mb) * 64 + lane] = acc[nb][mb];
    __syncthreads();
    // C layout of 16x16: lane l holds column l & 15, rows 4 * (l >> 4) + i
    for (int t = threadIdx.x; t < MB * 64; t += blockDim.x) {
        const int mb = t >> 6, l = t & 63;
        float4v s0 = rsum[mb * 64 + l];
        for (int q = 1; q < nw; ++q) s0 += rsum[(q * MB + mb) * 64 + l];
        float4v s1 = float4v{0.f, 0.f, 0.f, 0.f};
        if constexpr (MODE == 1) {
            s1 = rsum[(nw * MB + mb) * 64 + l];
            for (int q = 1; q < nw; ++q) s1 += rsum[((nw + q) * MB + mb) * 64 + l];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mb * 16 + (l >> 4) * 4 + i;
            if (row < p.m) gemm_store<MODE>(p, row, blockIdx.x * 16 + (l & 15), s0[i], s1[i]);
        }
    }
}

// Chunks of 64 k per wave for gemm_row_nt (0: not applicable): 2, or 3 for one row block when
// two would need more than 16 waves or do not divide k; m <= 64 and k * ceil(m/16) <= 3072.
// launch_row_mb instantiates three chunks per wave for one row block only.
inline int pick_row(int64_t m, int64_t k, int64_t cols) {
    if (m <= 0 || m > 64 || cols % 16 != 0 || cols / 16 >= 65536) return 0;
    const int64_t mb = (m + 15) / 16;
    if (k * mb > 3072) return 0;
    if (k % 128 == 0 && k / 128 <= 16) return 2;
    if (mb == 1 && k % 192 == 0 && k / 192 <= 16) return 3;
    return 0;
}

template <int MODE, int NCW>
hipError_t launch_row_mb(const GemmParams &p, hipStream_t stream) {
    const int nw = p.k / (NCW * 64);
    const int mb = (p.m + 15) / 16;
    const size_t lds = static_cast<size_t>(MODE == 1 ? 2 : 1) * nw * mb * 64 * sizeof(float4v);
    const dim3 grid(static_cast<unsigned>((MODE == 1 ? p.n / 2 : p.n) / 16));
    const dim3 block(static_cast<unsigned>(nw * 64));
    if constexpr (NCW == 3) {  // pick_row takes three chunks per wave for one row block only
        if (mb != 1) return hipErrorInvalidValue;
        gemm_row_nt<1, NCW, MODE><<<grid, block, lds, stream>>>(p);
    } else {
        switch (mb) {
            case 1: gemm_row_nt<1, NCW, MODE><<<grid, block, lds, stream>>>(p); break;
            case 2: gemm_row_nt<2, NCW, MODE><<<grid, block, lds, stream>>>(p); break;
            case 3: gemm_row_nt<3, NCW, MODE><<<grid, block, lds, stream>>>(p); break;
            default: gemm_row_nt<4, NCW, MODE><<<grid, block, lds, stream>>>(p); break;
        }
    }
    return hipGetLastError();
}

template <int MODE>
hipError_t launch_row(const GemmParams &p, int ncw, hipStream_t stream) {
    return ncw == 3 ? launch_row_mb<MODE, 3>(p, stream) : launch_row_mb<MODE, 2>(p, stream);
}

// ---------------------------------------------------------------- the A-sharing kernel
//
// Workgroup (x, y) = 4 waves: 64 weight rows (output columns; for gate|up, 32 gate rows and the
// matching 32 up rows) times the k range [y * KR, (y + 1) * KR), KR = NC * 64. The activation
// slab A[0:m, k range] is read once per workgroup with coalesced 16-byte loads and kept in LDS,
// where all four waves read their fragments: per workgroup A costs m/64 of the weight bytes
// instead of m/16 when every wave fetches its own. Each wave holds its 16 weight rows x KR in
// registers, every load issued before the first MFMA. With one k range the workgroup applies
// the epilogue; with several (gridDim.y > 1) it writes its partial tile to p.part
// [gridDim.y][m][n] and the ranges are summed in order afterwards, by gemm_merge_splits or by
// the consuming kernel.
constexpr int kLdsMaxTiles = 1 << 16;

template <int MB, int NC, int MODE>
__global__ __launch_bounds__(256) void gemm_lds_nt(GemmParams p) {
    constexpr int KR = NC * 64;
    constexpr int PITCH = KR + 8;  // halves; 16 bytes of padding spread the fragment reads over banks
    constexpr int TP = 64 + 4;     // f32 pitch of the 64-column tile
    extern __shared__ __attribute__((aligned(16))) half_t als[];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int g = lane >> 4, r = lane & 15;
    const int kb = blockIdx.y * KR;
    // A slab: MB*16 rows x KR/8 16-byte segments over 256 threads (rows >= m are zero)
    constexpr int SEGS = MB * 16 * (KR / 8);
    constexpr int APT = SEGS / 256;
    static_assert(SEGS % 256 == 0, "slab segments");
    half8_t av[APT];
#pragma unroll
    for (int i = 0; i < APT; ++i) {
        const int sg = t + i * 256;
        const int row = sg / (KR / 8), seg = sg % (KR / 8);
        av[i] = row < p.m ? *reinterpret_cast<const half8_t *>(p.a + static_cast<int64_t>(row) * p.k + kb + seg * 8)
                          : half8_t{};
    }
    int wrow;  // the weight row this lane streams
    if constexpr (MODE == 1)
        wrow = (wave < 2 ? 0 : p.n / 2) + blockIdx.x * 32 + (wave & 1) * 16 + r;
    else
        wrow = blockIdx.x * 64 + wave * 16 + r;
    const half_t *wr = p.w + static_cast<int64_t>(wrow) * p.k + kb + g * 16;
    half8_t b[NC][2];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        b[c][0] = *reinterpret_cast<const half8_t *>(wr + c * 64);
        b[c][1] = *reinterpret_cast<const half8_t *>(wr + c * 64 + 8);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is in flight before the first wait
#pragma unroll
    for (int i = 0; i < APT; ++i) {
        const int sg = t + i * 256;
        const int row = sg / (KR / 8), seg = sg % (KR / 8);
        *reinterpret_cast<half8_t *>(als + row * PITCH + seg * 8) = av[i];
    }
    __syncthreads();
    float4v acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = float4v{0.f, 0.f, 0.f, 0.f};
    const half_t *ab = als + r * PITCH + g * 16;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const half8_t a0 = *reinterpret_cast<const half8_t *>(ab + mb * 16 * PITCH + c * 64);
            const half8_t a1 = *reinterpret_cast<const half8_t *>(ab + mb * 16 * PITCH + c * 64 + 8);
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b[c][0], acc[mb], 0, 0, 0);
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b[c][1], acc[mb], 0, 0, 0);
        }
    // the 64-column tile, f32, through LDS (the slab is no longer read)
    __syncthreads();
    float *tile = reinterpret_cast<float *>(als);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) tile[(mb * 16 + g * 4 + i) * TP + wave * 16 + r] = acc[mb][i];
    __syncthreads();
    // tile column tc -> output column: gate|up tiles hold gate columns 0..31 then up columns
    auto gcol = [&](int tc) {
        if constexpr (MODE == 1) return (tc < 32 ? 0 : p.n / 2) + blockIdx.x * 32 + (tc & 31);
        return blockIdx.x * 64 + tc;
    };
    constexpr int OUTC = MODE == 1 ? 32 : 64;  // output columns of the tile
    if (gridDim.y > 1) {  // this range's partial tile, 4 columns per thread
        for (int e = t; e < p.m * 16; e += 256) {
            const int row = e >> 4, c4 = (e & 15) * 4;
            *reinterpret_cast<float4v *>(p.part + (static_cast<int64_t>(blockIdx.y) * p.m + row) * p.n + gcol(c4)) =
                *reinterpret_cast<const float4v *>(tile + row * TP + c4);
        }
        return;
    }
    for (int e = t; e < p.m * OUTC; e += 256) {
        const int row = e / OUTC, oc = e - (e / OUTC) * OUTC;
        const float s0 = tile[row * TP + oc];
        const float s1 = MODE == 1 ? tile[row * TP + oc + 32] : 0.f;
        gemm_store<MODE>(p, row, MODE == 1 ? blockIdx.x * 32 + oc : gcol(oc), s0, s1);
    }
}

// The A-sharing kernel's plan: NC chunks of 64 k per workgroup (8 when that still gives ~192
// workgroups or more, else 4; 2 when k is an odd multiple of 128), ys = k / (NC * 64) ranges.
// Needs m <= 64, k % 128 == 0 and 64 output columns per tile (32 for gate|up). nc == 0: not
// applicable.
struct LdsPlan {
    int nc, ys, tiles;
};

// max_m: callers other than the decode step (the stack's prefill) may pass up to 128 rows; past 64
// the range is four chunks up to 96 rows and two past that (the slab then stays within 51 KB of
// LDS).
inline LdsPlan pick_lds(int64_t m, int64_t k, int64_t n, int mode, int64_t max_m = 64) {
    const int64_t per = mode == 1 ? 32 : 64;
    const int64_t cols = mode == 1 ? n / 2 : n;
    if (m <= 0 || m > max_m || m > 128 || k % 128 != 0 || cols % per != 0 || cols / per > kLdsMaxTiles)
        return LdsPlan{0, 0, 0};
    const int64_t tiles = cols / per;
    const int nc = (k % 256 != 0 || m > 96) ? 2 : m > 64 ? 4 : (k % 512 == 0 && tiles * (k / 512) >= 192) ? 8 : 4;
    return LdsPlan{nc, static_cast<int>(k / (nc * 64)), static_cast<int>(tiles)};
}

inline size_t lds_partial_bytes(const LdsPlan &pl, int64_t m, int64_t n) {
    return pl.nc > 0 && pl.ys > 1 ? static_cast<size_t>(pl.ys) * m * n * sizeof(float) : 0;
}

// merge == false leaves the partial tiles for the consumer to sum (the stack step does).
template <int MODE>
hipError_t launch_lds_nt(const GemmParams &p0, const LdsPlan &pl, void *workspace, hipStream_t stream,
                         bool merge = true) {
    GemmParams p = p0;
    p.part = pl.ys > 1 ? static_cast<float *>(workspace) : nullptr;
    const int mb = (p.m + 15) / 16;
    const size_t slab = static_cast<size_t>(mb) * 16 * (pl.nc * 64 + 8) * 2;
    const size_t tile = static_cast<size_t>(mb) * 16 * 68 * 4;
    const size_t lds = slab > tile ? slab : tile;
    const dim3 grid(static_cast<unsigned>(pl.tiles), static_cast<unsigned>(pl.ys));
#define DTTS_LDS_NT(MB_)                                                                         \
    if (pl.nc == 8)                                                                               \
        gemm_lds_nt<MB_, 8, MODE><<<grid, 256, lds, stream>>>(p);                                 \
    else if (pl.nc == 4)                                                                          \
        gemm_lds_nt<MB_, 4, MODE><<<grid, 256, lds, stream>>>(p);                                 \
    else                                                                                          \
        gemm_lds_nt<MB_, 2, MODE><<<grid, 256, lds, stream>>>(p);
    switch (mb) {
        case 1: DTTS_LDS_NT(1) break;
        case 2: DTTS_LDS_NT(2) break;
        case 3: DTTS_LDS_NT(3) break;
        case 4: DTTS_LDS_NT(4) break;
        // more than 64 rows: four-chunk ranges up to 96 rows, two-chunk past that (pick_lds)
        case 5:
            if (pl.nc == 4)
                gemm_lds_nt<5, 4, MODE><<<grid, 256, lds, stream>>>(p);
            else
                gemm_lds_nt<5, 2, MODE><<<grid, 256, lds, stream>>>(p);
            break;
        case 6:
            if (pl.nc == 4)
                gemm_lds_nt<6, 4, MODE><<<grid, 256, lds, stream>>>(p);
            else
                gemm_lds_nt<6, 2, MODE><<<grid, 256, lds, stream>>>(p);
            break;
        case 7: gemm_lds_nt<7, 2, MODE><<<grid, 256, lds, stream>>>(p); break;
        default: gemm_lds_nt<8, 2, MODE><<<grid, 256, lds, stream>>>(p); break;
    }
#undef DTTS_LDS_NT
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || pl.ys == 1 || !merge) return e;
    const int64_t outs = int64_t(p.m) * (MODE == 1 ? p.n / 2 : p.n) / 4;
    gemm_merge_splits<MODE><<<grid_for(outs, 256, 4), 256, 0, stream>>>(p, pl.ys);
    return hipGetLastError();
}

// Workspace for a projection: the A-sharing kernel's partial tiles when it applies, else the
// per-wave kernel's split partials.
inline size_t wave_kernel_workspace_bytes(int64_t m, int64_t k, int64_t n, int mode) {
    if (m <= 0 || m > 64 || k % 64 != 0 || (mode == 1 ? n / 2 : n) % 16 != 0) return 0;
    const int nb = mode == 1 ? 2 : 1;
    const int64_t groups = (mode == 1 ? n / 2 : n) / 16;
    const NtSplit sp = pick_nt_split(groups, nb, k, true);
    return sp.ks > 0 && sp.ysplit > 1 ? static_cast<size_t>(sp.ysplit) * m * n * sizeof(float) : 0;
}

size_t nt_workspace_bytes(int64_t m, int64_t k, int64_t n, int mode) {
    if (pick_row(m, k, mode == 1 ? n / 2 : n) > 0) return 0;
    const LdsPlan pl = pick_lds(m, k, n, mode);
    if (pl.nc > 0) return lds_partial_bytes(pl, m, n);
    return wave_kernel_workspace_bytes(m, k, n, mode);
}

template <int MB, int MODE>
hipError_t launch_nt_mb(const GemmParams &p, dim3 grid, unsigned threads, size_t lds, int nc, hipStream_t stream) {
    switch (nc) {
        case 1: gemm_skinny_nt<MB, MODE, 1><<<grid, threads, lds, stream>>>(p); break;
        case 2: gemm_skinny_nt<MB, MODE, 2><<<grid, threads, lds, stream>>>(p); break;
        case 3: gemm_skinny_nt<MB, MODE, 3><<<grid, threads, lds, stream>>>(p); break;
        case 4: gemm_skinny_nt<MB, MODE, 4><<<grid, threads, lds, stream>>>(p); break;
        case 5: gemm_skinny_nt<MB, MODE, 5><<<grid, threads, lds, stream>>>(p); break;
        case 6: gemm_skinny_nt<MB, MODE, 6><<<grid, threads, lds, stream>>>(p); break;
        case 7: gemm_skinny_nt<MB, MODE, 7><<<grid, threads, lds, stream>>>(p); break;
        default: gemm_skinny_nt<MB, MODE, 8><<<grid, threads, lds, stream>>>(p); break;
    }
    return hipGetLastError();
}

template <int MODE>
hipError_t launch_nt(const GemmParams &p0, int mb_blocks, void *workspace, size_t ws_bytes, hipStream_t stream) {
    const int ncw = pick_row(p0.m, p0.k, MODE == 1 ? p0.n / 2 : p0.n);
    if (ncw > 0 && aligned(p0.a, 16) && aligned(p0.w, 16)) return launch_row<MODE>(p0, ncw, stream);
    const LdsPlan pl = pick_lds(p0.m, p0.k, p0.n, MODE);
    if (pl.nc > 0) {
        const size_t need = lds_partial_bytes(pl, p0.m, p0.n);
        if (need == 0 || (workspace && ws_bytes >= need && aligned(workspace, 16)))
            return launch_lds_nt<MODE>(p0, pl, workspace, stream);
    }
    GemmParams p = p0;
    const int nb = MODE == 1 ? 2 : 1;
    const int64_t groups = MODE == 1 ? p.n / 2 / 16 : p.n / 16;
    const size_t need = wave_kernel_workspace_bytes(p.m, p.k, p.n, MODE);
    const bool split_ok = need > 0 && workspace && ws_bytes >= need && aligned(workspace, 16);
    const NtSplit sp = pick_nt_split(groups, nb, p.k, split_ok);
    p.ks = sp.ks;
    p.slab = sp.nc * 64;
    p.part = sp.ysplit > 1 ? static_cast<float *>(workspace) : nullptr;
    const unsigned threads = static_cast<unsigned>(64 * p.ks * nb);
    const size_t lds = static_cast<size_t>(nb) * p.ks * mb_blocks * 256 * 4;
    const dim3 grid(static_cast<unsigned>(groups), static_cast<unsigned>(sp.ysplit));
    hipError_t e;
    switch (mb_blocks) {
        case 1: e = launch_nt_mb<1, MODE>(p, grid, threads, lds, sp.nc, stream); break;
        case 2: e = launch_nt_mb<2, MODE>(p, grid, threads, lds, sp.nc, stream); break;
        case 3: e = launch_nt_mb<3, MODE>(p, grid, threads, lds, sp.nc, stream); break;
        default: e = launch_nt_mb<4, MODE>(p, grid, threads, lds, sp.nc, stream); break;
    }
    if (e != hipSuccess || !p.part) return e;
    const int64_t outs = int64_t(p.m) * (MODE == 1 ? p.n / 2 : p.n) / 4;
    gemm_merge_splits<MODE><<<grid_for(outs, 256, 4), 256, 0, stream>>>(p, sp.ysplit);
    return hipGetLastError();
}

}  // namespace
}  // namespace dtts
