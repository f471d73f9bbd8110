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

// Sums the k splits' partials in split order (deterministic), then the mode's store.
template <int MODE>
__global__ __launch_bounds__(256) void gemm_merge_splits(GemmParams p, int ysplit) {
    const int cols = MODE == 1 ? p.n / 2 : p.n;
    const int64_t total = static_cast<int64_t>(p.m) * cols;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t row = e / cols;
        const int col = static_cast<int>(e - row * cols);
        float s0 = 0.f, s1 = 0.f;
        for (int y = 0; y < ysplit; ++y) {
            const float *pr = p.part + (static_cast<int64_t>(y) * p.m + row) * p.n + col;
            s0 += pr[0];
            if constexpr (MODE == 1) s1 += pr[p.n / 2];
        }
        gemm_store<MODE>(p, row, col, s0, s1);
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

size_t nt_workspace_bytes(int64_t m, int64_t k, int64_t n, int mode) {
    if (m <= 0 || m > 64 || k % 64 != 0 || (mode == 1 ? n / 2 : n) % 16 != 0) return 0;
    const int nb = mode == 1 ? 2 : 1;
    const int64_t groups = (mode == 1 ? n / 2 : n) / 16;
    const NtSplit sp = pick_nt_split(groups, nb, k, true);
    return sp.ks > 0 && sp.ysplit > 1 ? static_cast<size_t>(sp.ysplit) * m * n * sizeof(float) : 0;
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
    GemmParams p = p0;
    const int nb = MODE == 1 ? 2 : 1;
    const int64_t groups = MODE == 1 ? p.n / 2 / 16 : p.n / 16;
    const size_t need = nt_workspace_bytes(p.m, p.k, p.n, MODE);
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
    const int64_t outs = int64_t(p.m) * (MODE == 1 ? p.n / 2 : p.n);
    gemm_merge_splits<MODE><<<grid_for(outs, 256, 4), 256, 0, stream>>>(p, sp.ysplit);
    return hipGetLastError();
}

}  // namespace
}  // namespace dtts
