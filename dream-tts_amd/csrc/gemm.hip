// Decode-shape projection GEMMs: C[m, n] = A[m, k] . W^T with m <= 64 lanes, f16 operands,
// f32 accumulation and output.
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
//     silu(g) * u (SwigluMul fused into the GEMM epilogue).
#include "common.hpp"

namespace dtts {
namespace {

typedef float float4v __attribute__((ext_vector_type(4)));

struct GemmParams {
    const half_t *a;  // [m, k]
    const half_t *w;  // [n, k] (gate rows then up rows for the gate|up form)
    float *c;         // [m, n] (or [m, n/2] for gate|up)
    float *part;      // [ysplit][m][n] partial sums when k is split across workgroups, else null
    int m, k, n, ks, slab;
};

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// MODE 0: plain, NB = 1. MODE 1: gate|up + SiLU*mul, NB = 2 (block 0 gate, block 1 up).
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
    if constexpr (MODE == 0) {
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
            } else if constexpr (MODE == 0) {
                p.c[static_cast<int64_t>(row) * p.n + blockIdx.x * 16 + r] = s0[i];
            } else {
                p.c[static_cast<int64_t>(row) * (p.n / 2) + blockIdx.x * 16 + r] = silu_mul(s0[i], s1[i]);
            }
        }
    }
}

// Sums the k splits' partials in split order (deterministic), then the plain store or SiLU*mul.
template <int MODE>
__global__ __launch_bounds__(256) void gemm_merge_splits(const float *part, float *c, int m, int n, int ysplit) {
    const int cols = MODE == 1 ? n / 2 : n;
    const int64_t total = static_cast<int64_t>(m) * cols;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t row = e / cols, col = e - (e / cols) * cols;
        float s0 = 0.f, s1 = 0.f;
        for (int y = 0; y < ysplit; ++y) {
            const float *pr = part + (static_cast<int64_t>(y) * m + row) * n + col;
            s0 += pr[0];
            if constexpr (MODE == 1) s1 += pr[n / 2];
        }
        c[e] = MODE == 1 ? silu_mul(s0, s1) : s0;
    }
}

// The reference's own operand layout W[k, n] (skinny::matmul's b, crates/tts-nn/src/skinny.rs:
// 155-165): each wave turns its 64 x 16 slice of W into the [n, k] fragment layout through its
// own LDS tile, then proceeds as above.
template <int MB>
__global__ __launch_bounds__(1024) void gemm_skinny_kn(GemmParams p) {
    extern __shared__ __attribute__((aligned(16))) float red[];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int kslab = wave;
    const int g = lane >> 4;
    const int r = lane & 15;
    half_t *tile = reinterpret_cast<half_t *>(red + static_cast<int64_t>(p.ks) * MB * 256) + wave * (16 * 72);
    const int n0 = blockIdx.x * 16;
    const half_t *ar[MB];
    bool arow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int row = mb * 16 + r;
        arow[mb] = row < p.m;
        ar[mb] = p.a + static_cast<int64_t>(arow[mb] ? row : 0) * p.k + kslab * p.slab + g * 16;
    }
    float4v acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = float4v{0.f, 0.f, 0.f, 0.f};
    for (int kc = 0; kc < p.slab; kc += 64) {
        // lane l reads row k = kslab*slab + kc + l, columns n0 .. n0+15 (32 bytes)
        const half_t *src = p.w + static_cast<int64_t>(kslab * p.slab + kc + lane) * p.n + n0;
        const half8_t lo = *reinterpret_cast<const half8_t *>(src);
        const half8_t hi = *reinterpret_cast<const half8_t *>(src + 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            tile[j * 72 + lane] = lo[j];
            tile[(j + 8) * 72 + lane] = hi[j];
        }
        __syncthreads();
        const half8_t b0 = *reinterpret_cast<const half8_t *>(tile + r * 72 + g * 16);
        const half8_t b1 = *reinterpret_cast<const half8_t *>(tile + r * 72 + g * 16 + 8);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            half8_t a0 = *reinterpret_cast<const half8_t *>(ar[mb] + kc);
            half8_t a1 = *reinterpret_cast<const half8_t *>(ar[mb] + kc + 8);
            if (!arow[mb]) {
                a0 = half8_t{};
                a1 = half8_t{};
            }
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, acc[mb], 0, 0, 0);
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, acc[mb], 0, 0, 0);
        }
        __syncthreads();
    }
    float *mine = red + (static_cast<int64_t>(kslab) * MB) * 256;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) *reinterpret_cast<float4v *>(mine + mb * 256 + lane * 4) = acc[mb];
    __syncthreads();
    if (kslab != 0) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        float4v s0 = float4v{0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < p.ks; ++s) s0 += *reinterpret_cast<const float4v *>(red + (s * MB + mb) * 256 + lane * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mb * 16 + g * 4 + i;
            if (row < p.m) p.c[static_cast<int64_t>(row) * p.n + n0 + r] = s0[i];
        }
    }
}

// Any shape: one thread per output, f32 accumulation in k order.
__global__ __launch_bounds__(256) void gemm_generic(const half_t *a, const half_t *w, float *c, int m, int k, int n,
                                                    int w_is_kn, int mode) {
    const int outs_n = mode == 1 ? n / 2 : n;
    const int64_t total = static_cast<int64_t>(m) * outs_n;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int row = static_cast<int>(e / outs_n);
        const int col = static_cast<int>(e % outs_n);
        float s0 = 0.f, s1 = 0.f;
        for (int kk = 0; kk < k; ++kk) {
            const float av = static_cast<float>(a[static_cast<int64_t>(row) * k + kk]);
            const float w0 = static_cast<float>(w_is_kn ? w[static_cast<int64_t>(kk) * n + col] : w[static_cast<int64_t>(col) * k + kk]);
            s0 += av * w0;
            if (mode == 1) s1 += av * static_cast<float>(w[static_cast<int64_t>(col + outs_n) * k + kk]);
        }
        c[e] = mode == 1 ? silu_mul(s0, s1) : s0;
    }
}

__global__ __launch_bounds__(256) void swiglu_kernel(const float *g, const float *u, float *y, int64_t n) {
    for (int64_t i = blockIdx.x * int64_t(256) + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256)
        y[i] = silu_mul(g[i], u[i]);
}

int pick_ks(int64_t groups, int nb, int64_t k) {
    int ks = 1;
    while (ks * 2 * nb <= 16 && k % (64 * ks * 2) == 0 && k / (ks * 2) >= 128 && groups * ks * nb < 1024) ks *= 2;
    return ks;
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
    gemm_merge_splits<MODE><<<grid_for(outs, 256, 4), 256, 0, stream>>>(p.part, p.c, p.m, p.n, sp.ysplit);
    return hipGetLastError();
}

hipError_t launch_kn(const GemmParams &p0, int mb_blocks, hipStream_t stream) {
    GemmParams p = p0;
    const int64_t groups = p.n / 16;
    p.ks = pick_ks(groups, 1, p.k);
    p.slab = p.k / p.ks;
    const unsigned threads = static_cast<unsigned>(64 * p.ks);
    const size_t lds = static_cast<size_t>(p.ks) * mb_blocks * 256 * 4 + static_cast<size_t>(p.ks) * 16 * 72 * 2;
    switch (mb_blocks) {
        case 1: gemm_skinny_kn<1><<<static_cast<unsigned>(groups), threads, lds, stream>>>(p); break;
        case 2: gemm_skinny_kn<2><<<static_cast<unsigned>(groups), threads, lds, stream>>>(p); break;
        case 3: gemm_skinny_kn<3><<<static_cast<unsigned>(groups), threads, lds, stream>>>(p); break;
        default: gemm_skinny_kn<4><<<static_cast<unsigned>(groups), threads, lds, stream>>>(p); break;
    }
    return hipGetLastError();
}

// layout: 0 = W [n, k], 1 = W [k, n]; mode: 0 plain, 1 gate|up SiLU*mul
int gemm(const char *name, const dtts_f16 *a, const dtts_f16 *w, float *c, int64_t m, int64_t k, int64_t n, int layout,
         int mode, void *workspace, size_t ws_bytes, hipStream_t stream) {
    DTTS_REQUIRE(m >= 0 && k > 0 && n > 0, "%s: bad shape (%lld, %lld, %lld)", name, (long long)m, (long long)k,
                 (long long)n);
    DTTS_REQUIRE(mode == 0 || n % 2 == 0, "%s: gate|up width %lld is odd", name, (long long)n);
    if (m == 0) return DTTS_OK;
    DTTS_REQUIRE(a && w && c, "%s: null pointer", name);
    DTTS_REQUIRE(m < (int64_t(1) << 31) && k < (int64_t(1) << 31) && n < (int64_t(1) << 31), "%s: shape too large", name);
    GemmParams p{};
    p.a = reinterpret_cast<const half_t *>(a);
    p.w = reinterpret_cast<const half_t *>(w);
    p.c = c;
    p.m = static_cast<int>(m);
    p.k = static_cast<int>(k);
    p.n = static_cast<int>(n);
    const int64_t cols = mode == 1 ? n / 2 : n;
    const bool tiled = m <= 64 && k % 64 == 0 && cols % 16 == 0 && aligned(a, 16) && aligned(w, 16);
    const int mb_blocks = static_cast<int>((m + 15) / 16);
    const bool nt_ok = tiled && layout == 0 && pick_nt_split(cols / 16, mode == 1 ? 2 : 1, k, false).ks > 0;
    hipError_t e;
    if (nt_ok)
        e = mode == 1 ? launch_nt<1>(p, mb_blocks, workspace, ws_bytes, stream)
                      : launch_nt<0>(p, mb_blocks, workspace, ws_bytes, stream);
    else if (tiled && layout == 1 && mode == 0)
        e = launch_kn(p, mb_blocks, stream);
    else {
        gemm_generic<<<grid_for(m * cols, 256), 256, 0, stream>>>(p.a, p.w, c, p.m, p.k, p.n, layout, mode);
        e = hipGetLastError();
    }
    DTTS_HIP_CHECK(e, name);
    return DTTS_OK;
}

}  // namespace
}  // namespace dtts

extern "C" int dtts_gemm_f16_skinny(const dtts_f16 *a, const dtts_f16 *b_kn, float *c, int64_t m, int64_t k, int64_t n,
                                    hipStream_t stream) {
    return dtts::gemm("dtts_gemm_f16_skinny", a, b_kn, c, m, k, n, 1, 0, nullptr, 0, stream);
}

extern "C" size_t dtts_gemm_f16_workspace_bytes(int64_t m, int64_t k, int64_t n, int32_t gateup) {
    return dtts::nt_workspace_bytes(m, k, gateup ? 2 * n : n, gateup ? 1 : 0);
}

extern "C" int dtts_gemm_f16_nt(const dtts_f16 *a, const dtts_f16 *w_nk, float *c, int64_t m, int64_t k, int64_t n,
                                void *workspace, size_t ws_bytes, hipStream_t stream) {
    return dtts::gemm("dtts_gemm_f16_nt", a, w_nk, c, m, k, n, 0, 0, workspace, ws_bytes, stream);
}

extern "C" int dtts_gemm_f16_gateup_silu(const dtts_f16 *a, const dtts_f16 *w_gu, float *y, int64_t m, int64_t k,
                                         int64_t ffn, void *workspace, size_t ws_bytes, hipStream_t stream) {
    return dtts::gemm("dtts_gemm_f16_gateup_silu", a, w_gu, y, m, k, 2 * ffn, 0, 1, workspace, ws_bytes, stream);
}

extern "C" int dtts_swiglu_mul_f32(const float *g, const float *u, float *y, int64_t n, hipStream_t stream) {
    DTTS_REQUIRE(n >= 0, "dtts_swiglu_mul_f32: negative size");
    if (n == 0) return DTTS_OK;
    DTTS_REQUIRE(g && u && y, "dtts_swiglu_mul_f32: null pointer");
    dtts::swiglu_kernel<<<dtts::grid_for(n, 256), 256, 0, stream>>>(g, u, y, n);
    DTTS_LAUNCH_CHECK("dtts_swiglu_mul_f32");
    return DTTS_OK;
}
