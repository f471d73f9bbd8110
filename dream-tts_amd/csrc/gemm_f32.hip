// Decode-shape f32 projections: y[m, n] = x[m, k] . W[n, k]^T with W in the checkpoint's [out, in]
// layout, f32 in and out -- Proj::Dense's forward (matmul_2d of the f32 hidden state,
// crates/tts-nn/src/lib.rs:438-459, 527), the weight kind Stack::load takes for Weight::F32
// (crates/qwen3tts/src/qwen3.rs:236-250).
//
// At f32 accuracy on the f16 matrix cores. A workgroup of 4 waves owns 64 output columns (16 per
// wave) and a k range of KB 32-element blocks. Every lane requests its weights for the whole range
// first (two 16-byte loads per block: the 8 consecutive k of its lane group) and its share of the
// activation slab x[0:m, range]. Each weight column is scaled by a power of two 2^e (its largest
// magnitude over the range then in [2^14, 2^15)) and split into f16 wh = f16(s) and wl =
// f16(s - wh) (s - wh is exact in f32, so the pair holds s to 2^-22 of itself); each 32-element
// block of an activation row likewise, and the slab's hi and lo halves go to LDS with the block
// scales. A block's product is then three v_mfma_f32_16x16x32_f16 (xl.wh, xh.wl, xh.wh; the
// dropped xl.wl is ~2^-22 of a term), rescaled by the row's block scale and summed in block order
// in f32; the column scale is undone at the store. Against the f32 matrix cores' 16x16x4 this is
// 3 products of K = 32 per block instead of 8 of K = 4. With several ranges each workgroup writes
// its partial [m, 64] tile to part[range] and the ranges are summed in order afterwards (by a merge
// launch here, by the consuming kernel inside the decoder-stack step).
#include "common.hpp"
#include "proj.hpp"

namespace dtts {
namespace {

typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kXPitch(int kb) { return kb * 32 + 8; }  // slab row in halves: 16 bytes of padding

// The power-of-two exponent that brings amax into [2^14, 2^15) (0 for amax == 0).
__device__ __forceinline__ int split_exponent(float amax) {
    if (!(amax > 0.0f)) return 0;
    int ex;
    frexpf(amax, &ex);  // amax = f * 2^ex, f in [0.5, 1)
    return min(max(15 - ex, -126), 126);
}

template <int MB, int KB>
__global__ __launch_bounds__(256) void gemm_f32_split(const float *x, const float *w, float *y, float *part, int m,
                                                      int k, int n) {
#pragma clang fp contract(off)
    constexpr int KR = KB * 32, PITCH = kXPitch(KB), SEGS = KR / 8;  // 8-element segments per slab row
    constexpr int TOTAL = MB * 16 * SEGS, ITERS = (TOTAL + 255) / 256;
    __shared__ __attribute__((aligned(16))) half_t xs[2][MB * 16 * PITCH];  // hi, lo
    __shared__ __attribute__((aligned(16))) float xsc[KB][MB * 16];           // 2^-e per (block, row)
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, r = lane & 15;
    const int col = blockIdx.x * 64 + wave * 16 + r;
    const int k0 = blockIdx.y * KR;
    float4v wr[KB][2];
    const float *wrow = w + static_cast<int64_t>(col) * k + k0 + 8 * g;
#pragma unroll
    for (int b = 0; b < KB; ++b) {
        wr[b][0] = *reinterpret_cast<const float4v *>(wrow + 32 * b);
        wr[b][1] = *reinterpret_cast<const float4v *>(wrow + 32 * b + 4);
    }
    // segment e = (row, sg): 8 activations at k0 + 8 sg; a row's 32-block is four consecutive
    // segments, held by four consecutive threads (every thread runs every iteration, so the quad
    // shuffles below see all four)
    float4v xv[ITERS][2];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int e = tid + it * 256;
        const int row = e / SEGS, sg = e - (e / SEGS) * SEGS;
        xv[it][0] = xv[it][1] = float4v{0.f, 0.f, 0.f, 0.f};
        if (e < TOTAL && row < m) {
            const float *src = x + static_cast<int64_t>(row) * k + k0 + 8 * sg;
            xv[it][0] = *reinterpret_cast<const float4v *>(src);
            xv[it][1] = *reinterpret_cast<const float4v *>(src + 4);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is in flight before the first wait
    // the lane's column over the range: one scale, from the four lane groups' amax
    float wmax = 0.0f;
#pragma unroll
    for (int b = 0; b < KB; ++b)
#pragma unroll
        for (int j = 0; j < 8; ++j) wmax = fmaxf(wmax, fabsf(wr[b][j / 4][j % 4]));
    wmax = fmaxf(wmax, __shfl_xor(wmax, 16, 64));
    wmax = fmaxf(wmax, __shfl_xor(wmax, 32, 64));
    const int ew = split_exponent(wmax);
    half8_t wh[KB], wl[KB];
#pragma unroll
    for (int b = 0; b < KB; ++b)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float sv = ldexpf(wr[b][j / 4][j % 4], ew);
            const half_t h = static_cast<half_t>(sv);
            wh[b][j] = h;
            wl[b][j] = static_cast<half_t>(sv - static_cast<float>(h));
        }
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int e = tid + it * 256;
        const int row = e / SEGS, sg = e - (e / SEGS) * SEGS;
        float xmax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) xmax = fmaxf(xmax, fabsf(xv[it][j / 4][j % 4]));
        xmax = fmaxf(xmax, __shfl_xor(xmax, 1, 64));
        xmax = fmaxf(xmax, __shfl_xor(xmax, 2, 64));
        const int ex = split_exponent(xmax);
        half8_t hi, lo;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float sv = ldexpf(xv[it][j / 4][j % 4], ex);
            const half_t h = static_cast<half_t>(sv);
            hi[j] = h;
            lo[j] = static_cast<half_t>(sv - static_cast<float>(h));
        }
        if (e < TOTAL) {
            *reinterpret_cast<half8_t *>(&xs[0][row * PITCH + 8 * sg]) = hi;
            *reinterpret_cast<half8_t *>(&xs[1][row * PITCH + 8 * sg]) = lo;
            if ((sg & 3) == 0) xsc[sg >> 2][row] = ldexpf(1.0f, -ex);
        }
    }
    __syncthreads();
    float4v acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < KB; ++b)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int o = (mb * 16 + r) * PITCH + 32 * b + 8 * g;
            const half8_t xh = *reinterpret_cast<const half8_t *>(&xs[0][o]);
            const half8_t xl = *reinterpret_cast<const half8_t *>(&xs[1][o]);
            float4v pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, wh[b], float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, wl[b], pr, 0, 0, 0);
            pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, wh[b], pr, 0, 0, 0);
            // the C fragment: lane (g, r) holds rows 4g + i of column r
            const float4v sc = *reinterpret_cast<const float4v *>(&xsc[b][mb * 16 + 4 * g]);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mb][i] += pr[i] * sc[i];
        }
    const float winv = ldexpf(1.0f, -ew);
    float *dst = part ? part + static_cast<int64_t>(blockIdx.y) * m * n : y;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mb * 16 + 4 * g + i;
            if (row < m) dst[static_cast<int64_t>(row) * n + col] = acc[mb][i] * winv;
        }
}

// y = the k ranges' partials summed in range order.
__global__ __launch_bounds__(256) void f32_merge(const float *part, float *y, int64_t mn, int ranges) {
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

// Blocks per k range: the widest (8, 4, 2, 1 blocks of 32) giving at least 192 workgroups, else
// the narrowest that divides k. (A 512-workgroup floor split config 4's k = 3072 into 48 ranges,
// whose partials outweighed the weights: 22.9 against 13.8 us.)
int pick_f32_kb(int64_t m, int64_t k, int64_t n) {
    if (m <= 0 || m > 64 || n % 64 != 0 || k % 32 != 0 || n / 64 >= 65536) return 0;
    const int64_t blocks = k / 32, tiles = n / 64;
    int last = 0;
    for (int kb : {8, 4, 2, 1}) {
        if (blocks % kb) continue;
        last = kb;
        if (tiles * (blocks / kb) >= 192) return kb;
    }
    return last;
}

template <int MB>
void launch_mb(int kb, dim3 grid, hipStream_t stream, const float *x, const float *w, float *y, float *part, int m,
               int k, int n) {
    switch (kb) {
        case 8: gemm_f32_split<MB, 8><<<grid, 256, 0, stream>>>(x, w, y, part, m, k, n); break;
        case 4: gemm_f32_split<MB, 4><<<grid, 256, 0, stream>>>(x, w, y, part, m, k, n); break;
        case 2: gemm_f32_split<MB, 2><<<grid, 256, 0, stream>>>(x, w, y, part, m, k, n); break;
        default: gemm_f32_split<MB, 1><<<grid, 256, 0, stream>>>(x, w, y, part, m, k, n); break;
    }
}

}  // namespace

int f32_proj_ranges(int64_t m, int64_t k, int64_t n) {
    const int kb = pick_f32_kb(m, k, n);
    return kb ? static_cast<int>(k / 32 / kb) : 0;
}

hipError_t f32_proj_launch(const float *x, const float *w, float *y, float *part, int64_t m, int64_t k, int64_t n,
                           bool merge, hipStream_t stream) {
    const int kb = pick_f32_kb(m, k, n);
    const int64_t ranges = k / 32 / kb;
    float *pp = ranges > 1 ? part : nullptr;
    const dim3 grid(static_cast<unsigned>(n / 64), static_cast<unsigned>(ranges));
    const int mi = static_cast<int>(m), ki = static_cast<int>(k), ni = static_cast<int>(n);
    switch ((m + 15) / 16) {
        case 1: launch_mb<1>(kb, grid, stream, x, w, y, pp, mi, ki, ni); break;
        case 2: launch_mb<2>(kb, grid, stream, x, w, y, pp, mi, ki, ni); break;
        case 3: launch_mb<3>(kb, grid, stream, x, w, y, pp, mi, ki, ni); break;
        default: launch_mb<4>(kb, grid, stream, x, w, y, pp, mi, ki, ni); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !pp || !merge) return e;
    f32_merge<<<grid_for(m * n, 256), 256, 0, stream>>>(pp, y, m * n, static_cast<int>(ranges));
    return hipGetLastError();
}

}  // namespace dtts

extern "C" size_t dtts_gemm_f32_nt_workspace_bytes(int64_t m, int64_t k, int64_t n) {
    const int ranges = dtts::f32_proj_ranges(m, k, n);
    return ranges > 1 ? static_cast<size_t>(ranges * m * n) * sizeof(float) : 0;
}

extern "C" int dtts_gemm_f32_nt(const float *x, const float *w, float *y, int64_t m, int64_t k, int64_t n,
                                void *workspace, size_t ws_bytes, hipStream_t stream) {
    const char *name = "dtts_gemm_f32_nt";
    DTTS_REQUIRE(m >= 0 && k > 0 && n > 0, "%s: bad shape (%lld, %lld, %lld)", name, (long long)m, (long long)k,
                 (long long)n);
    if (m == 0) return DTTS_OK;
    DTTS_REQUIRE(x && w && y, "%s: null pointer", name);
    DTTS_REQUIRE(m <= 64 && k % 32 == 0 && n % 64 == 0,
                 "%s: shape (%lld, %lld, %lld): m <= 64, k a multiple of 32 and n of 64", name, (long long)m,
                 (long long)k, (long long)n);
    DTTS_REQUIRE(k < (int64_t(1) << 30) && n < (int64_t(1) << 22), "%s: shape too large", name);
    DTTS_REQUIRE(dtts::aligned(x, 16) && dtts::aligned(w, 16), "%s: x and w must be 16-byte aligned", name);
    const size_t need = dtts_gemm_f32_nt_workspace_bytes(m, k, n);
    DTTS_REQUIRE(!need || (workspace && ws_bytes >= need && dtts::aligned(workspace, 16)),
                 "%s: workspace %zu bytes (16-byte aligned) < %zu needed", name, ws_bytes, need);
    DTTS_HIP_CHECK(dtts::f32_proj_launch(x, w, y, static_cast<float *>(workspace), m, k, n, true, stream), name);
    return DTTS_OK;
}
