// Decode-shape f32 projections: y[m, n] = x[m, k] . W[n, k]^T with W in the checkpoint's [out, in]
// layout, f32 throughout -- Proj::Dense's forward (matmul_2d of the f32 hidden state,
// crates/tts-nn/src/lib.rs:438-459, 527), the weight kind Stack::load takes for Weight::F32
// (crates/qwen3tts/src/qwen3.rs:236-250).
//
// The A-sharing form of the f16 and Q8_0 decode GEMMs on the f32 matrix cores
// (v_mfma_f32_16x16x4_f32): a workgroup of 4 waves owns 64 output columns (16 per wave) and a k
// range of KB 32-element blocks. Every lane requests its weights for the whole range first (two
// 16-byte loads per block: the 8 consecutive k of its lane group), then the activation slab
// x[0:m, range] is staged once in LDS, where the four waves read it. MFMA step e of a block's
// half s pairs k = 32b + 8g + 4s + e across the lane groups g, so each lane's operands are its own
// registers and one 16-byte LDS read per half. With several ranges each workgroup writes its
// partial [m, 64] tile to part[range] and the ranges are summed in order afterwards (by a merge
// launch here, by the consuming kernel inside the decoder-stack step).
#include "common.hpp"
#include "proj.hpp"

namespace dtts {
namespace {

typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kF32Pitch(int kb) { return kb * 32 + 4; }  // slab row: 4 floats of padding (bank offset 4 per row)
constexpr size_t f32_lds_bytes(int mb, int kb) { return static_cast<size_t>(mb) * 16 * kF32Pitch(kb) * 4; }

template <int MB, int KB>
__global__ __launch_bounds__(256) void gemm_f32_lds(const float *x, const float *w, float *y, float *part, int m, int k,
                                                    int n) {
    constexpr int KR = KB * 32, PITCH = kF32Pitch(KB), SEGS = KR / 4;
    __shared__ __attribute__((aligned(16))) float xs[MB * 16 * PITCH];
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
    for (int e = tid; e < MB * 16 * SEGS; e += 256) {
        const int row = e / SEGS, sg = e - (e / SEGS) * SEGS;
        float4v v = float4v{0.f, 0.f, 0.f, 0.f};
        if (row < m) v = *reinterpret_cast<const float4v *>(x + static_cast<int64_t>(row) * k + k0 + 4 * sg);
        *reinterpret_cast<float4v *>(xs + row * PITCH + 4 * sg) = v;
    }
    __syncthreads();
    float4v acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < KB; ++b)
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const float4v xa = *reinterpret_cast<const float4v *>(xs + (mb * 16 + r) * PITCH + 32 * b + 8 * g + 4 * s);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[e], wr[b][s][e], acc[mb], 0, 0, 0);
            }
    // the C fragment: lane (g, r) holds rows 4g + i of column r
    float *dst = part ? part + static_cast<int64_t>(blockIdx.y) * m * n : y;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mb * 16 + 4 * g + i;
            if (row < m) dst[static_cast<int64_t>(row) * n + col] = acc[mb][i];
        }
}

// y = the k ranges' partials summed in range order.
__global__ __launch_bounds__(256) void f32_merge(const float *part, float *y, int64_t mn, int ranges) {
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < mn; e += int64_t(gridDim.x) * 256) {
        float s = part[e];
        for (int q = 1; q < ranges; ++q) s += part[q * mn + e];
        y[e] = s;
    }
}

// Blocks per k range: the widest (8, 4, 2, 1 blocks of 32) giving at least 512 workgroups (two
// per CU), else the narrowest that divides k.
int pick_f32_kb(int64_t m, int64_t k, int64_t n) {
    if (m <= 0 || m > 64 || n % 64 != 0 || k % 32 != 0 || n / 64 >= 65536) return 0;
    const int64_t blocks = k / 32, tiles = n / 64;
    int last = 0;
    for (int kb : {8, 4, 2, 1}) {
        if (blocks % kb) continue;
        last = kb;
        if (tiles * (blocks / kb) >= 512) return kb;
    }
    return last;
}

template <int MB>
void launch_mb(int kb, dim3 grid, hipStream_t stream, const float *x, const float *w, float *y, float *part, int m,
               int k, int n) {
    switch (kb) {
        case 8: gemm_f32_lds<MB, 8><<<grid, 256, 0, stream>>>(x, w, y, part, m, k, n); break;
        case 4: gemm_f32_lds<MB, 4><<<grid, 256, 0, stream>>>(x, w, y, part, m, k, n); break;
        case 2: gemm_f32_lds<MB, 2><<<grid, 256, 0, stream>>>(x, w, y, part, m, k, n); break;
        default: gemm_f32_lds<MB, 1><<<grid, 256, 0, stream>>>(x, w, y, part, m, k, n); break;
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
