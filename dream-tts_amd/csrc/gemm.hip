// Decode-shape projection GEMMs: the entry points, the [k, n] operand kernel and the direct
// kernel for shapes the matrix-core kernels do not tile. The NT kernel is in gemm_nt.hpp.
#include <mutex>

#include "gemm_nt.hpp"

// Scratch of dtts_gemm_f16_nt_noalloc: the k-range partial tiles [ranges][m][n] f32 that
// dtts_gemm_f16_nt keeps in a caller's workspace. Each GPU the library runs on holds its own copy
// until the process ends. Host code never passes this name to a kernel (on the host it is a
// stand-in, not a device address): it passes the address hipGetSymbolAddress gave for the device.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace dtts {

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchDevices];  // per device: scratch's device address there
}  // namespace

// Resolves scratch's address on the current device once (dtts_init calls this; the entry point
// calls it again on a device it has not seen).
int noalloc_scratch_address(const char *name, void **out) {
    int dev = 0;
    DTTS_HIP_CHECK(hipGetDevice(&dev), name);
    DTTS_REQUIRE(dev >= 0 && dev < kScratchDevices, "%s: device %d beyond the %d this library tracks", name, dev,
                 kScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        DTTS_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), name);
        DTTS_REQUIRE(p && aligned(p, 256), "%s: scratch address %p", name, p);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return DTTS_OK;
}

namespace {

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

extern "C" int dtts_gemm_f16_nt_noalloc(const dtts_f16 *a, const dtts_f16 *w_nk, float *c, int64_t m, int64_t k,
                                        int64_t n, hipStream_t stream) {
    const char *name = "dtts_gemm_f16_nt_noalloc";
    DTTS_REQUIRE(m >= 0 && k > 0 && n > 0, "%s: bad shape (%lld, %lld, %lld)", name, (long long)m, (long long)k,
                 (long long)n);
    if (m == 0) return DTTS_OK;
    const size_t need = dtts::nt_workspace_bytes(m, k, n, 0);
    DTTS_REQUIRE(need <= kNoAllocScratchBytes,
                 "%s: (%lld, %lld, %lld) needs %zu bytes of scratch, more than the %zu this library holds", name,
                 (long long)m, (long long)k, (long long)n, need, kNoAllocScratchBytes);
    void *ws = nullptr;
    if (need > 0) {
        const int rc = dtts::noalloc_scratch_address(name, &ws);
        if (rc != DTTS_OK) return rc;
    }
    return dtts::gemm(name, a, w_nk, c, m, k, n, 0, 0, ws, need, stream);
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
