// The codec's convs at f32 accuracy on the f16 matrix cores: every f32 activation is stored as a
// pair of f16 values, hi = f16(v) and lo = f16(v - hi) (v - hi is exact in f32, so the pair holds
// v to 2^-22 of itself, in the same 4 bytes), a stored row of C channels being [hi(C) | lo(C)];
// every conv weight is scaled by a power of two 2^s (its largest magnitude then in [2^14, 2^15),
// which keeps the low halves of its large entries normal) and split the same way. A conv over cin
// channels is then one f16 implicit GEMM over K' = 3 cin channels per tap,
//
//   sum_c x w = sum_c (xh wh + xl wh + xh wl) + O(2^-22)        (xl wl, ~2^-22 of a term, dropped)
//
// with the window's chunks reading hi, lo, hi (conv_mainloop_direct's SPLIT mode) against weights
// [wh | wh | wl]. The epilogue takes the f32 sum (times 2^-s, exact), adds the f32 bias and the
// split residual in f32, stores the pre-activation value split, applies SnakeBeta at full precision
// (sinf) and stores the result split. A transposed conv's output (rate x cout phase columns per
// input position) is written in its consumer's layout, position l*rate + p, channel c.
//
// This is the reference's own precision (its codec is f32: WAV_DTYPE, crates/qwen3tts/src/
// codec.rs:33-43; NlcConv, crates/tts-nn/src/nlcconv.rs:15-198) at three f16 products per term.
#include "conv_tile.hpp"

namespace dtts {
namespace {

struct SplitArgs {
    ConvArgs c;      // x, w (the split weight), L, cin (= 3 cs), cout (GEMM columns), k, dil, pad_left, tiles
    float w_inv;     // 2^-s
    const float *bias;
    const half_t *res;  // split, the output's layout
    half_t *y_pre, *y;  // split, the output's layout
    const float *a_out, *r_out;  // per GEMM column
    int cv;          // channels of the output's rows (cout, or cout / rate for a transposed conv)
};

__device__ __forceinline__ void split_store8(half_t *dst, int cv, const float (&v)[8]) {
    half8_t hi, lo;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        hi[q] = static_cast<half_t>(v[q]);
        lo[q] = static_cast<half_t>(v[q] - static_cast<float>(hi[q]));
    }
    *reinterpret_cast<half8_t *>(dst) = hi;
    *reinterpret_cast<half8_t *>(dst + cv) = lo;
}

// The tile's per-column constants in LDS, past the stages and the epilogue's staging: the f32 bias,
// and SnakeBeta's alpha and 1/beta, of its BN GEMM columns. They are written before the main loop,
// whose barriers publish them, so the epilogue reads them from LDS instead of waiting on global
// loads inside its loop.
template <typename Cfg>
struct SplitTab {
    static constexpr int OFFSET = Cfg::TAB_OFFSET;
    static constexpr int BYTES = OFFSET + 3 * Cfg::BN * 4;
};

template <typename Cfg>
__device__ __forceinline__ void split_table(char *smem, int n0, const SplitArgs &a) {
    float *tab = reinterpret_cast<float *>(smem + SplitTab<Cfg>::OFFSET);
    for (int c = threadIdx.x; c < Cfg::BN; c += Cfg::THREADS) {
        tab[c] = a.bias ? a.bias[n0 + c] : 0.0f;
        tab[Cfg::BN + c] = a.a_out ? a.a_out[n0 + c] : 0.0f;
        tab[2 * Cfg::BN + c] = a.r_out ? a.r_out[n0 + c] : 0.0f;
    }
}

__device__ __forceinline__ void split_store8_buf(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint32_t lo_off,
                                                 const float (&v)[8]) {
    half8_t hi, lo;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        hi[q] = static_cast<half_t>(v[q]);
        lo[q] = static_cast<half_t>(v[q] - static_cast<float>(hi[q]));
    }
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u_t, hi), rs, off, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u_t, lo), rs, off + lo_off, 0, 0);
}

// The tile's outputs, one 32-row block per wave at a time through the wave's LDS region (as the
// f16 epilogue does): a lane then owns 8 consecutive GEMM columns of one position. The residual,
// y_pre and y rows of the tile's lane are reached through buffer resources sized to that lane's
// rows, and a position past the sequence gets an offset beyond them: its loads read zeros and its
// stores are dropped by the hardware's range check, so no branch splits a block and the loads of
// a block's groups are all in flight together (conv_split_supported keeps a lane's output rows
// under 2^31 bytes).
template <typename Cfg>
__device__ __forceinline__ void split_epilogue(const float16_t (&acc)[Cfg::TM][Cfg::TN], char *smem, int64_t row0,
                                               int l0, int n0, const SplitArgs &a) {
#pragma clang fp contract(off)
    constexpr int CG = Cfg::WTN / 8;
    constexpr int NG = 32 * CG / 64;
    static_assert((32 * CG) % 64 == 0, "a 32-row block splits evenly over the lanes");
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int l32 = lane & 31, hf = lane >> 5;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
    float *E = reinterpret_cast<float *>(smem) + wave * 32 * Cfg::EPI_PITCH;
    const float *tab = reinterpret_cast<const float *>(smem + SplitTab<Cfg>::OFFSET);
    const int nw = n0 + wn * Cfg::WTN;
    const int cv = a.cv, R = a.c.cout / a.cv;
    const int lmax = a.c.L;
    const uint32_t lane_bytes = static_cast<uint32_t>(static_cast<int64_t>(lmax) * R * 2 * cv * 2);
    const int64_t base = row0 * R * 2 * cv;
    const __amdgpu_buffer_rsrc_t rs_res =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t *>(a.res ? a.res + base : a.y + base), 0, lane_bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rs_y = __builtin_amdgcn_make_buffer_rsrc(a.y + base, 0, lane_bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rs_yp =
        __builtin_amdgcn_make_buffer_rsrc(a.y_pre ? a.y_pre + base : a.y + base, 0, lane_bytes, kBufferWord3);
    const uint32_t lo_off = static_cast<uint32_t>(cv * 2);
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i) {
        const int lb = l0 + wm * Cfg::WTM + i * 32;
        if (i > 0) wave_lds_order();
#pragma unroll
        for (int j = 0; j < Cfg::TN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<float4_t *>(E + l32 * Cfg::EPI_PITCH + 32 * j + 8 * g + 4 * hf) =
                    float4_t{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        wave_lds_order();
#pragma unroll
        for (int u = 0; u < NG; ++u) {
            const int g = lane + 64 * u;
            const int mr = g / CG, cg = g - (g / CG) * CG;
            const int l = lb + mr;
            const int n = nw + cg * 8;
            const int ph = n / cv, c = n - ph * cv;
            const uint32_t off = l < lmax ? static_cast<uint32_t>(((static_cast<int64_t>(l) * R + ph) * 2 * cv + c) * 2)
                                          : kOutOfRange;
            const float4_t *src = reinterpret_cast<const float4_t *>(E + mr * Cfg::EPI_PITCH + cg * 8);
            const float4_t v0 = src[0], v1 = src[1];
            const int tc = n - n0;
            const float4_t b0 = *reinterpret_cast<const float4_t *>(tab + tc);
            const float4_t b1 = *reinterpret_cast<const float4_t *>(tab + tc + 4);
            float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            const float b[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
#pragma unroll
            for (int q = 0; q < 8; ++q) v[q] = v[q] * a.w_inv + b[q];
            if (a.res) {
                const half8_t rh = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(rs_res, off, 0, 0));
                const half8_t rl = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(rs_res, off + lo_off, 0, 0));
#pragma unroll
                for (int q = 0; q < 8; ++q) v[q] = v[q] + (static_cast<float>(rh[q]) + static_cast<float>(rl[q]));
            }
            if (a.y_pre) split_store8_buf(rs_yp, off, lo_off, v);
            if (a.a_out) {
                const float4_t a0 = *reinterpret_cast<const float4_t *>(tab + Cfg::BN + tc);
                const float4_t a1 = *reinterpret_cast<const float4_t *>(tab + Cfg::BN + tc + 4);
                const float4_t r0 = *reinterpret_cast<const float4_t *>(tab + 2 * Cfg::BN + tc);
                const float4_t r1 = *reinterpret_cast<const float4_t *>(tab + 2 * Cfg::BN + tc + 4);
                const float aa[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
                const float rr[8] = {r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]};
                snake_f32_group<8>(v, aa, rr);
            }
            split_store8_buf(rs_y, off, lo_off, v);
        }
    }
}

template <typename Cfg, int KT>
__global__ __launch_bounds__(Cfg::THREADS, Cfg::MIN_WG) void conv_split_mfma(SplitArgs a) {
    static_assert(Cfg::STAGING == kStageDirect, "split operands use direct staging");
    __shared__ __attribute__((aligned(16))) char smem[SplitTab<Cfg>::BYTES];
    int lane_idx, m_tile, n_tile;
    if (!conv_tile_coords(a.c, lane_idx, m_tile, n_tile)) return;
    const int l0 = m_tile * Cfg::BM;
    const int n0 = n_tile * Cfg::BN;
    split_table<Cfg>(smem, n0, a);
    const half_t *xl = a.c.x + static_cast<int64_t>(lane_idx) * a.c.L * (2 * (a.c.cin / 3));
    float16_t acc[Cfg::TM][Cfg::TN];
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::TN; ++j) acc[i][j] = float16_t{};
    conv_mainloop_direct<Cfg, false, KT, true>(a.c, xl, l0, n0, smem, acc);
    split_epilogue<Cfg>(acc, smem, static_cast<int64_t>(lane_idx) * a.c.L, l0, n0, a);
}

template <typename Cfg>
struct STile {
    typedef Cfg type;
};

// The split tiles: the f16 codec's direct-staging tiles for each class (their sweeps on the same
// GEMM shapes), with 96-wide k = 1 tiles for the narrowest stage. Returns false when no tile
// takes the shape. cin here is K' = 3 cs; every tile's KC divides cs (KC | 3 cs and 3 is odd).
template <int KMAX, int HMAX, typename F>
bool with_split_tile(int64_t lanes, int len, int cin, int cout, F &&f) {
    if constexpr (KMAX == 7) {
        if (cout % 96 == 0 && len >= 1024) return f(STile<ConvTile<512, 96, 8, 1, 32, KMAX, HMAX, 2, kStageDirect>>{}), true;
        if (cout % 96 == 0) return f(STile<ConvTile<256, 96, 4, 1, 16, KMAX, HMAX, 2, kStageDirect>>{}), true;
    }
    if constexpr (KMAX == 2) {
        if (cout % 128 == 0 && cin >= 768) return f(STile<ConvTile<256, 128, 2, 2, 32, KMAX, HMAX, 2, kStageDirect>>{}), true;
        if (cout % 128 == 0) return f(STile<ConvTile<128, 128, 2, 2, 32, KMAX, HMAX, 2, kStageDirect>>{}), true;
        if (cout % 96 == 0) return f(STile<ConvTile<128, 96, 4, 1, 32, KMAX, HMAX, 2, kStageDirect>>{}), true;
    }
    if constexpr (KMAX == 1) {
        const int64_t tiles128 = lanes * ((len + 127) / 128) * (cout / 128);
        // 96 wide: 128 x 96 over four waves, three stages (three workgroups per CU; 15-23% faster
        // than 256 x 96 with two, on the codec's 96-channel k = 1 convs)
        if (cout == 96) return f(STile<ConvTile<128, 96, 4, 1, 32, KMAX, HMAX, 3, kStageDirect>>{}), true;
        if (cout % 64 == 0 && cin % 64 == 0 && (cout % 128 != 0 || tiles128 < 1024))
            return f(STile<ConvTile<128, 64, 2, 2, 64, KMAX, HMAX, 2, kStageDirect>>{}), true;
        if (cout % 128 == 0 && cin % 64 == 0 && cin > 2048)
            return f(STile<ConvTile<128, 128, 2, 2, 64, KMAX, HMAX, 2, kStageDirect>>{}), true;
        if (cout % 128 == 0) return f(STile<ConvTile<128, 128, 2, 2, 32, KMAX, HMAX, 3, kStageDirect>>{}), true;
        if (cout % 96 == 0) return f(STile<ConvTile<256, 96, 4, 1, 32, KMAX, HMAX, 2, kStageDirect>>{}), true;
    }
    return false;
}

// The class of a conv: (KMAX, HMAX) as the f16 tiles group them, or 0 when the k and halo fit none.
int split_class(int64_t k, int64_t dil, int &hmax) {
    const int64_t halo = (k - 1) * dil;
    if (k == 1) return hmax = 0, 1;
    if (k <= 2 && halo <= 8) return hmax = 8, 2;
    if (k <= 7 && halo <= 64) return hmax = 64, 7;
    return 0;
}

template <typename F>
bool with_split_tile_k(int kmax, int64_t lanes, int len, int cin, int cout, F &&f) {
    if (kmax == 1) return with_split_tile<1, 0>(lanes, len, cin, cout, f);
    if (kmax == 2) return with_split_tile<2, 8>(lanes, len, cin, cout, f);
    return with_split_tile<7, 64>(lanes, len, cin, cout, f);
}

template <typename Cfg>
hipError_t launch_split(SplitArgs a, int64_t lanes, hipStream_t stream) {
    ConvArgs &p = a.c;
    p.tiles_m = (p.L + Cfg::BM - 1) / Cfg::BM;
    p.tiles_n = p.cout / Cfg::BN;
    p.tiles_ng = pick_tiles_ng(p.tiles_n, int64_t(Cfg::BN) * p.k * p.cin * 2);
    const int64_t total = lanes * p.tiles_m * p.tiles_n;
    p.total_tiles = static_cast<int>(total);
    p.tiles_per_xcd = static_cast<int>((total + 7) / 8);
    const unsigned grid = static_cast<unsigned>(int64_t(p.tiles_per_xcd) * 8);
    if (p.k == Cfg::KMAX)
        conv_split_mfma<Cfg, Cfg::KMAX><<<grid, Cfg::THREADS, 0, stream>>>(a);
    else
        conv_split_mfma<Cfg, 0><<<grid, Cfg::THREADS, 0, stream>>>(a);
    return hipGetLastError();
}

// Largest |w| over n floats, as the bit pattern of a non-negative float (ordered like the value).
__global__ __launch_bounds__(256) void absmax_bits(const float *w, int64_t n, unsigned *out) {
    float m = 0.0f;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < n; e += int64_t(gridDim.x) * 256) m = fmaxf(m, fabsf(w[e]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((threadIdx.x & 63) == 0) atomicMax(out, __float_as_uint(m));
}

// Tap-major f32 w [cout, k cs] -> [cout, k * 3 cs]: per tap [wh | wh | wl] of w * scale.
__global__ __launch_bounds__(256) void split_weight_kernel(const float *w, half_t *w3, int64_t cout, int k, int cs,
                                                           float scale) {
#pragma clang fp contract(off)
    const int64_t total = cout * k * cs;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t row = e / (int64_t(k) * cs);
        const int rest = static_cast<int>(e - row * k * cs);
        const int t = rest / cs, ci = rest - t * cs;
        const float v = w[e] * scale;
        const half_t h = static_cast<half_t>(v);
        const half_t l = static_cast<half_t>(v - static_cast<float>(h));
        half_t *dst = w3 + row * (int64_t(3) * k * cs) + int64_t(t) * 3 * cs + ci;
        dst[0] = h;
        dst[cs] = h;
        dst[2 * cs] = l;
    }
}

// Split rows [hi(C) | lo(C)] -> f32 [rows, C] (hi + lo), 8 values per thread.
__global__ __launch_bounds__(256) void join_act_kernel(const half_t *x, float *y, int64_t rows, int C) {
    const int c8 = C / 8;
    const int64_t total = rows * c8;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t r = e / c8;
        const int c = static_cast<int>(e - r * c8) * 8;
        const half8_t hi = *reinterpret_cast<const half8_t *>(x + r * 2 * C + c);
        const half8_t lo = *reinterpret_cast<const half8_t *>(x + r * 2 * C + C + c);
        float4_t a, b;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            a[q] = static_cast<float>(hi[q]) + static_cast<float>(lo[q]);
            b[q] = static_cast<float>(hi[4 + q]) + static_cast<float>(lo[4 + q]);
        }
        *reinterpret_cast<float4_t *>(y + r * C + c) = a;
        *reinterpret_cast<float4_t *>(y + r * C + c + 4) = b;
    }
}

// f32 [rows, C] -> split rows [hi(C) | lo(C)], 8 values per thread.
__global__ __launch_bounds__(256) void split_act_kernel(const float *x, half_t *y, int64_t rows, int C) {
#pragma clang fp contract(off)
    const int c8 = C / 8;
    const int64_t total = rows * c8;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t r = e / c8;
        const int c = static_cast<int>(e - r * c8) * 8;
        const float4_t a = *reinterpret_cast<const float4_t *>(x + r * C + c);
        const float4_t b = *reinterpret_cast<const float4_t *>(x + r * C + c + 4);
        const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        split_store8(y + r * 2 * C + c, C, v);
    }
}

}  // namespace

bool conv_split_supported(int64_t lanes, int64_t len, int64_t cs, int64_t cout, int64_t k, int64_t dil) {
    int hmax;
    const int kmax = split_class(k, dil, hmax);
    // a lane's split output rows (len positions x cout GEMM columns, 4 bytes each) are one epilogue
    // buffer range, below the 2^31 offset that marks rows past the sequence
    if (!kmax || cs % 32 != 0 || cout % 32 != 0 || !direct_offsets_fit(len, 3 * cs, cout, k) ||
        len * cout * 4 >= (int64_t(1) << 31))
        return false;
    return with_split_tile_k(kmax, lanes, static_cast<int>(len), static_cast<int>(3 * cs), static_cast<int>(cout),
                             [](auto) {});
}

const char *conv_split_kernel_name(int64_t lanes, int64_t len, int64_t cs, int64_t cout, int64_t k, int64_t dil) {
    static thread_local char buf[128];
    int hmax;
    const int kmax = split_class(k, dil, hmax);
    buf[0] = 0;
    with_split_tile_k(kmax, lanes, static_cast<int>(len), static_cast<int>(3 * cs), static_cast<int>(cout), [&](auto t) {
        typedef typename decltype(t)::type Cfg;
        tile_kernel_name<Cfg>(buf, sizeof(buf), "conv_split_mfma", k == Cfg::KMAX ? (Cfg::KMAX == 7 ? ", 7>" : Cfg::KMAX == 2 ? ", 2>" : ", 1>") : ", 0>");
    });
    return buf;
}

int conv1d_nlc_split(const SplitConv &s, hipStream_t stream) {
    const char *name = "dtts_codec (split conv)";
    DTTS_REQUIRE(conv_split_supported(s.lanes, s.len, s.cs, s.cout, s.k, s.dil), "%s: shape not supported", name);
    DTTS_REQUIRE(s.cv > 0 && s.cout % s.cv == 0 && s.cv % 8 == 0 && (!s.res || s.cv == s.cout), "%s: bad output view",
                 name);
    SplitArgs a{};
    a.c.x = s.x;
    a.c.w = s.w;
    a.c.L = static_cast<int>(s.len);
    a.c.cin = static_cast<int>(3 * s.cs);
    a.c.cout = static_cast<int>(s.cout);
    a.c.k = static_cast<int>(s.k);
    a.c.dil = static_cast<int>(s.dil);
    a.c.pad_left = static_cast<int>(s.pad_left);
    a.w_inv = s.w_inv;
    a.bias = s.bias;
    a.res = s.res;
    a.y_pre = s.y_pre;
    a.y = s.y;
    a.a_out = s.a_out;
    a.r_out = s.r_out;
    a.cv = static_cast<int>(s.cv);
    int hmax;
    const int kmax = split_class(s.k, s.dil, hmax);
    hipError_t e = hipSuccess;
    with_split_tile_k(kmax, s.lanes, a.c.L, a.c.cin, a.c.cout, [&](auto t) {
        typedef typename decltype(t)::type Cfg;
        e = launch_split<Cfg>(a, s.lanes, stream);
    });
    DTTS_HIP_CHECK(e, name);
    return DTTS_OK;
}

int split_weight(const float *w, int64_t cout, int64_t k, int64_t cs, half_t *w3, float &w_inv, hipStream_t stream,
                 const char *name) {
    const int64_t n = cout * k * cs;
    unsigned *bits = nullptr;
    DTTS_HIP_CHECK(hipMalloc(&bits, sizeof(unsigned)), name);
    unsigned host = 0;
    hipError_t e = hipMemsetAsync(bits, 0, sizeof(unsigned), stream);
    if (e == hipSuccess) {
        absmax_bits<<<grid_for(n, 256), 256, 0, stream>>>(w, n, bits);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpyAsync(&host, bits, sizeof(unsigned), hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    (void)hipFree(bits);
    DTTS_HIP_CHECK(e, name);
    float amax;
    std::memcpy(&amax, &host, sizeof(float));
    DTTS_REQUIRE(std::isfinite(amax), "%s: a weight is not finite", name);
    int ex = 0;
    if (amax > 0.0f) std::frexp(amax, &ex);  // amax = f 2^ex, f in [0.5, 1)
    const int sh = amax > 0.0f ? 15 - ex : 0;  // amax * 2^sh in [2^14, 2^15)
    const float scale = std::ldexp(1.0f, sh);
    w_inv = std::ldexp(1.0f, -sh);
    split_weight_kernel<<<grid_for(n, 256), 256, 0, stream>>>(w, w3, cout, static_cast<int>(k), static_cast<int>(cs),
                                                               scale);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

int split_activations(const float *x, half_t *y, int64_t rows, int64_t C, hipStream_t stream) {
    const char *name = "dtts_codec_decode_f32 (split latent)";
    DTTS_REQUIRE(C % 8 == 0 && rows * C < (int64_t(1) << 40), "%s: bad shape", name);
    DTTS_REQUIRE(aligned(x, 16) && aligned(y, 16), "%s: operands must be 16-byte aligned", name);
    split_act_kernel<<<grid_for(rows * (C / 8), 256), 256, 0, stream>>>(x, y, rows, static_cast<int>(C));
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

}  // namespace dtts

// ---------------------------------------------------------------- the op-level entry points
//
// NlcConv on f32 operands through the split route: the weight is split once at load
// (dtts_conv_split_weight), and each call splits x (and the residual) into the workspace, runs the
// split conv and joins the outputs back to f32.

using dtts::half_t;

namespace {

size_t split_ws_align(size_t b) { return (b + 255) & ~size_t(255); }

struct SplitWs {
    size_t x, res, y, y_pre, total;
};

SplitWs split_ws_plan(const dtts_conv_desc *d) {
    SplitWs w{};
    const size_t rows = static_cast<size_t>(d->lanes) * static_cast<size_t>(d->len);
    w.x = split_ws_align(rows * d->cin * 4);
    w.res = d->residual ? split_ws_align(rows * d->cout * 4) : 0;
    w.y = split_ws_align(rows * d->cout * 4);
    w.y_pre = d->y_pre ? split_ws_align(rows * d->cout * 4) : 0;
    w.total = w.x + w.res + w.y + w.y_pre;
    return w;
}

}  // namespace

extern "C" size_t dtts_conv_split_weight_bytes(int64_t cout, int64_t k, int64_t cin) {
    return cout > 0 && k > 0 && cin > 0 ? static_cast<size_t>(cout) * k * 3 * cin * sizeof(half_t) : 0;
}

extern "C" int dtts_conv_split_weight(const float *w_tm, int64_t cout, int64_t k, int64_t cin, void *w_split,
                                      float *w_inv, hipStream_t stream) {
    const char *name = "dtts_conv_split_weight";
    DTTS_REQUIRE(cout > 0 && k > 0 && k <= 7 && cin > 0 && cin % 8 == 0, "%s: bad shape (cout %lld, k %lld, cin %lld)",
                 name, (long long)cout, (long long)k, (long long)cin);
    DTTS_REQUIRE(w_tm && w_split && w_inv, "%s: null pointer", name);
    DTTS_REQUIRE(cout * k * cin < (int64_t(1) << 31), "%s: weight too large", name);
    float inv = 1.0f;
    const int rc = dtts::split_weight(w_tm, cout, k, cin, static_cast<half_t *>(w_split), inv, stream, name);
    if (rc != DTTS_OK) return rc;
    *w_inv = inv;
    return DTTS_OK;
}

extern "C" size_t dtts_conv1d_nlc_f32_split_workspace_bytes(const dtts_conv_desc *desc) {
    if (!desc || desc->lanes <= 0 || desc->len <= 0 || desc->cin <= 0 || desc->cout <= 0) return 0;
    return split_ws_plan(desc).total;
}

extern "C" int dtts_conv1d_nlc_f32_split(const dtts_conv_desc *desc, float w_inv, void *workspace,
                                         size_t workspace_bytes, hipStream_t stream) {
    const char *name = "dtts_conv1d_nlc_f32_split";
    DTTS_REQUIRE(desc, "%s: null descriptor", name);
    const dtts_conv_desc &d = *desc;
    DTTS_REQUIRE(d.lanes >= 0 && d.len >= 0 && d.cin > 0 && d.cout > 0 && d.k >= 1 && d.dilation >= 1 &&
                     d.pad_left >= 0 && d.pad_left <= (d.k - 1) * d.dilation,
                 "%s: bad shape", name);
    if (d.lanes == 0 || d.len == 0) return DTTS_OK;
    DTTS_REQUIRE(d.x && d.w && d.y, "%s: null pointer", name);
    if (d.in_alpha || d.act != 0 || d.out_scale || (d.out_alpha == nullptr) != (d.out_brecip == nullptr) ||
        !dtts::conv_split_supported(d.lanes, d.len, d.cin, d.cout, d.k, d.dilation)) {
        dtts::set_error("%s: no split kernel for this conv (prologue SnakeBeta, activation, out_scale, or shape "
                        "cin %lld cout %lld k %lld dilation %lld); use dtts_conv1d_nlc_f32_ex",
                        name, (long long)d.cin, (long long)d.cout, (long long)d.k, (long long)d.dilation);
        return DTTS_ERR_UNSUPPORTED;
    }
    int w_exp = 0;
    DTTS_REQUIRE(std::isfinite(w_inv) && w_inv > 0.0f && std::frexp(w_inv, &w_exp) == 0.5f,
                 "%s: w_inv %g is not a positive power of two", name, w_inv);
    const SplitWs plan = split_ws_plan(desc);
    DTTS_REQUIRE(workspace && workspace_bytes >= plan.total && dtts::aligned(workspace, 256),
                 "%s: workspace %zu bytes (256-byte aligned) < %zu needed", name, workspace_bytes, plan.total);
    DTTS_REQUIRE(dtts::aligned(d.x, 16) && dtts::aligned(d.w, 16) && dtts::aligned(d.y, 16) &&
                     (!d.residual || dtts::aligned(d.residual, 16)) && (!d.y_pre || dtts::aligned(d.y_pre, 16)) &&
                     (!d.bias || dtts::aligned(d.bias, 16)) && (!d.out_alpha || dtts::aligned(d.out_alpha, 16)) &&
                     (!d.out_brecip || dtts::aligned(d.out_brecip, 16)),
                 "%s: x, w, bias, residual, y_pre, y and the SnakeBeta vectors must be 16-byte aligned", name);
    char *ws = static_cast<char *>(workspace);
    half_t *xs = reinterpret_cast<half_t *>(ws);
    half_t *rs = d.residual ? reinterpret_cast<half_t *>(ws + plan.x) : nullptr;
    half_t *ys = reinterpret_cast<half_t *>(ws + plan.x + plan.res);
    half_t *yps = d.y_pre ? reinterpret_cast<half_t *>(ws + plan.x + plan.res + plan.y) : nullptr;
    const int64_t rows = d.lanes * d.len;
    int rc = dtts::split_activations(static_cast<const float *>(d.x), xs, rows, d.cin, stream);
    if (rc == DTTS_OK && rs) rc = dtts::split_activations(static_cast<const float *>(d.residual), rs, rows, d.cout, stream);
    if (rc != DTTS_OK) return rc;
    dtts::SplitConv sc{};
    sc.lanes = d.lanes;
    sc.len = d.len;
    sc.cs = d.cin;
    sc.cout = d.cout;
    sc.k = d.k;
    sc.dil = d.dilation;
    sc.pad_left = d.pad_left;
    sc.cv = d.cout;
    sc.x = xs;
    sc.w = static_cast<const half_t *>(d.w);
    sc.w_inv = w_inv;
    sc.bias = static_cast<const float *>(d.bias);
    sc.res = rs;
    sc.y_pre = yps;
    sc.y = ys;
    sc.a_out = d.out_alpha;
    sc.r_out = d.out_brecip;
    rc = dtts::conv1d_nlc_split(sc, stream);
    if (rc != DTTS_OK) return rc;
    const unsigned grid = dtts::grid_for(rows * (d.cout / 8), 256);
    dtts::join_act_kernel<<<grid, 256, 0, stream>>>(ys, static_cast<float *>(d.y), rows, static_cast<int>(d.cout));
    DTTS_LAUNCH_CHECK(name);
    if (yps) {
        dtts::join_act_kernel<<<grid, 256, 0, stream>>>(yps, static_cast<float *>(d.y_pre), rows,
                                                        static_cast<int>(d.cout));
        DTTS_LAUNCH_CHECK(name);
    }
    return DTTS_OK;
}

