// Channels-last conv1d as an implicit GEMM on the matrix cores, with the tap gather inside.
//
//   y[b, l, n] = act( bias[n] + res[b, l, n] + sum_t sum_c xs[b, l + t*dil - pad_left, c] * w[n, t*cin + c] )
//
// xs is x, or SnakeBeta(x) when a prologue snake is given; out-of-range taps read zero (and
// snake(0) = 0, so padding before or after the snake is the same). Optionally the rounded sum is
// stored (y_pre) and SnakeBeta is applied to it before the final store (the next activation,
// moved into this kernel's epilogue).
//
// GEMM view per lane: M = positions, N = output channels, K = k*cin (tap-major). One workgroup
// owns BM positions x BN channels. Per 32-channel chunk it stages, in LDS:
//   A: the whole dilated window, BM + (k-1)*dil rows x 32 channels, loaded once and read by
//      all k taps at row offsets t*dil (the im2col never exists, not even in LDS);
//   B: w[n0 .. n0+BN, t*cin + c0 .. +32] for every tap t.
// Four waves split M (64 rows each) and cover all BN columns with 32x32x16 f16 MFMAs (f32
// accumulate). The next chunk is prefetched into registers while the current one computes.
// The epilogue goes through LDS so bias/residual/stores move 16 bytes per lane, coalesced.
#include "conv_tile.hpp"

namespace dtts {
namespace {

typedef ConvArgs ConvParams;

template <typename Cfg, bool SNAKE_IN, int KT>
__global__ __launch_bounds__(Cfg::THREADS, Cfg::MIN_WG) void conv_nlc_f16_mfma(ConvArgs p) {
    __shared__ __attribute__((aligned(16))) char smem[Cfg::LDS_BYTES];
    int lane_idx, m_tile, n_tile;
    if (!conv_tile_coords(p, lane_idx, m_tile, n_tile)) return;
    const int l0 = m_tile * Cfg::BM;
    const int n0 = n_tile * Cfg::BN;
    const half_t *xl = p.x + static_cast<int64_t>(lane_idx) * p.L * p.cin;
    float16_t acc[Cfg::TM][Cfg::TN];
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::TN; ++j) acc[i][j] = float16_t{};
    conv_snake_table<Cfg>(smem, n0, p.a_out, p.r_out);
    conv_mainloop<Cfg, SNAKE_IN, KT>(p, xl, l0, n0, smem, acc);
    conv_epilogue<Cfg>(acc, smem, static_cast<int64_t>(lane_idx) * p.L, l0, n0, p.L, p.cout, p.bias, p.res, p.y_pre,
                       p.y, p.a_out, p.act, p.scale);
}

// Any shape: one thread per output element, taps and channels looped directly. For shapes the
// tiled kernel declines (channel counts off its tile, wide halos, a single output channel).
__global__ __launch_bounds__(256) void conv_nlc_f16_direct(ConvParams p, int64_t total) {
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int n = static_cast<int>(e % p.cout);
        const int64_t row = e / p.cout;  // lane * L + l
        const int l = static_cast<int>(row % p.L);
        const int64_t lane_base = (row - l) * p.cin;
        float acc = 0.0f;
        const int64_t K = int64_t(p.k) * p.cin;
        for (int t = 0; t < p.k; ++t) {
            const int s = l + t * p.dil - p.pad_left;
            if (s < 0 || s >= p.L) continue;
            const half_t *xr = p.x + lane_base + int64_t(s) * p.cin;
            const half_t *wr = p.w + int64_t(n) * K + int64_t(t) * p.cin;
            for (int c = 0; c < p.cin; ++c) {
                float xv = static_cast<float>(xr[c]);
                if (p.a_in) xv = static_cast<float>(static_cast<half_t>(snake_f16out(xv, p.a_in[c], p.r_in[c])));
                acc += xv * static_cast<float>(wr[c]);
            }
        }
        const float v = conv_sum(acc, p.bias ? static_cast<float>(p.bias[n]) : 0.0f, p.scale, n,
                                 p.res ? static_cast<float>(p.res[e]) : 0.0f);
        half_t h = static_cast<half_t>(conv_act(v, p.act));
        if (p.y_pre) p.y_pre[e] = h;
        if (p.a_out) h = static_cast<half_t>(snake_f16out(static_cast<float>(h), p.a_out[n], p.r_out[n]));
        p.y[e] = h;
    }
}

template <typename Cfg>
hipError_t launch_tiled(const ConvParams &p0, int64_t lanes, hipStream_t stream) {
    ConvParams p = p0;
    p.tiles_m = (p.L + Cfg::BM - 1) / Cfg::BM;
    p.tiles_n = p.cout / Cfg::BN;
    if (p.tiles_ng <= 0) p.tiles_ng = pick_tiles_ng(p.tiles_n, int64_t(Cfg::BN) * p.k * p.cin * 2);
    const int64_t total = lanes * p.tiles_m * p.tiles_n;
    p.total_tiles = static_cast<int>(total);
    p.tiles_per_xcd = static_cast<int>((total + 7) / 8);
    const unsigned grid = static_cast<unsigned>(int64_t(p.tiles_per_xcd) * 8);
    // taps fixed at compile time when the shape fills the class's KMAX (k = 7, 2, 1)
    if (p.k == Cfg::KMAX) {
        if (p.a_in)
            conv_nlc_f16_mfma<Cfg, true, Cfg::KMAX><<<grid, Cfg::THREADS, 0, stream>>>(p);
        else
            conv_nlc_f16_mfma<Cfg, false, Cfg::KMAX><<<grid, Cfg::THREADS, 0, stream>>>(p);
    } else {
        if (p.a_in)
            conv_nlc_f16_mfma<Cfg, true, 0><<<grid, Cfg::THREADS, 0, stream>>>(p);
        else
            conv_nlc_f16_mfma<Cfg, false, 0><<<grid, Cfg::THREADS, 0, stream>>>(p);
    }
    return hipGetLastError();
}

template <typename Cfg>
struct Tile {
    typedef Cfg type;
};

// The one place a (taps, halo, length, cin, cout) class is mapped to its tile: launches and kernel
// names both go through it. f is called with Tile<Cfg>. `direct` says the shape's byte offsets
// fit the direct-staging buffer loads. Every tile needs cin % KC == 0 (the caller guarantees
// cin % 32 == 0) and cout % BN == 0.
template <int KMAX, int HMAX, typename F>
auto with_tile(int64_t lanes, int len, int cin, int cout, bool direct, F &&f) {
    if (direct) {
        // k <= 7 (dilated) at 96-multiples: eight waves of 64 x 96; short sequences take 256-row
        // tiles (two workgroups per CU) so the last tile of a lane is not mostly padding
        if constexpr (KMAX == 7) {
            if (cout % 96 == 0 && len >= 1024) return f(Tile<ConvTile<512, 96, 8, 1, 32, KMAX, HMAX, 2, kStageDirect>>{});
            if (cout % 96 == 0) return f(Tile<ConvTile<256, 96, 4, 1, 16, KMAX, HMAX, 2, kStageDirect>>{});
        }
        // k = 2 (the transposed convs) at 128-multiples: 2 x 2 waves of 128 x 64 when the input is
        // wide (cin >= 768: more matrix work per staged chunk), else 2 x 2 waves of 64 x 64; at
        // 96-multiples four waves of 32 x 96. Two 32-channel stages: with the epilogue's plain form
        // the smaller footprint (more workgroups per CU) beats a third stage in flight, 9% at
        // 128 x 128 and 16% at 128 x 96 on the codec's shapes (A/B; three stages stay better for
        // k = 1). Measured on the codec's four upsampling shapes: 10-20% over one 256 x 96 tile.
        if constexpr (KMAX == 2) {
            if (cout % 128 == 0 && cin >= 768) return f(Tile<ConvTile<256, 128, 2, 2, 32, KMAX, HMAX, 2, kStageDirect>>{});
            if (cout % 128 == 0) return f(Tile<ConvTile<128, 128, 2, 2, 32, KMAX, HMAX, 2, kStageDirect>>{});
            if (cout % 96 == 0) return f(Tile<ConvTile<128, 96, 4, 1, 32, KMAX, HMAX, 2, kStageDirect>>{});
        }
        // k = 1 at 128-multiples: 2 x 2 waves of 64 x 64. Three 32-channel stages in flight (three
        // workgroups per CU) up to cin 2048; beyond, two 64-channel stages (fewer barriers per
        // output). When that leaves fewer than 1024 tiles, 64-channel-wide tiles instead, to fill
        // the 256 CUs. k = 1 at 192-multiples otherwise: 256 x 192 over eight waves.
        if constexpr (KMAX == 1) {
            const int64_t tiles128 = lanes * ((len + 127) / 128) * (cout / 128);
            if (cout % 64 == 0 && cin % 64 == 0 && (cout % 128 != 0 || tiles128 < 1024))
                return f(Tile<ConvTile<128, 64, 2, 2, 64, KMAX, HMAX, 2, kStageDirect>>{});
            if (cout % 128 == 0 && cin % 64 == 0 && cin > 2048)
                return f(Tile<ConvTile<128, 128, 2, 2, 64, KMAX, HMAX, 2, kStageDirect>>{});
            if (cout % 128 == 0) return f(Tile<ConvTile<128, 128, 2, 2, 32, KMAX, HMAX, 3, kStageDirect>>{});
            if (cout % 192 == 0 && cin % 64 == 0)
                return f(Tile<ConvTile<256, 192, 4, 2, 64, KMAX, HMAX, 2, kStageDirect>>{});
        }
    }
    if (cout % 96 == 0) return f(Tile<ConvTile<256, 96, 4, 1, 32, KMAX, HMAX>>{});
    if (cout % 64 == 0) return f(Tile<ConvTile<256, 64, 4, 1, 32, KMAX, HMAX>>{});
    return f(Tile<ConvTile<256, 32, 4, 1, 32, KMAX, HMAX>>{});
}

template <typename F>
auto with_tile_k(int kmax, int64_t lanes, int len, int cin, int cout, bool direct, F &&f) {
    if (kmax == 1) return with_tile<1, 0>(lanes, len, cin, cout, direct, f);
    if (kmax == 2) return with_tile<2, 8>(lanes, len, cin, cout, direct, f);
    return with_tile<7, 64>(lanes, len, cin, cout, direct, f);
}

}  // namespace

namespace {

// Which kernel a descriptor runs on.
struct Choice {
    const char *path;  // "narrow", "mfma" or "direct"
    int kmax, hmax;
    bool snake;
    bool direct_ok;  // byte offsets fit direct-staging buffer loads
};

Choice choose(const dtts_conv_desc *d) {
    Choice c{"direct", 0, 0, d->in_alpha != nullptr, direct_offsets_fit(d->len, d->cin, d->cout, d->k)};
    if (conv_narrow_eligible(d) && d->act != 2 && !d->out_scale) {
        c.path = "narrow";
        return c;
    }
    const int64_t halo = (d->k - 1) * d->dilation;
    const bool aligned16 = aligned(d->x, 16) && aligned(d->w, 16) && aligned(d->y, 16) &&
                           (!d->bias || aligned(d->bias, 16)) && (!d->residual || aligned(d->residual, 16)) &&
                           (!d->y_pre || aligned(d->y_pre, 16)) && (!d->out_scale || aligned(d->out_scale, 16));
    // the tile epilogue addresses a lane's output rows (len x cout halves) as one buffer range
    if (!aligned16 || d->cin % 32 != 0 || d->cout % 32 != 0 || d->k > 7 || d->len * d->cout * 2 >= (int64_t(1) << 31))
        return c;
    if (d->k == 1) {
        c.kmax = 1;
        c.hmax = 0;
    } else if (d->k <= 2 && halo <= 8) {
        c.kmax = 2;
        c.hmax = 8;
    } else if (halo <= 64) {
        c.kmax = 7;
        c.hmax = 64;
    } else {
        return c;
    }
    c.path = "mfma";
    return c;
}

}  // namespace

const char *conv_path_name(const dtts_conv_desc *d) { return choose(d).path; }

const char *conv_kernel_name(const dtts_conv_desc *d) {
    static thread_local char buf[128];
    const Choice c = choose(d);
    if (std::strcmp(c.path, "mfma") == 0)
        with_tile_k(c.kmax, d->lanes, static_cast<int>(d->len), static_cast<int>(d->cin), static_cast<int>(d->cout), c.direct_ok,
                    [&](auto t) {
            typedef typename decltype(t)::type Cfg;
            char tail[32];
            snprintf(tail, sizeof(tail), ", %s, %d>", c.snake ? "true" : "false", d->k == Cfg::KMAX ? Cfg::KMAX : 0);
            return tile_kernel_name<Cfg>(buf, sizeof(buf), "conv_nlc_f16_mfma", tail);
        });
    else if (std::strcmp(c.path, "narrow") == 0)
        snprintf(buf, sizeof(buf), "%s", conv_narrow_kernel_name(d));
    else
        snprintf(buf, sizeof(buf), "conv_nlc_f16_%s", c.path);
    return buf;
}

int conv1d_nlc_f16(const dtts_conv_desc *d, hipStream_t stream) {
    const char *name = "dtts_conv1d_nlc_f16";
    DTTS_REQUIRE(d, "%s: null descriptor", name);
    DTTS_REQUIRE(d->lanes >= 0 && d->len >= 0 && d->cin > 0 && d->cout > 0 && d->k > 0 &&
                     d->dilation > 0 && d->pad_left >= 0,
                 "%s: bad shape (lanes %lld, len %lld, cin %lld, cout %lld, k %lld, dil %lld, pad %lld)",
                 name, (long long)d->lanes, (long long)d->len, (long long)d->cin, (long long)d->cout,
                 (long long)d->k, (long long)d->dilation, (long long)d->pad_left);
    DTTS_REQUIRE(d->pad_left <= (d->k - 1) * d->dilation,
                 "%s: pad_left %lld exceeds the receptive field (k-1)*dil = %lld", name,
                 (long long)d->pad_left, (long long)((d->k - 1) * d->dilation));
    DTTS_REQUIRE(d->act >= 0 && d->act <= 3, "%s: act %d unknown", name, d->act);
    if (d->lanes == 0 || d->len == 0) return DTTS_OK;
    DTTS_REQUIRE(d->x && d->w && d->y, "%s: null x, w or y", name);
    DTTS_REQUIRE((d->in_alpha == nullptr) == (d->in_brecip == nullptr), "%s: in_alpha and in_brecip go together", name);
    DTTS_REQUIRE((d->out_alpha == nullptr) == (d->out_brecip == nullptr), "%s: out_alpha and out_brecip go together", name);
    DTTS_REQUIRE(d->lanes * d->len * d->cout < (int64_t(1) << 40) && d->cin * d->k < (int64_t(1) << 30) &&
                     d->len < (int64_t(1) << 30) && d->cout < (int64_t(1) << 30),
                 "%s: shape too large", name);

    ConvParams p{};
    p.x = reinterpret_cast<const half_t *>(d->x);
    p.w = reinterpret_cast<const half_t *>(d->w);
    p.bias = reinterpret_cast<const half_t *>(d->bias);
    p.a_in = d->in_alpha;
    p.r_in = d->in_brecip;
    p.res = reinterpret_cast<const half_t *>(d->residual);
    p.y_pre = reinterpret_cast<half_t *>(d->y_pre);
    p.y = reinterpret_cast<half_t *>(d->y);
    p.a_out = d->out_alpha;
    p.r_out = d->out_brecip;
    p.L = static_cast<int>(d->len);
    p.cin = static_cast<int>(d->cin);
    p.cout = static_cast<int>(d->cout);
    p.k = static_cast<int>(d->k);
    p.dil = static_cast<int>(d->dilation);
    p.pad_left = static_cast<int>(d->pad_left);
    p.act = d->act;
    p.scale = d->out_scale;

    const Choice ch = choose(d);
    hipError_t e;
    if (std::strcmp(ch.path, "narrow") == 0) {
        DTTS_REQUIRE(d->lanes * ((d->len + 255) / 256) < (int64_t(1) << 31), "%s: too many tiles", name);
        e = conv_narrow_launch(d, stream);
    } else if (std::strcmp(ch.path, "mfma") == 0) {
        DTTS_REQUIRE(d->lanes * ((d->len + 255) / 256) * (d->cout / 32) < (int64_t(1) << 31),
                     "%s: too many tiles", name);
        e = with_tile_k(ch.kmax, d->lanes, p.L, p.cin, p.cout, ch.direct_ok, [&](auto t) {
            return launch_tiled<typename decltype(t)::type>(p, d->lanes, stream);
        });
    } else {
        const int64_t total = d->lanes * d->len * d->cout;
        conv_nlc_f16_direct<<<grid_for(total, 256, 16), 256, 0, stream>>>(p, total);
        e = hipGetLastError();
    }
    DTTS_HIP_CHECK(e, name);
    return DTTS_OK;
}

}  // namespace dtts

extern "C" int dtts_conv1d_nlc_f16_ex(const dtts_conv_desc *desc, hipStream_t stream) {
    return dtts::conv1d_nlc_f16(desc, stream);
}

extern "C" int dtts_causal_conv1d_nlc_f16(const dtts_f16 *x, const dtts_f16 *w_tm, const dtts_f16 *bias,
                                          dtts_f16 *y, int64_t lanes, int64_t len, int64_t cin,
                                          int64_t cout, int64_t k, int64_t dilation, hipStream_t stream) {
    dtts_conv_desc d{};
    d.lanes = lanes;
    d.len = len;
    d.cin = cin;
    d.cout = cout;
    d.k = k;
    d.dilation = dilation;
    d.pad_left = (k - 1) * dilation;
    d.x = x;
    d.w = w_tm;
    d.bias = bias;
    d.y = y;
    return dtts::conv1d_nlc_f16(&d, stream);
}

extern "C" int dtts_snake_conv_residual_nlc_f16(const dtts_f16 *x, const dtts_f16 *w_tm, const dtts_f16 *bias,
                                                int64_t dilation, const float *alpha, const float *brecip,
                                                const dtts_f16 *residual, dtts_f16 *y, int64_t lanes,
                                                int64_t len, int64_t cin, int64_t cout, int64_t k,
                                                hipStream_t stream) {
    dtts_conv_desc d{};
    d.lanes = lanes;
    d.len = len;
    d.cin = cin;
    d.cout = cout;
    d.k = k;
    d.dilation = dilation;
    d.pad_left = (k - 1) * dilation;
    d.x = x;
    d.w = w_tm;
    d.bias = bias;
    d.in_alpha = alpha;
    d.in_brecip = brecip;
    d.residual = residual;
    d.y = y;
    if (!alpha || !brecip || !residual) {
        dtts::set_error("dtts_snake_conv_residual_nlc_f16: alpha, brecip and residual are required");
        return DTTS_ERR_INVALID;
    }
    return dtts::conv1d_nlc_f16(&d, stream);
}
