// Channel-major f32 conv1d (the reference's NCL route, crates/tts-nn/src/lib.rs:704-860) as an
// implicit GEMM on the f32 matrix cores, and the tap-major im2col gather it replaces.
//
//   y[b, n, l] = act(bias[n] + res[b, n, l] + sum_t sum_c w[n, t*cin + c] * xs[b, c, l + t*dil - pad_left])
//
// xs is x or SnakeBeta(x) (full-precision sinf; f32 outputs are held to 1e-5). GEMM view per
// lane: M = output channels, N = positions, K = (tap, channel). A workgroup owns 64 channels x
// 64 positions; per KC-channel chunk (8 for k = 7, 16 for k = 1) it stages the dilated window of
// x position-major (64 + (k-1)*dil rows of KC channels, transposed as it is stored) and the
// 64 x k x KC weight slice in LDS (two buffers, the next chunk prefetched through registers),
// then four waves (2 x 2) run v_mfma_f32_32x32x2_f32, each tap reading the window at row offset
// t*dil. MFMA step s pairs channel s (lanes 0-31) with channel KC/2 + s (lanes 32-63), so a
// lane's operands of a tap are consecutive floats of one row: 16-byte LDS reads for both the
// weights and the window; with k = KMAX the taps are unrolled and tap t+1's reads issue under
// tap t's MFMAs. The epilogue writes straight from the accumulators: the 32 lanes of a C column
// are 32 consecutive positions.
#include "conv.hpp"
#include "snake.hpp"

namespace dtts {
namespace {

struct NclParams {
    const float *x, *w, *bias, *a_in, *r_in, *res;
    float *y_pre, *y;
    const float *a_out, *r_out;
    int L, cin, cout, k, dil, pad_left, act;
    int tiles_m, tiles_n, total, per_xcd;
};

constexpr int kBM = 64, kBN = 64;

// One workgroup = 64 output channels x 64 positions of one lane; four waves (2 x 2), each one
// 32 x 32 accumulator block. Per KC-channel chunk the window (64 + (k-1)*dil positions x KC
// channels, SnakeBeta applied as it is staged) and the 64 x k x KC weight slice sit in one of two
// LDS buffers: chunk c+1 is stored from registers into the other buffer while chunk c+2 is
// loaded into registers and chunk c is multiplied, one barrier per chunk. KT = KMAX when k fills
// the class (taps unrolled), 0 for fewer taps.
template <int KMAX, int HMAX, int KT, int KC, bool SNAKE>
__global__ __launch_bounds__(256, 2) void conv_ncl_f32_mfma(NclParams p) {
    constexpr int XR = kBN + HMAX;                             // window positions
    constexpr int XP = KC + 4;                                 // window row (one position) pitch, floats
    constexpr int WP = KMAX * KC + 4;                          // weight row pitch: 16-byte aligned rows
    constexpr int C4 = KC / 4;
    constexpr int XE = (KC * XR + 255) / 256;                  // window elements per thread
    constexpr int WV = (kBM * KMAX * C4 + 255) / 256;          // weight float4s per thread
    constexpr int H = KC / 2, HV = H / 4;                      // MFMA steps per tap, float4s per operand
    static_assert(KC % 8 == 0, "chunk width");
    __shared__ __attribute__((aligned(16))) float xs[2][XR * XP];
    __shared__ __attribute__((aligned(16))) float ws[2][kBM * WP];
    const int tile = (blockIdx.x & 7) * p.per_xcd + (blockIdx.x >> 3);
    if (tile >= p.total) return;
    const int m_tile = tile % p.tiles_m;  // output channels fastest: neighbours share the window
    const int rest = tile / p.tiles_m;
    const int n_tile = rest % p.tiles_n;
    const int lane_idx = rest / p.tiles_n;
    const int co0 = m_tile * kBM;
    const int l0 = n_tile * kBN;
    const int k = KT > 0 ? KT : p.k;
    const int rows = kBN + (k - 1) * p.dil;
    const int K = k * p.cin;
    const float *xl = p.x + static_cast<int64_t>(lane_idx) * p.cin * p.L;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int kh = lane >> 5, lr = lane & 31;
    const int nx = KC * rows, nw = kBM * k * C4;

    float xr[XE];
    float4_t wr[WV];
    auto load = [&](int c0) {
        // window: element e is channel e / rows at position e % rows, so consecutive threads read
        // consecutive positions of one channel row
#pragma unroll
        for (int i = 0; i < XE; ++i) {
            const int e = tid + i * 256;
            const int ci = e / rows, j = e - (e / rows) * rows;
            const int s = l0 - p.pad_left + j;
            float v = 0.0f;
            if (e < nx && s >= 0 && s < p.L) v = xl[static_cast<int64_t>(c0 + ci) * p.L + s];
            xr[i] = v;
        }
        // weights: KC consecutive input channels of one (output channel, tap) are KC/4 float4s
#pragma unroll
        for (int i = 0; i < WV; ++i) {
            const int e = tid + i * 256;
            const int m = e / (k * C4), q = e - (e / (k * C4)) * (k * C4);
            const int t = q / C4, c4 = q % C4;
            wr[i] = e < nw ? *reinterpret_cast<const float4_t *>(p.w + static_cast<int64_t>(co0 + m) * K + t * p.cin + c0 +
                                                               c4 * 4)
                           : float4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    };
    auto store = [&](int c0, int b) {
        if constexpr (SNAKE) {
            // the window's SnakeBeta as one group (alpha 0 leaves a padding or idle value as it is)
            float a[XE], r[XE];
#pragma unroll
            for (int i = 0; i < XE; ++i) {
                const int e = tid + i * 256;
                const int ci = e / rows, j = e - (e / rows) * rows;
                const int s = l0 - p.pad_left + j;
                const bool live = e < nx && s >= 0 && s < p.L;
                a[i] = live ? p.a_in[c0 + ci] : 0.0f;
                r[i] = live ? p.r_in[c0 + ci] : 0.0f;
            }
            snake_f32_group<XE>(xr, a, r);
        }
#pragma unroll
        for (int i = 0; i < XE; ++i) {
            const int e = tid + i * 256;
            if (e < nx) {
                const int ci = e / rows, j = e - (e / rows) * rows;
                xs[b][j * XP + ci] = xr[i];  // transposed: row = position
            }
        }
#pragma unroll
        for (int i = 0; i < WV; ++i) {
            const int e = tid + i * 256;
            if (e < nw) {
                const int m = e / (k * C4), q = e - (e / (k * C4)) * (k * C4);
                *reinterpret_cast<float4_t *>(&ws[b][m * WP + q * 4]) = wr[i];
            }
        }
    };

    float16_t acc = float16_t{};
    const int nchunks = p.cin / KC;
    load(0);
    store(0, 0);
    if (nchunks > 1) load(KC);
    __syncthreads();
    for (int c = 0; c < nchunks; ++c) {
        const int b = c & 1;
        if (c + 1 < nchunks) {
            store((c + 1) * KC, b ^ 1);  // that buffer was last read by chunk c-1, before the barrier
            if (c + 2 < nchunks) load((c + 2) * KC);
        }
        // A[m][kk] = w[co0 + m][tap t, channel kk]; B[kk][n] = window[position n + t*dil][channel kk]
        auto frag = [&](int t, float4_t (&fa)[HV], float4_t (&fb)[HV]) {
            const float *wa = ws[b] + (wm * 32 + lr) * WP + t * KC + kh * H;
            const float *xb = xs[b] + (wn * 32 + lr + t * p.dil) * XP + kh * H;
#pragma unroll
            for (int h = 0; h < HV; ++h) {
                fa[h] = *reinterpret_cast<const float4_t *>(wa + 4 * h);
                fb[h] = *reinterpret_cast<const float4_t *>(xb + 4 * h);
            }
        };
        auto mma = [&](const float4_t (&fa)[HV], const float4_t (&fb)[HV]) {
#pragma unroll
            for (int st = 0; st < H; ++st)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[st >> 2][st & 3], fb[st >> 2][st & 3], acc, 0, 0, 0);
        };
        if constexpr (KT > 0) {
            float4_t fa[2][HV], fb[2][HV];
            frag(0, fa[0], fb[0]);
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                if (t + 1 < KT) frag(t + 1, fa[(t + 1) & 1], fb[(t + 1) & 1]);
                mma(fa[t & 1], fb[t & 1]);
            }
        } else {
            for (int t = 0; t < k; ++t) {
                float4_t fa[HV], fb[HV];
                frag(t, fa, fb);
                mma(fa, fb);
            }
        }
        __syncthreads();
    }
    const int64_t ybase = static_cast<int64_t>(lane_idx) * p.cout * p.L;
    const int pos = l0 + wn * 32 + lr;
    if (pos >= p.L) return;
    // the block's residuals are requested together before its stores (res may alias the
    // outputs, so a load issued after a store would wait for it)
    float rv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int co = co0 + wm * 32 + (r >> 2) * 8 + kh * 4 + (r & 3);
        rv[r] = p.res ? p.res[ybase + static_cast<int64_t>(co) * p.L + pos] : 0.0f;
    }
    float v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int co = co0 + wm * 32 + (r >> 2) * 8 + kh * 4 + (r & 3);
        v[r] = acc[r];
        if (p.bias) v[r] += p.bias[co];
        if (p.res) v[r] += rv[r];
        if (p.act == 1) v[r] = tanhf(v[r]);
        if (p.y_pre) p.y_pre[ybase + static_cast<int64_t>(co) * p.L + pos] = v[r];
    }
    if (p.a_out) {
        float a[16], rr[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int co = co0 + wm * 32 + (r >> 2) * 8 + kh * 4 + (r & 3);
            a[r] = p.a_out[co];
            rr[r] = p.r_out[co];
        }
        snake_f32_group<16>(v, a, rr);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int co = co0 + wm * 32 + (r >> 2) * 8 + kh * 4 + (r & 3);
        p.y[ybase + static_cast<int64_t>(co) * p.L + pos] = v[r];
    }
}


__global__ __launch_bounds__(256) void conv_ncl_f32_direct(NclParams p, int64_t total) {
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int l = static_cast<int>(e % p.L);
        const int64_t bc = e / p.L;
        const int co = static_cast<int>(bc % p.cout);
        const int64_t b = bc / p.cout;
        const float *xl = p.x + b * p.cin * p.L;
        const float *wr = p.w + static_cast<int64_t>(co) * p.k * p.cin;
        float acc = 0.0f;
        for (int t = 0; t < p.k; ++t) {
            const int s = l + t * p.dil - p.pad_left;
            if (s < 0 || s >= p.L) continue;
            for (int c = 0; c < p.cin; ++c) {
                float v = xl[static_cast<int64_t>(c) * p.L + s];
                if (p.a_in) v = snake_f32(v, p.a_in[c], p.r_in[c]);
                acc += wr[t * p.cin + c] * v;
            }
        }
        float v = acc;
        if (p.bias) v += p.bias[co];
        if (p.res) v += p.res[e];
        if (p.act == 1) v = tanhf(v);
        if (p.y_pre) p.y_pre[e] = v;
        if (p.a_out) v = snake_f32(v, p.a_out[co], p.r_out[co]);
        p.y[e] = v;
    }
}

__global__ __launch_bounds__(256) void im2col_kernel(const float *x, float *cols, int cin, int L, int k, int dil,
                                                     int pad_left) {
    const int64_t total = static_cast<int64_t>(k) * cin * L;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int l = static_cast<int>(e % L);
        const int64_t row = e / L;  // t * cin + c
        const int t = static_cast<int>(row / cin);
        const int c = static_cast<int>(row - int64_t(t) * cin);
        const int s = l + t * dil - pad_left;
        cols[e] = (s >= 0 && s < L) ? x[static_cast<int64_t>(c) * L + s] : 0.0f;
    }
}

template <int KMAX, int HMAX, int KT, int KC>
hipError_t launch_ncl(NclParams p, int64_t lanes, bool snake, hipStream_t stream) {
    p.tiles_m = p.cout / kBM;
    p.tiles_n = (p.L + kBN - 1) / kBN;
    const int64_t total = lanes * p.tiles_m * p.tiles_n;
    p.total = static_cast<int>(total);
    p.per_xcd = static_cast<int>((total + 7) / 8);
    const unsigned grid = static_cast<unsigned>(int64_t(p.per_xcd) * 8);
    if (snake)
        conv_ncl_f32_mfma<KMAX, HMAX, KT, KC, true><<<grid, 256, 0, stream>>>(p);
    else
        conv_ncl_f32_mfma<KMAX, HMAX, KT, KC, false><<<grid, 256, 0, stream>>>(p);
    return hipGetLastError();
}

}  // namespace
}  // namespace dtts

extern "C" int dtts_conv1d_ncl_f32_ex(const dtts_conv_desc *d, hipStream_t stream) {
    const char *name = "dtts_conv1d_ncl_f32";
    DTTS_REQUIRE(d, "%s: null descriptor", name);
    DTTS_REQUIRE(d->lanes >= 0 && d->len >= 0 && d->cin > 0 && d->cout > 0 && d->k > 0 && d->dilation > 0 &&
                     d->pad_left >= 0 && d->pad_left <= (d->k - 1) * d->dilation,
                 "%s: bad shape or pad_left", name);
    DTTS_REQUIRE(d->act == 0 || d->act == 1, "%s: act %d unknown", name, d->act);
    if (d->lanes == 0 || d->len == 0) return DTTS_OK;
    DTTS_REQUIRE(d->x && d->w && d->y, "%s: null x, w or y", name);
    DTTS_REQUIRE((d->in_alpha == nullptr) == (d->in_brecip == nullptr) &&
                     (d->out_alpha == nullptr) == (d->out_brecip == nullptr),
                 "%s: snake alpha and brecip go together", name);
    DTTS_REQUIRE(d->lanes * d->cout * d->len < (int64_t(1) << 40) && d->len < (int64_t(1) << 30) &&
                     d->cin * d->k < (int64_t(1) << 30),
                 "%s: shape too large", name);
    dtts::NclParams p{};
    p.x = static_cast<const float *>(d->x);
    p.w = static_cast<const float *>(d->w);
    p.bias = static_cast<const float *>(d->bias);
    p.a_in = d->in_alpha;
    p.r_in = d->in_brecip;
    p.res = static_cast<const float *>(d->residual);
    p.y_pre = static_cast<float *>(d->y_pre);
    p.y = static_cast<float *>(d->y);
    p.a_out = d->out_alpha;
    p.r_out = d->out_brecip;
    p.L = static_cast<int>(d->len);
    p.cin = static_cast<int>(d->cin);
    p.cout = static_cast<int>(d->cout);
    p.k = static_cast<int>(d->k);
    p.dil = static_cast<int>(d->dilation);
    p.pad_left = static_cast<int>(d->pad_left);
    p.act = d->act;
    const int64_t halo = (d->k - 1) * d->dilation;
    hipError_t e;
    // the tile's classes: k = 1 on 16-channel chunks, k <= 7 on 8-channel chunks
    const int64_t kc = d->k == 1 ? 16 : 8;
    if (d->cin % kc == 0 && d->cout % dtts::kBM == 0 && d->k <= 7 && halo <= 64 && dtts::aligned(d->w, 16)) {
        DTTS_REQUIRE(d->lanes * (d->cout / dtts::kBM) * ((d->len + dtts::kBN - 1) / dtts::kBN) < (int64_t(1) << 31),
                     "%s: too many tiles", name);
        const bool snake = d->in_alpha != nullptr;
        if (d->k == 1)
            e = dtts::launch_ncl<1, 0, 1, 16>(p, d->lanes, snake, stream);
        else if (d->k == 7)
            e = dtts::launch_ncl<7, 64, 7, 8>(p, d->lanes, snake, stream);
        else
            e = dtts::launch_ncl<7, 64, 0, 8>(p, d->lanes, snake, stream);
    } else {
        const int64_t total = d->lanes * d->cout * d->len;
        dtts::conv_ncl_f32_direct<<<dtts::grid_for(total, 256, 16), 256, 0, stream>>>(p, total);
        e = hipGetLastError();
    }
    DTTS_HIP_CHECK(e, name);
    return DTTS_OK;
}

extern "C" int dtts_im2col_tap_major_f32(const float *x, float *cols, int64_t cin, int64_t len, int64_t k,
                                         int64_t dilation, int64_t pad_left, hipStream_t stream) {
    DTTS_REQUIRE(cin > 0 && len >= 0 && k > 0 && dilation > 0 && pad_left >= 0, "dtts_im2col_tap_major_f32: bad shape");
    if (len == 0) return DTTS_OK;
    DTTS_REQUIRE(x && cols, "dtts_im2col_tap_major_f32: null pointer");
    DTTS_REQUIRE(k * cin * len < (int64_t(1) << 40) && len < (int64_t(1) << 30) && k * cin < (int64_t(1) << 30),
                 "dtts_im2col_tap_major_f32: shape too large");
    dtts::im2col_kernel<<<dtts::grid_for(k * cin * len, 256), 256, 0, stream>>>(
        x, cols, static_cast<int>(cin), static_cast<int>(len), static_cast<int>(k), static_cast<int>(dilation),
        static_cast<int>(pad_left));
    DTTS_LAUNCH_CHECK("dtts_im2col_tap_major_f32");
    return DTTS_OK;
}
