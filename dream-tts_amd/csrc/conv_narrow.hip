// Channels-last conv with a single output channel (the codec's 96 -> 1 waveform conv).
//
// HBM-bound: every input element is read once and feeds k products. A workgroup stages a
// window of BM + (k-1)*dil positions x cin channels in LDS (row pitch padded by 8 halves so 16
// consecutive rows hit 16 disjoint bank quads), then each thread reduces one output position
// over k taps x cin channels (LDS sized per launch) with packed f16 dot products accumulating in f32.
#include "conv.hpp"
#include "snake.hpp"

namespace dtts {
namespace {

constexpr int kBM = 256;
constexpr int kMaxCin = 128;
constexpr int kMaxHalo = 64;
constexpr int kMaxVec = (kBM + kMaxHalo) * (kMaxCin / 8) / 256;  // window vectors per thread, at most

struct NarrowParams {
    const half_t *x;
    const half_t *w;  // [k * cin]
    const half_t *bias;
    const float *a_in;
    const float *r_in;
    const half_t *res;
    half_t *y_pre;
    half_t *y;
    const float *a_out;
    const float *r_out;
    int L, cin, k, dil, pad_left, act, tiles_m;
};

__global__ __launch_bounds__(256) void conv_nlc_f16_narrow(NarrowParams p) {
    extern __shared__ __attribute__((aligned(16))) char dyn[];
    const int pitch = p.cin + 8;
    const int rows = kBM + (p.k - 1) * p.dil;
    half_t *win = reinterpret_cast<half_t *>(dyn);
    half_t *wsh = win + rows * pitch;
    const int lane_idx = blockIdx.x / p.tiles_m;
    const int l0 = (blockIdx.x - lane_idx * p.tiles_m) * kBM;
    const int cv = p.cin / 8;  // 16-byte vectors per row
    const half_t *xl = p.x + static_cast<int64_t>(lane_idx) * p.L * p.cin;
    for (int i = threadIdx.x; i < p.k * p.cin; i += 256) wsh[i] = p.w[i];
    // every 16-byte vector of the window is loaded before any is stored, so the loads' latencies
    // overlap instead of adding up
    const int nvec = rows * cv;
    half8_t buf[kMaxVec];
#pragma unroll
    for (int i = 0; i < kMaxVec; ++i) {
        const int v = threadIdx.x + i * 256;
        buf[i] = half8_t{};
        if (v < nvec) {
            const int r = v / cv;
            const int s = l0 - p.pad_left + r;
            if (s >= 0 && s < p.L)
                buf[i] = *reinterpret_cast<const half8_t *>(xl + static_cast<int64_t>(s) * p.cin + (v - r * cv) * 8);
        }
    }
#pragma unroll
    for (int i = 0; i < kMaxVec; ++i) {
        const int v = threadIdx.x + i * 256;
        if (v < nvec) {
            const int r = v / cv;
            const int q = v - r * cv;
            half8_t h = buf[i];
            if (p.a_in) {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    h[j] = static_cast<half_t>(snake_f16out(static_cast<float>(h[j]), p.a_in[q * 8 + j], p.r_in[q * 8 + j]));
            }
            *reinterpret_cast<half8_t *>(win + r * pitch + q * 8) = h;
        }
    }
    __syncthreads();
    const int l = l0 + threadIdx.x;
    if (l >= p.L) return;
    float acc = 0.0f;
    for (int t = 0; t < p.k; ++t) {
        const half_t *row = win + (threadIdx.x + t * p.dil) * pitch;
        const half_t *wr = wsh + t * p.cin;
        for (int q = 0; q < cv; ++q) {
            const half8_t xv = *reinterpret_cast<const half8_t *>(row + q * 8);
            const half8_t wv = *reinterpret_cast<const half8_t *>(wr + q * 8);
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const half2_t a = {xv[j], xv[j + 1]};
                const half2_t b = {wv[j], wv[j + 1]};
                acc = __builtin_amdgcn_fdot2(a, b, acc, false);
            }
        }
    }
    const int64_t off = static_cast<int64_t>(lane_idx) * p.L + l;
    float v = acc;
    if (p.bias) v += static_cast<float>(p.bias[0]);
    if (p.res) v += static_cast<float>(p.res[off]);
    if (p.act == 1) v = tanhf(v);
    if (p.act == 3) v = fminf(fmaxf(v, -1.0f), 1.0f);
    half_t h = static_cast<half_t>(v);
    if (p.y_pre) p.y_pre[off] = h;
    if (p.a_out) h = static_cast<half_t>(snake_f16out(static_cast<float>(h), p.a_out[0], p.r_out[0]));
    p.y[off] = h;
}

}  // namespace

bool conv_narrow_eligible(const dtts_conv_desc *d) {
    return d->cout == 1 && d->cin % 8 == 0 && d->cin <= kMaxCin && d->k <= 7 &&
           (d->k - 1) * d->dilation <= kMaxHalo && aligned(d->x, 16) && aligned(d->w, 16);
}

hipError_t conv_narrow_launch(const dtts_conv_desc *d, hipStream_t stream) {
    NarrowParams p{};
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
    p.k = static_cast<int>(d->k);
    p.dil = static_cast<int>(d->dilation);
    p.pad_left = static_cast<int>(d->pad_left);
    p.act = d->act;
    p.tiles_m = static_cast<int>((d->len + kBM - 1) / kBM);
    const int64_t grid = d->lanes * p.tiles_m;
    const size_t lds = (static_cast<size_t>(kBM + (p.k - 1) * p.dil) * (p.cin + 8) + static_cast<size_t>(p.k) * p.cin) * 2;
    conv_nlc_f16_narrow<<<static_cast<unsigned>(grid), 256, lds, stream>>>(p);
    return hipGetLastError();
}

}  // namespace dtts
