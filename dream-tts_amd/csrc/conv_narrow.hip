// Channels-last conv with a single output channel (the codec's 96 -> 1 waveform conv).
//
// HBM-bound: every input element is read once and feeds k products. A workgroup owns kBM
// positions of one lane, a thread one position. Per 32-channel chunk the window (kBM + (k-1)*dil
// rows) goes through registers into LDS (the prologue SnakeBeta applied on the way), rows 40
// halves apart so the 16-byte reads of 16 consecutive rows hit 16 disjoint bank quads. Packed f16
// dot products accumulate in f32, in (chunk, tap, channel) order.
//
// Two kernels share that order, so their outputs agree bit for bit:
//   conv_nlc_f16_narrow_k<K, SNAKE>  k = K (7: the codec's), 32-channel multiples, the prologue
//       SnakeBeta optional. The next chunk's window is loaded into registers while the current
//       one is on the dot products, into the other of two LDS windows (one barrier per chunk); the
//       weights are uniform loads (scalar registers). ~51 KB of LDS: three workgroups per CU.
//   conv_nlc_f16_narrow       any k <= 7, 8-channel multiples, optional prologue SnakeBeta: one
//       window, loaded, stored and consumed a chunk at a time, the chunk's weights in LDS.
// Both apply the prologue SnakeBeta through snake_f16out, as the standalone snake does.
#include "conv.hpp"
#include "snake.hpp"

namespace dtts {
namespace {

constexpr int kBM = 256;
constexpr int kKC = 32;                // channels per chunk
constexpr int kPitch = kKC + 8;        // LDS row pitch, halves
constexpr int kMaxHalo = 64;
constexpr int kRows = kBM + kMaxHalo;
constexpr int kMaxVec = (kRows * (kKC / 8) + 255) / 256;  // window vectors per thread, at most

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

// The epilogue both kernels share: bias, residual, activation, f16 rounding, the optional plain
// store and output SnakeBeta.
__device__ __forceinline__ void narrow_store(const NarrowParams &p, int lane_idx, int l, float acc) {
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

__global__ __launch_bounds__(256) void conv_nlc_f16_narrow(NarrowParams p) {
    __shared__ __attribute__((aligned(16))) half_t win[kRows * kPitch];
    __shared__ __attribute__((aligned(16))) half_t wsh[7 * kKC];
    const int lane_idx = blockIdx.x / p.tiles_m;
    const int l0 = (blockIdx.x - lane_idx * p.tiles_m) * kBM;
    const int rows = kBM + (p.k - 1) * p.dil;
    const half_t *xl = p.x + static_cast<int64_t>(lane_idx) * p.L * p.cin;
    const int tid = threadIdx.x;
    float acc = 0.0f;
    for (int c0 = 0; c0 < p.cin; c0 += kKC) {
        const int cv = (p.cin - c0 < kKC ? p.cin - c0 : kKC) / 8;  // 16-byte vectors per row in this chunk
        const int nvec = rows * cv;
        // every vector of the chunk's window is loaded before any is stored, so the loads'
        // latencies overlap instead of adding up
        half8_t buf[kMaxVec];
#pragma unroll
        for (int i = 0; i < kMaxVec; ++i) {
            const int v = tid + i * 256;
            buf[i] = half8_t{};
            const int r = v / cv;
            const int s = l0 - p.pad_left + r;
            if (v < nvec && s >= 0 && s < p.L)
                buf[i] = *reinterpret_cast<const half8_t *>(xl + static_cast<int64_t>(s) * p.cin + c0 + (v - r * cv) * 8);
        }
        if (c0 > 0) __syncthreads();  // every thread is done with the previous chunk's window and weights
        if (tid < p.k * cv * 8) {
            const int t = tid / (cv * 8), c = tid - t * (cv * 8);
            wsh[t * kKC + c] = p.w[t * p.cin + c0 + c];
        }
#pragma unroll
        for (int i = 0; i < kMaxVec; ++i) {
            const int v = tid + i * 256;
            if (v < nvec) {
                const int r = v / cv;
                const int q = v - r * cv;
                half8_t h = buf[i];
                if (p.a_in) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int c = c0 + q * 8 + j;
                        h[j] = static_cast<half_t>(snake_f16out(static_cast<float>(h[j]), p.a_in[c], p.r_in[c]));
                    }
                }
                *reinterpret_cast<half8_t *>(win + r * kPitch + q * 8) = h;
            }
        }
        __syncthreads();
        for (int t = 0; t < p.k; ++t) {
            const half_t *row = win + (tid + t * p.dil) * kPitch;
            const half_t *wr = wsh + t * kKC;
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
    }
    const int l = l0 + tid;
    if (l < p.L) narrow_store(p, lane_idx, l, acc);
}

template <int K, bool SNAKE>
__global__ __launch_bounds__(256) void conv_nlc_f16_narrow_k(NarrowParams p) {
    constexpr int SEGS = kKC / 8;
    constexpr int NVEC = (kRows * SEGS + 255) / 256;
    __shared__ __attribute__((aligned(16))) half_t win[2][kRows * kPitch];
    const int lane_idx = blockIdx.x / p.tiles_m;
    const int l0 = (blockIdx.x - lane_idx * p.tiles_m) * kBM;
    const int nvec = (kBM + (K - 1) * p.dil) * SEGS;
    const half_t *xl = p.x + static_cast<int64_t>(lane_idx) * p.L * p.cin;
    const half_t *__restrict__ w = p.w;
    const int tid = threadIdx.x;
    half8_t buf[NVEC];
    auto load = [&](int c0) {
#pragma unroll
        for (int i = 0; i < NVEC; ++i) {
            const int v = tid + i * 256;
            const int r = v / SEGS;
            const int s = l0 - p.pad_left + r;
            buf[i] = half8_t{};
            if (v < nvec && s >= 0 && s < p.L)
                buf[i] = *reinterpret_cast<const half8_t *>(xl + static_cast<int64_t>(s) * p.cin + c0 + (v % SEGS) * 8);
        }
    };
    float acc = 0.0f;
    load(0);
    int st = 0;
    for (int c0 = 0; c0 < p.cin; c0 += kKC, st ^= 1) {
        // the thread's 8 channels of this chunk (segment tid % SEGS of every row it stages)
        float ka[8], kr[8];
        if constexpr (SNAKE) {
            const int c = c0 + (tid % SEGS) * 8;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                ka[j] = p.a_in[c + j];
                kr[j] = p.r_in[c + j];
            }
        }
        // window st was last read two chunks ago, before the barrier that closed the last chunk
#pragma unroll
        for (int i = 0; i < NVEC; ++i) {
            const int v = tid + i * 256;
            if (v < nvec) {
                half8_t h = buf[i];
                if constexpr (SNAKE) {
                    // rows outside the sequence hold 0, which SnakeBeta keeps 0
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        h[j] = static_cast<half_t>(snake_f16out(static_cast<float>(h[j]), ka[j], kr[j]));
                }
                *reinterpret_cast<half8_t *>(win[st] + (v / SEGS) * kPitch + (v % SEGS) * 8) = h;
            }
        }
        if (c0 + kKC < p.cin) load(c0 + kKC);
        __syncthreads();
#pragma unroll
        for (int t = 0; t < K; ++t) {
            const half_t *row = win[st] + (tid + t * p.dil) * kPitch;
#pragma unroll
            for (int q = 0; q < SEGS; ++q) {
                const half8_t xv = *reinterpret_cast<const half8_t *>(row + q * 8);
                const half8_t wv = *reinterpret_cast<const half8_t *>(w + t * p.cin + c0 + q * 8);
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    const half2_t a = {xv[j], xv[j + 1]};
                    const half2_t b = {wv[j], wv[j + 1]};
                    acc = __builtin_amdgcn_fdot2(a, b, acc, false);
                }
            }
        }
    }
    const int l = l0 + tid;
    if (l < p.L) narrow_store(p, lane_idx, l, acc);
}

// The specialised kernel's shapes: k = 7, 32-channel multiples, 16-byte weight rows.
bool narrow_k7(const dtts_conv_desc *d) { return d->k == 7 && d->cin % kKC == 0 && aligned(d->w, 16); }

}  // namespace

const char *conv_narrow_kernel_name(const dtts_conv_desc *d) {
    if (!narrow_k7(d)) return "conv_nlc_f16_narrow";
    return d->in_alpha ? "conv_nlc_f16_narrow_k<7, true>" : "conv_nlc_f16_narrow_k<7, false>";
}

bool conv_narrow_eligible(const dtts_conv_desc *d) {
    return d->cout == 1 && d->cin % 8 == 0 && d->k <= 7 && (d->k - 1) * d->dilation <= kMaxHalo &&
           aligned(d->x, 16);
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
    if (narrow_k7(d) && d->in_alpha)
        conv_nlc_f16_narrow_k<7, true><<<static_cast<unsigned>(grid), 256, 0, stream>>>(p);
    else if (narrow_k7(d))
        conv_nlc_f16_narrow_k<7, false><<<static_cast<unsigned>(grid), 256, 0, stream>>>(p);
    else
        conv_nlc_f16_narrow<<<static_cast<unsigned>(grid), 256, 0, stream>>>(p);
    return hipGetLastError();
}

}  // namespace dtts
