// Channels-last f32 conv1d at NlcConv's own precision (crates/tts-nn/src/nlcconv.rs:15-198, its
// CPU form nlcconv.rs:33-73; kernel nlc_conv_f32, mtl.rs:937-1065), as an implicit GEMM on the f32
// matrix cores:
//
//   s[b, l, n] = bias[n] + sum_t sum_c xs[b, l + t*dil - pad_left, c] * w[n, t*cin + c]
//   y[b, l, n] = act(res[b, l, n] + scale[n] * s)         (scale 1 and res 0 when absent)
//
// xs is x, or SnakeBeta(x) applied as the window is staged (full-precision sinf; a padded tap
// stays 0, as snake(0) = 0 gives). GEMM view per lane: M = positions, N = output channels,
// K = (tap, channel). A workgroup owns BM positions x BN output channels of one lane: BN 64
// (k = 7: 256 positions over 4 x 2 waves of 64 x 32, four waves per SIMD; otherwise 128 over 2 x 2),
// 96 (128 over 4 x 1 waves of 32 x 96) or 32 (128 over 4 x 1 waves of 32 x 32), the widest BN that
// divides cout. Per KC-channel chunk (8; 16 at k = 1) it stages the dilated window
// (BM + (k-1)*dil rows) and the BN x k x KC weight slice in LDS (two buffers: chunk c+1 goes from
// registers into one while chunk c+2's loads are in flight and chunk c is multiplied, one barrier
// per chunk). The waves run
// v_mfma_f32_32x32x2_f32; step s of a tap pairs channel s (lanes 0-31) with channel KC/2 + s
// (lanes 32-63), so a lane's operands of a tap are 16-byte LDS reads (one per 32-row or 32-column
// block at KC = 8), and with k = KMAX the taps are unrolled and tap t+1's reads issue under tap
// t's MFMAs.
// The 32 lanes of an accumulator row are 32 consecutive output channels of one position, so the
// epilogue's loads and stores are 128-byte runs straight from the accumulators.
// A single output channel (the codec's 96 -> 1 output conv) runs a window kernel of its own;
// other shapes off the tile (channel counts not multiples of 8 / 32) run a direct kernel.
#include "conv.hpp"
#include "snake.hpp"

namespace dtts {
namespace {

struct NlcF32Params {
    const float *x, *w, *bias, *a_in, *r_in, *res, *scale;
    float *y_pre, *y;
    const float *a_out, *r_out;
    int L, cin, cout, k, dil, pad_left, act;
    int tiles_m, tiles_n, total, per_xcd;
};

constexpr int kF32KC = 8;

__device__ __forceinline__ float conv_f32_epilogue(float s, int co, int64_t off, const NlcF32Params &p) {
    float v = s;
    if (p.bias) v += p.bias[co];
    if (p.scale) v = p.scale[co] * v;
    if (p.res) v += p.res[off];
    if (p.act == 1) v = tanhf(v);
    if (p.act == 3) v = fminf(fmaxf(v, -1.0f), 1.0f);
    return v;
}

// BM x BN tile over WM x WN waves (wave tile (BM/WM) x (BN/WN) in 32 x 32 blocks); KT = KMAX when
// k fills the class (taps unrolled, the next tap's operands read under the current tap's MFMAs),
// 0 for fewer taps.
template <int KMAX, int HMAX, int KT, int BM, int BN, int WM, int WN, int KC, bool SNAKE>
__global__ __launch_bounds__(64 * WM * WN, WM * WN / 2) void conv_nlc_f32_mfma(NlcF32Params p) {
    constexpr int NT = 64 * WM * WN;
    constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 32, TN = WTN / 32;
    constexpr int XR = BM + HMAX;               // window rows
    constexpr int XP = KC + 4;                  // row pitch: 48 B, so 16 consecutive rows' 16-byte reads
    constexpr int WP = KMAX * KC + 4;           //   hit 16 distinct bank groups (likewise 16 * odd here)
    constexpr int C4 = KC / 4;                  // float4s per row of a chunk
    constexpr int XN = (XR * C4 + NT - 1) / NT;            // window float4s per thread
    constexpr int WV = (BN * KMAX * C4 + NT - 1) / NT;     // weight float4s per thread
    constexpr int H = KC / 2;                   // MFMA steps per tap; step s pairs channels s and H + s
    constexpr int HV = H / 4;                   // float4s per operand block and tap
    static_assert(WTM % 32 == 0 && WTN % 32 == 0 && KC % 8 == 0, "f32 tile shape");
    __shared__ __attribute__((aligned(16))) float xs[2][XR * XP];
    __shared__ __attribute__((aligned(16))) float ws[2][BN * WP];
    const int tile = (blockIdx.x & 7) * p.per_xcd + (blockIdx.x >> 3);
    if (tile >= p.total) return;
    const int n_tile = tile % p.tiles_n;  // output channels fastest: neighbours share the window
    const int rest = tile / p.tiles_n;
    const int m_tile = rest % p.tiles_m;
    const int lane_idx = rest / p.tiles_m;
    const int co0 = n_tile * BN;
    const int l0 = m_tile * BM;
    const int k = KT > 0 ? KT : p.k;
    const int rows = BM + (k - 1) * p.dil;
    const int K = k * p.cin;
    const float *xl = p.x + static_cast<int64_t>(lane_idx) * p.L * p.cin;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WN, wn = wave % WN;
    const int kh = lane >> 5, lr = lane & 31;
    const int nx = rows * C4, nw = BN * k * C4;

    float4_t xr[XN], wr[WV];
    auto load = [&](int c0) {
        // window: row j holds positions l0 - pad_left + j, channels c0 .. c0+7 (two float4s)
#pragma unroll
        for (int i = 0; i < XN; ++i) {
            const int e = tid + i * NT;
            const int j = e / C4, c4 = e % C4;
            const int s = l0 - p.pad_left + j;
            float4_t v = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
            if (e < nx && s >= 0 && s < p.L)
                v = *reinterpret_cast<const float4_t *>(xl + static_cast<int64_t>(s) * p.cin + c0 + c4 * 4);
            xr[i] = v;
        }
        // weights: 8 consecutive input channels of one (output channel, tap) are two float4s
#pragma unroll
        for (int i = 0; i < WV; ++i) {
            const int e = tid + i * NT;
            const int m = e / (k * C4), q = e - (e / (k * C4)) * (k * C4);
            const int t = q / C4, c4 = q % C4;
            float4_t v = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
            if (e < nw && co0 + m < p.cout)
                v = *reinterpret_cast<const float4_t *>(p.w + static_cast<int64_t>(co0 + m) * K + t * p.cin + c0 + c4 * 4);
            wr[i] = v;
        }
    };
    auto store = [&](int c0, int b) {
#pragma unroll
        for (int i = 0; i < XN; ++i) {
            const int e = tid + i * NT;
            if (e < nx) {
                const int j = e / C4, c4 = e % C4;
                float4_t v = xr[i];
                if constexpr (SNAKE) {
                    const int s = l0 - p.pad_left + j;
                    if (s >= 0 && s < p.L) {
                        float x[4] = {v[0], v[1], v[2], v[3]}, a[4], r[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q) a[q] = p.a_in[c0 + c4 * 4 + q], r[q] = p.r_in[c0 + c4 * 4 + q];
                        snake_f32_group<4>(x, a, r);
                        v = float4_t{x[0], x[1], x[2], x[3]};
                    }
                }
                *reinterpret_cast<float4_t *>(&xs[b][j * XP + c4 * 4]) = v;
            }
        }
#pragma unroll
        for (int i = 0; i < WV; ++i) {
            const int e = tid + i * NT;
            if (e < nw) {
                const int m = e / (k * C4), q = e - (e / (k * C4)) * (k * C4);
                *reinterpret_cast<float4_t *>(&ws[b][m * WP + q * 4]) = wr[i];
            }
        }
    };

    float16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = float16_t{};
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
        // operands of tap t: A[m][kk] = window[row m + t*dil][channel], B[kk][n] = w[n][tap t, channel];
        // a lane's H operands of a block are HV float4s
        typedef float4_t FragA[TM][HV];
        typedef float4_t FragB[TN][HV];
        auto frag = [&](int t, FragA &fa, FragB &fb) {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const float *xa = xs[b] + (wm * WTM + i * 32 + lr + t * p.dil) * XP + kh * H;
#pragma unroll
                for (int h = 0; h < HV; ++h) fa[i][h] = *reinterpret_cast<const float4_t *>(xa + 4 * h);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const float *wb = ws[b] + (wn * WTN + j * 32 + lr) * WP + t * KC + kh * H;
#pragma unroll
                for (int h = 0; h < HV; ++h) fb[j][h] = *reinterpret_cast<const float4_t *>(wb + 4 * h);
            }
        };
        auto mma = [&](const FragA &fa, const FragB &fb) {
#pragma unroll
            for (int st = 0; st < H; ++st)
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][st >> 2][st & 3], fb[j][st >> 2][st & 3],
                                                                         acc[i][j], 0, 0, 0);
        };
        if constexpr (KT > 0) {
            FragA fa[2];
            FragB fb[2];
            frag(0, fa[0], fb[0]);
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                if (t + 1 < KT) frag(t + 1, fa[(t + 1) & 1], fb[(t + 1) & 1]);
                mma(fa[t & 1], fb[t & 1]);
            }
        } else {
            for (int t = 0; t < k; ++t) {
                FragA fa;
                FragB fb;
                frag(t, fa, fb);
                mma(fa, fb);
            }
        }
        __syncthreads();
    }
    // each 32 x 32 block's residuals are requested together before its stores (res may alias the
    // outputs, so a load issued after a store waits for it: one memory round trip per block,
    // not per value)
    const int64_t lbase = static_cast<int64_t>(lane_idx) * p.L;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int co = co0 + wn * WTN + j * 32 + lr;
        if (co >= p.cout) continue;
        const float a_o = p.a_out ? p.a_out[co] : 0.0f, r_o = p.a_out ? p.r_out[co] : 0.0f;
        const float bias = p.bias ? p.bias[co] : 0.0f, scale = p.scale ? p.scale[co] : 1.0f;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int pos0 = l0 + wm * WTM + i * 32 + kh * 4;
            float rv[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int pos = pos0 + (r >> 2) * 8 + (r & 3);
                rv[r] = p.res && pos < p.L ? p.res[(lbase + pos) * p.cout + co] : 0.0f;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int pos = pos0 + (r >> 2) * 8 + (r & 3);
                if (pos >= p.L) continue;
                const int64_t off = (lbase + pos) * p.cout + co;
                // as conv_f32_epilogue: bias, scale, residual, activation
                float v = acc[i][j][r] + bias;
                if (p.scale) v = scale * v;
                if (p.res) v += rv[r];
                if (p.act == 1) v = tanhf(v);
                if (p.act == 3) v = fminf(fmaxf(v, -1.0f), 1.0f);
                if (p.y_pre) p.y_pre[off] = v;
                if (p.a_out) v = snake_f32(v, a_o, r_o);
                p.y[off] = v;
            }
        }
    }
}

// Any shape: one thread per output, f32 accumulation in (tap, channel) order.
__global__ __launch_bounds__(256) void conv_nlc_f32_direct(NlcF32Params p, int64_t total) {
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int co = static_cast<int>(e % p.cout);
        const int64_t row = e / p.cout;  // lane * L + position
        const int l = static_cast<int>(row % p.L);
        const float *xl = p.x + (row - l) * p.cin;
        const float *wr = p.w + static_cast<int64_t>(co) * p.k * p.cin;
        float acc = 0.0f;
        for (int t = 0; t < p.k; ++t) {
            const int s = l + t * p.dil - p.pad_left;
            if (s < 0 || s >= p.L) continue;
            const float *xs = xl + static_cast<int64_t>(s) * p.cin;
            for (int c = 0; c < p.cin; ++c) {
                float v = xs[c];
                if (p.a_in) v = snake_f32(v, p.a_in[c], p.r_in[c]);
                acc += v * wr[t * p.cin + c];
            }
        }
        float v = conv_f32_epilogue(acc, co, e, p);
        if (p.y_pre) p.y_pre[e] = v;
        if (p.a_out) v = snake_f32(v, p.a_out[co], p.r_out[co]);
        p.y[e] = v;
    }
}

// A single output channel (the waveform conv, cin -> 1): HBM-bound, every input element feeds k
// products. A workgroup owns kNarrowBM positions of one lane, a thread one position. Per
// 32-channel chunk the window (kNarrowBM + (k-1)*dil rows) is loaded into registers whole, then
// stored to LDS (the prologue SnakeBeta applied on the way), rows 36 floats apart so the 16-byte
// reads of 16 consecutive rows hit 16 disjoint bank quads; the chunk's k x 32 weights sit beside
// it and are read as broadcasts. Products accumulate in f32 in (chunk, tap, channel) order.
constexpr int kNarrowBM = 256, kNarrowKC = 32, kNarrowPitch = kNarrowKC + 4, kNarrowMaxHalo = 64;
constexpr int kNarrowRows = kNarrowBM + kNarrowMaxHalo;
constexpr int kNarrowVec = (kNarrowRows * (kNarrowKC / 4) + 255) / 256;  // window float4s per thread, at most

// SPLIT: x holds rows [hi(cin) | lo(cin)] of f16 (an f32 codec's split storage), each value read
// as hi + lo in f32.
template <bool SPLIT>
__global__ __launch_bounds__(256) void conv_nlc_f32_narrow(NlcF32Params p) {
    __shared__ __attribute__((aligned(16))) float win[kNarrowRows * kNarrowPitch];
    __shared__ __attribute__((aligned(16))) float wsh[7 * kNarrowKC];
    const int tile = blockIdx.x;
    const int lane_idx = tile / p.tiles_m;
    const int l0 = (tile - lane_idx * p.tiles_m) * kNarrowBM;
    const int rows = kNarrowBM + (p.k - 1) * p.dil;
    const int nvec = rows * (kNarrowKC / 4);
    const float *xl = p.x + static_cast<int64_t>(lane_idx) * p.L * p.cin;  // f32 rows (SPLIT: the same byte count)
    const int tid = threadIdx.x;
    float acc = 0.0f;
    for (int c0 = 0; c0 < p.cin; c0 += kNarrowKC) {
        float4_t buf[kNarrowVec];
        if constexpr (SPLIT) {
            // 8 channels a thread: 16 bytes of hi and 16 of lo, two float4 of the window (16-byte
            // loads: 26% faster than 4 channels of 8 bytes each at the codec's output conv)
            constexpr int V8 = (kNarrowRows * (kNarrowKC / 8) + 255) / 256;
            static_assert(2 * V8 <= kNarrowVec + 1, "register budget");
            half8_t hh[V8], ll[V8];
#pragma unroll
            for (int i = 0; i < V8; ++i) {
                const int v = tid + i * 256;
                const int r = v >> 2, q = v & 3;
                const int s = l0 - p.pad_left + r;
                hh[i] = half8_t{};
                ll[i] = half8_t{};
                if (v < rows * 4 && s >= 0 && s < p.L) {
                    const half_t *hr = reinterpret_cast<const half_t *>(xl) + static_cast<int64_t>(s) * 2 * p.cin + c0 + q * 8;
                    hh[i] = *reinterpret_cast<const half8_t *>(hr);
                    ll[i] = *reinterpret_cast<const half8_t *>(hr + p.cin);
                }
            }
            if (c0 > 0) __syncthreads();
            if (tid < p.k * kNarrowKC) {
                const int t = tid / kNarrowKC, c = tid - t * kNarrowKC;
                wsh[tid] = p.w[t * p.cin + c0 + c];
            }
#pragma unroll
            for (int i = 0; i < V8; ++i) {
                const int v = tid + i * 256;
                if (v < rows * 4) {
                    const int r = v >> 2, q = v & 3;
                    float4_t a, b;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        a[j] = static_cast<float>(hh[i][j]) + static_cast<float>(ll[i][j]);
                        b[j] = static_cast<float>(hh[i][j + 4]) + static_cast<float>(ll[i][j + 4]);
                    }
                    *reinterpret_cast<float4_t *>(win + r * kNarrowPitch + q * 8) = a;
                    *reinterpret_cast<float4_t *>(win + r * kNarrowPitch + q * 8 + 4) = b;
                }
            }
        } else {
#pragma unroll
        for (int i = 0; i < kNarrowVec; ++i) {
            const int v = tid + i * 256;
            buf[i] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
            const int r = v >> 3, q = v & 7;
            const int s = l0 - p.pad_left + r;
            if (v < nvec && s >= 0 && s < p.L)
                buf[i] = *reinterpret_cast<const float4_t *>(xl + static_cast<int64_t>(s) * p.cin + c0 + q * 4);
        }
        if (c0 > 0) __syncthreads();  // every thread is done with the previous chunk's window
        if (tid < p.k * kNarrowKC) {
            const int t = tid / kNarrowKC, c = tid - t * kNarrowKC;
            wsh[tid] = p.w[t * p.cin + c0 + c];
        }
#pragma unroll
        for (int i = 0; i < kNarrowVec; ++i) {
            const int v = tid + i * 256;
            if (v < nvec) {
                const int r = v >> 3, q = v & 7;
                float4_t x = buf[i];
                const int s = l0 - p.pad_left + r;
                if (p.a_in && s >= 0 && s < p.L) {
                    float xv[4] = {x[0], x[1], x[2], x[3]};
                    float a[4], rr[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) a[j] = p.a_in[c0 + q * 4 + j], rr[j] = p.r_in[c0 + q * 4 + j];
                    snake_f32_group<4>(xv, a, rr);
                    x = float4_t{xv[0], xv[1], xv[2], xv[3]};
                }
                *reinterpret_cast<float4_t *>(win + r * kNarrowPitch + q * 4) = x;
            }
        }
        }
        __syncthreads();
        for (int t = 0; t < p.k; ++t) {
            const float *row = win + (tid + t * p.dil) * kNarrowPitch;
            const float *wr = wsh + t * kNarrowKC;
#pragma unroll
            for (int q = 0; q < kNarrowKC / 4; ++q) {
                const float4_t x = *reinterpret_cast<const float4_t *>(row + q * 4);
                const float4_t w = *reinterpret_cast<const float4_t *>(wr + q * 4);
                acc = __builtin_fmaf(x[0], w[0], acc);
                acc = __builtin_fmaf(x[1], w[1], acc);
                acc = __builtin_fmaf(x[2], w[2], acc);
                acc = __builtin_fmaf(x[3], w[3], acc);
            }
        }
    }
    const int l = l0 + tid;
    if (l >= p.L) return;
    const int64_t off = static_cast<int64_t>(lane_idx) * p.L + l;
    float v = conv_f32_epilogue(acc, 0, off, p);
    if (p.y_pre) p.y_pre[off] = v;
    if (p.a_out) v = snake_f32(v, p.a_out[0], p.r_out[0]);
    p.y[off] = v;
}

// The tile's output-channel width: the widest of 64, 96 and 32 that divides cout.
int f32_tile_bn(int64_t cout) { return cout % 64 == 0 ? 64 : cout % 96 == 0 ? 96 : 32; }
// Its rows: 256 for the 64-wide k = 7 tile, 128 otherwise.
int f32_tile_bm(int kmax, int bn) { return kmax == 7 && bn == 64 ? 256 : 128; }
// Channels per chunk: 16 for k = 1 (half the barriers of 8; 7-9% faster on the codec's k = 1
// shapes), 8 otherwise.
constexpr int f32_tile_kc(int kmax) { return kmax == 1 ? 16 : kF32KC; }

template <int KMAX, int HMAX, int KT, int BM, int BN, int WM, int WN, int KC = kF32KC>
hipError_t launch_f32_tile(NlcF32Params p, int64_t lanes, bool snake, hipStream_t stream) {
    p.tiles_n = p.cout / BN;
    p.tiles_m = (p.L + BM - 1) / BM;
    const int64_t total = lanes * p.tiles_m * p.tiles_n;
    p.total = static_cast<int>(total);
    p.per_xcd = static_cast<int>((total + 7) / 8);
    const unsigned grid = static_cast<unsigned>(int64_t(p.per_xcd) * 8);
    if (snake)
        conv_nlc_f32_mfma<KMAX, HMAX, KT, BM, BN, WM, WN, KC, true><<<grid, 64 * WM * WN, 0, stream>>>(p);
    else
        conv_nlc_f32_mfma<KMAX, HMAX, KT, BM, BN, WM, WN, KC, false><<<grid, 64 * WM * WN, 0, stream>>>(p);
    return hipGetLastError();
}

template <int KMAX, int HMAX, int KT>
hipError_t launch_nlc_f32(const NlcF32Params &p, int64_t lanes, bool snake, hipStream_t stream) {
    constexpr int KC = f32_tile_kc(KMAX);
    switch (f32_tile_bn(p.cout)) {
    case 64:  // the k = 7 class on 256 rows over 4 x 2 waves (four waves per SIMD), the others on 128
        if constexpr (KMAX == 7) return launch_f32_tile<KMAX, HMAX, KT, 256, 64, 4, 2, KC>(p, lanes, snake, stream);
        else return launch_f32_tile<KMAX, HMAX, KT, 128, 64, 2, 2, KC>(p, lanes, snake, stream);
    case 96: return launch_f32_tile<KMAX, HMAX, KT, 128, 96, 4, 1, KC>(p, lanes, snake, stream);
    default: return launch_f32_tile<KMAX, HMAX, KT, 128, 32, 4, 1, KC>(p, lanes, snake, stream);
    }
}

// (KMAX, HMAX, KT) of the class a tiled shape runs in: k = 1, k = 2 without dilation, k = 7, or
// fewer taps (KMAX 7, taps at run time)
void f32_class(const dtts_conv_desc *d, int &kmax, int &hmax, int &kt) {
    if (d->k == 1) kmax = 1, hmax = 0, kt = 1;
    else if (d->k == 2 && d->dilation == 1) kmax = 2, hmax = 1, kt = 2;
    else kmax = 7, hmax = 64, kt = d->k == 7 ? 7 : 0;
}

bool nlc_f32_narrow(const dtts_conv_desc *d) {
    return d->cout == 1 && d->cin % kNarrowKC == 0 && d->k <= 7 && (d->k - 1) * d->dilation <= kNarrowMaxHalo &&
           aligned(d->x, 16);
}

bool nlc_f32_tiled(const dtts_conv_desc *d) {
    return d->cin % f32_tile_kc(d->k == 1 ? 1 : 7) == 0 && d->cout % 32 == 0 && d->k <= 7 &&
           (d->k - 1) * d->dilation <= 64 && aligned(d->x, 16) && aligned(d->w, 16);
}

}  // namespace

const char *conv_f32_kernel_name(const dtts_conv_desc *d) {
    if (nlc_f32_narrow(d)) return "conv_nlc_f32_narrow";
    if (!nlc_f32_tiled(d)) return "conv_nlc_f32_direct";
    static thread_local char buf[96];
    int kmax, hmax, kt;
    f32_class(d, kmax, hmax, kt);
    const int bn = f32_tile_bn(d->cout), bm = f32_tile_bm(kmax, bn);
    const int wm = bn == 64 ? bm / 64 : 4, wn = bn == 64 ? 2 : 1;
    snprintf(buf, sizeof(buf), "conv_nlc_f32_mfma<%d, %d, %d, %d, %d, %d, %d, %d", kmax, hmax, kt, bm, bn, wm, wn,
             f32_tile_kc(kmax));
    return buf;
}

int conv1d_nlc_f32(const dtts_conv_desc *d, hipStream_t stream) {
    const char *name = "dtts_conv1d_nlc_f32";
    DTTS_REQUIRE(d, "%s: null descriptor", name);
    DTTS_REQUIRE(d->lanes >= 0 && d->len >= 0 && d->cin > 0 && d->cout > 0 && d->k > 0 && d->dilation > 0 &&
                     d->pad_left >= 0 && d->pad_left <= (d->k - 1) * d->dilation,
                 "%s: bad shape or pad_left", name);
    DTTS_REQUIRE(d->act == 0 || d->act == 1 || d->act == 3, "%s: act %d unknown (0, 1 tanh, 3 clamp)", name, d->act);
    if (d->lanes == 0 || d->len == 0) return DTTS_OK;
    DTTS_REQUIRE(d->x && d->w && d->y, "%s: null x, w or y", name);
    DTTS_REQUIRE((d->in_alpha == nullptr) == (d->in_brecip == nullptr) &&
                     (d->out_alpha == nullptr) == (d->out_brecip == nullptr),
                 "%s: snake alpha and brecip go together", name);
    DTTS_REQUIRE(d->lanes * d->len * d->cout < (int64_t(1) << 40) && d->lanes * d->len * d->cin < (int64_t(1) << 40) &&
                     d->len < (int64_t(1) << 30) && d->cin * d->k < (int64_t(1) << 30),
                 "%s: shape too large", name);
    NlcF32Params p{};
    p.x = static_cast<const float *>(d->x);
    p.w = static_cast<const float *>(d->w);
    p.bias = static_cast<const float *>(d->bias);
    p.a_in = d->in_alpha;
    p.r_in = d->in_brecip;
    p.res = static_cast<const float *>(d->residual);
    p.scale = d->out_scale;
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
    hipError_t e;
    if (nlc_f32_narrow(d)) {
        p.tiles_m = static_cast<int>((d->len + kNarrowBM - 1) / kNarrowBM);
        DTTS_REQUIRE(d->lanes * p.tiles_m < (int64_t(1) << 31), "%s: too many tiles", name);
        conv_nlc_f32_narrow<false><<<static_cast<unsigned>(d->lanes * p.tiles_m), 256, 0, stream>>>(p);
        e = hipGetLastError();
    } else if (nlc_f32_tiled(d)) {
        DTTS_REQUIRE(d->lanes * (d->cout / f32_tile_bn(d->cout)) * ((d->len + 127) / 128) < (int64_t(1) << 31),
                     "%s: too many tiles", name);
        const bool snake = d->in_alpha != nullptr;
        int kmax, hmax, kt;
        f32_class(d, kmax, hmax, kt);
        if (kmax == 1)
            e = launch_nlc_f32<1, 0, 1>(p, d->lanes, snake, stream);
        else if (kmax == 2)
            e = launch_nlc_f32<2, 1, 2>(p, d->lanes, snake, stream);
        else if (kt == 7)
            e = launch_nlc_f32<7, 64, 7>(p, d->lanes, snake, stream);
        else
            e = launch_nlc_f32<7, 64, 0>(p, d->lanes, snake, stream);
    } else {
        const int64_t total = d->lanes * d->len * d->cout;
        conv_nlc_f32_direct<<<grid_for(total, 256, 16), 256, 0, stream>>>(p, total);
        e = hipGetLastError();
    }
    DTTS_HIP_CHECK(e, name);
    return DTTS_OK;
}

bool conv_f32_narrow_split_eligible(const dtts_conv_desc *d) { return d && nlc_f32_narrow(d); }

int conv1d_nlc_f32_narrow_split(const dtts_conv_desc *d, hipStream_t stream) {
    const char *name = "dtts_codec (split output conv)";
    DTTS_REQUIRE(conv_f32_narrow_split_eligible(d) && d->lanes > 0 && d->len > 0 && d->w && d->y && !d->in_alpha,
                 "%s: shape not supported (or a prologue SnakeBeta, which split input does not take)", name);
    DTTS_REQUIRE(d->act == 0 || d->act == 1 || d->act == 3, "%s: act %d unknown", name, d->act);
    NlcF32Params p{};
    p.x = static_cast<const float *>(d->x);
    p.w = static_cast<const float *>(d->w);
    p.bias = static_cast<const float *>(d->bias);
    p.a_in = d->in_alpha;
    p.r_in = d->in_brecip;
    p.res = static_cast<const float *>(d->residual);
    p.scale = d->out_scale;
    p.y_pre = static_cast<float *>(d->y_pre);
    p.y = static_cast<float *>(d->y);
    p.a_out = d->out_alpha;
    p.r_out = d->out_brecip;
    p.L = static_cast<int>(d->len);
    p.cin = static_cast<int>(d->cin);
    p.cout = 1;
    p.k = static_cast<int>(d->k);
    p.dil = static_cast<int>(d->dilation);
    p.pad_left = static_cast<int>(d->pad_left);
    p.act = d->act;
    p.tiles_m = static_cast<int>((d->len + kNarrowBM - 1) / kNarrowBM);
    DTTS_REQUIRE(d->lanes * p.tiles_m < (int64_t(1) << 31), "%s: too many tiles", name);
    conv_nlc_f32_narrow<true><<<static_cast<unsigned>(d->lanes * p.tiles_m), 256, 0, stream>>>(p);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

}  // namespace dtts

extern "C" int dtts_conv1d_nlc_f32_ex(const dtts_conv_desc *desc, hipStream_t stream) {
    return dtts::conv1d_nlc_f32(desc, stream);
}
