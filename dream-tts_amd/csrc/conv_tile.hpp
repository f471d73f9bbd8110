// The channels-last implicit-GEMM conv tile shared by the conv kernel and the fused residual
// unit: the staged dilated window, the MFMA main loop, and the LDS-staged epilogue.
//
// GEMM view per lane: M = positions, N = output channels, K = k*cin tap-major. A workgroup of
// WM x WN waves owns BM positions x BN channels. Per KC-channel chunk it stages, in LDS:
//   A: the whole dilated window, BM + (k-1)*dil rows x KC channels, loaded once and read by
//      all k taps at row offsets t*dil (the im2col never exists, not even in LDS);
//   B: w[n0 .. n0+BN, t*cin + c0 .. +KC] for every tap t.
// Each wave owns (BM/WM) x (BN/WN) on 32x32x16 f16 MFMAs with f32 accumulation. The next chunk
// is prefetched into registers while the current one computes, into a second LDS stage when the
// tile has two (one barrier per chunk). Row pitches are padded by 8 halves (16 bytes) so the
// 16-byte fragment reads of consecutive rows hit distinct banks.
#pragma once

#include "conv.hpp"
#include "snake.hpp"

// Halves of padding per LDS row of the A window and B tile (a multiple of 8 keeps the rows
// 16-byte aligned for ds_read_b128).
#ifndef DTTS_LDS_PAD
#define DTTS_LDS_PAD 8
#endif

namespace dtts {

template <int BM_, int BN_, int WM_, int WN_, int KC_, int KMAX_, int HMAX_, int NBUF_ = 1>
struct ConvTile {
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, KC = KC_, KMAX = KMAX_, HMAX = HMAX_;
    static constexpr int NBUF = NBUF_;  // LDS stages: 2 overlaps staging chunk c+1 with computing chunk c
    static constexpr int THREADS = 64 * WM * WN;
    static constexpr int WTM = BM / WM, WTN = BN / WN;  // per-wave tile
    static constexpr int TM = WTM / 32, TN = WTN / 32;  // 32x32 blocks per wave
    static constexpr int LDA = KC + DTTS_LDS_PAD;       // LDS pitch (halves) of A and B rows
    static constexpr int SEGS = KC / 8;                 // 16-byte segments per row chunk
    static constexpr int A_ROWS = BM + HMAX;
    static constexpr int A_HALVES = A_ROWS * LDA;
    static constexpr int B_HALVES = KMAX * BN * LDA;
    static constexpr int STAGE_HALVES = A_HALVES + B_HALVES;
    static constexpr int MAIN_BYTES = NBUF * STAGE_HALVES * 2;
    static constexpr int A_SEGS = A_ROWS * SEGS;
    static constexpr int A_PER_T = (A_SEGS + THREADS - 1) / THREADS;
    static constexpr int B_SEGS = KMAX * BN * SEGS;
    static constexpr int B_PER_T = (B_SEGS + THREADS - 1) / THREADS;
    static constexpr int EPI_PITCH = WTN + 4;  // floats, per-wave epilogue tile
    static constexpr int EPI_BYTES = WM * WN * 32 * EPI_PITCH * 4;
    // workgroups per CU the register budget is sized for (two when two fit in LDS)
    static constexpr int MIN_WG = (THREADS <= 256 && 2 * MAIN_BYTES <= 160 * 1024) ? 2 : 1;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0 && KC % 16 == 0, "tile shape");
};

// The demangled name of kernel<ConvTile<...>, ...> as profilers print it; `tail` closes the
// template argument list (", true>", " >").
template <typename Cfg>
inline const char *tile_kernel_name(char *buf, size_t n, const char *kernel, const char *tail) {
    snprintf(buf, n, "%s<dtts::ConvTile<%d, %d, %d, %d, %d, %d, %d, %d>%s", kernel, Cfg::BM, Cfg::BN, Cfg::WM, Cfg::WN,
             Cfg::KC, Cfg::KMAX, Cfg::HMAX, Cfg::NBUF, tail);
    return buf;
}

struct ConvArgs {
    const half_t *x;
    const half_t *w;
    const half_t *bias;
    const float *a_in;
    const float *r_in;
    const half_t *res;
    half_t *y_pre;
    half_t *y;
    const float *a_out;
    const float *r_out;
    int L, cin, cout, k, dil, pad_left, act;
    int tiles_m, tiles_n, total_tiles, tiles_per_xcd;
};

__device__ __forceinline__ float conv_act(float v, int act) { return act == 1 ? tanhf(v) : v; }

// XCD-aware tile order: dispatch slot b runs on XCD b % 8; each XCD takes a contiguous range of
// (lane, m, n) tiles, N fastest, so an M tile's window is fetched into one L2 and reused by its
// N tiles there. Returns false for the padding slots past the last tile.
__device__ __forceinline__ bool conv_tile_coords(const ConvArgs &p, int &lane_idx, int &m_tile, int &n_tile) {
    const int tile = (blockIdx.x & 7) * p.tiles_per_xcd + (blockIdx.x >> 3);
    if (tile >= p.total_tiles) return false;
    n_tile = tile % p.tiles_n;
    const int rest = tile / p.tiles_n;
    m_tile = rest % p.tiles_m;
    lane_idx = rest / p.tiles_m;
    return true;
}

// acc[i][j] += sum over taps and cin of window(x) . w for the workgroup's BM x BN tile.
template <typename Cfg, bool SNAKE_IN>
__device__ __forceinline__ void conv_mainloop(const ConvArgs &p, const half_t *xl, int l0, int n0, half_t *As,
                                              half_t *Bs, float16_t (&acc)[Cfg::TM][Cfg::TN]) {
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
    const int rows = Cfg::BM + (p.k - 1) * p.dil;
    const int win0 = l0 - p.pad_left;
    const int K = p.k * p.cin;
    const int bsegs = p.k * Cfg::BN * Cfg::SEGS;

    half8_t ra[Cfg::A_PER_T];
    half8_t rb[Cfg::B_PER_T];
    auto load_chunk = [&](int c0) {
#pragma unroll
        for (int i = 0; i < Cfg::A_PER_T; ++i) {
            const int seg = tid + i * Cfg::THREADS;
            const int r = seg / Cfg::SEGS;
            const int q = seg % Cfg::SEGS;
            half8_t v = half8_t{};
            const int s = win0 + r;
            if (seg < Cfg::A_SEGS && r < rows && s >= 0 && s < p.L)
                v = *reinterpret_cast<const half8_t *>(xl + static_cast<int64_t>(s) * p.cin + c0 + q * 8);
            ra[i] = v;
        }
#pragma unroll
        for (int i = 0; i < Cfg::B_PER_T; ++i) {
            const int seg = tid + i * Cfg::THREADS;
            half8_t v = half8_t{};
            if (seg < Cfg::B_SEGS && seg < bsegs) {
                const int row = seg / Cfg::SEGS;  // t * BN + n
                const int q = seg % Cfg::SEGS;
                const int t = row / Cfg::BN;
                const int n = row - t * Cfg::BN;
                v = *reinterpret_cast<const half8_t *>(p.w + static_cast<int64_t>(n0 + n) * K + t * p.cin + c0 + q * 8);
            }
            rb[i] = v;
        }
    };
    auto store_chunk = [&](int c0, half_t *As, half_t *Bs) {
#pragma unroll
        for (int i = 0; i < Cfg::A_PER_T; ++i) {
            const int seg = tid + i * Cfg::THREADS;
            if (seg < Cfg::A_SEGS) {
                const int r = seg / Cfg::SEGS;
                const int q = seg % Cfg::SEGS;
                half8_t v = ra[i];
                if constexpr (SNAKE_IN) {
                    const int c = c0 + q * 8;
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        v[j] = static_cast<half_t>(snake_f16out(static_cast<float>(v[j]), p.a_in[c + j], p.r_in[c + j]));
                }
                *reinterpret_cast<half8_t *>(As + r * Cfg::LDA + q * 8) = v;
            }
        }
#pragma unroll
        for (int i = 0; i < Cfg::B_PER_T; ++i) {
            const int seg = tid + i * Cfg::THREADS;
            if (seg < Cfg::B_SEGS) {
                const int row = seg / Cfg::SEGS;
                const int q = seg % Cfg::SEGS;
                *reinterpret_cast<half8_t *>(Bs + row * Cfg::LDA + q * 8) = rb[i];
            }
        }
    };

    const int nchunks = p.cin / Cfg::KC;
    const int arow0 = wm * Cfg::WTM + (lane & 31);
    const int bcol0 = wn * Cfg::WTN + (lane & 31);
    const int koff = (lane >> 5) * 8;
    auto compute = [&](const half_t *A, const half_t *B) {
        for (int t = 0; t < p.k; ++t) {
            const half_t *at = A + (arow0 + t * p.dil) * Cfg::LDA + koff;
            const half_t *bt = B + (t * Cfg::BN + bcol0) * Cfg::LDA + koff;
#pragma unroll
            for (int kk = 0; kk < Cfg::KC; kk += 16) {
                half8_t af[Cfg::TM], bf[Cfg::TN];
#pragma unroll
                for (int i = 0; i < Cfg::TM; ++i) af[i] = *reinterpret_cast<const half8_t *>(at + i * 32 * Cfg::LDA + kk);
#pragma unroll
                for (int j = 0; j < Cfg::TN; ++j) bf[j] = *reinterpret_cast<const half8_t *>(bt + j * 32 * Cfg::LDA + kk);
#pragma unroll
                for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
                    for (int j = 0; j < Cfg::TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        }
    };
    load_chunk(0);
    if constexpr (Cfg::NBUF == 1) {
        for (int c = 0; c < nchunks; ++c) {
            store_chunk(c * Cfg::KC, As, Bs);
            __syncthreads();
            if (c + 1 < nchunks) load_chunk((c + 1) * Cfg::KC);
            compute(As, Bs);
            __syncthreads();
        }
    } else {
        // stage c+1 is written while stage c is read; the one barrier per chunk also guarantees
        // that the stage being overwritten was finished by every wave one chunk ago
        store_chunk(0, As, Bs);
        __syncthreads();
        for (int c = 0; c < nchunks; ++c) {
            const int cur = c & 1;
            half_t *Ac = As + cur * Cfg::STAGE_HALVES;
            half_t *Bc = Bs + cur * Cfg::STAGE_HALVES;
            if (c + 1 < nchunks) load_chunk((c + 1) * Cfg::KC);
            compute(Ac, Bc);
            if (c + 1 < nchunks) store_chunk((c + 1) * Cfg::KC, As + (cur ^ 1) * Cfg::STAGE_HALVES, Bs + (cur ^ 1) * Cfg::STAGE_HALVES);
            __syncthreads();
        }
    }
}

// Writes acc (+ bias, + residual, act, rounded; y_pre; SnakeBeta_out; y) for the tile, one 32-row
// block per wave at a time through the wave's own LDS region (16-byte coalesced rows). `ld` is the
// output row length (cout), `n0` the tile's first output channel, `lmax` the lane's length.
template <typename Cfg>
__device__ __forceinline__ void conv_epilogue(const float16_t (&acc)[Cfg::TM][Cfg::TN], char *smem, int64_t row0,
                                              int l0, int n0, int lmax, int ld, const half_t *bias, const half_t *res,
                                              half_t *y_pre, half_t *y, const float *a_out, const float *r_out,
                                              int act) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
    float *E = reinterpret_cast<float *>(smem) + wave * 32 * Cfg::EPI_PITCH;
    const int nw = n0 + wn * Cfg::WTN;
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i) {
        __syncthreads();
#pragma unroll
        for (int j = 0; j < Cfg::TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int mr = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                E[mr * Cfg::EPI_PITCH + j * 32 + (lane & 31)] = acc[i][j][r];
            }
        __syncthreads();
        constexpr int CG = Cfg::WTN / 8;
        for (int g = lane; g < 32 * CG; g += 64) {
            const int mr = g / CG;
            const int cg = g - mr * CG;
            const int l = l0 + wm * Cfg::WTM + i * 32 + mr;
            if (l >= lmax) continue;
            const int n = nw + cg * 8;
            const float4_t *src = reinterpret_cast<const float4_t *>(E + mr * Cfg::EPI_PITCH + cg * 8);
            const float4_t v0 = src[0], v1 = src[1];
            float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            if (bias) {
                const half8_t bb = *reinterpret_cast<const half8_t *>(bias + n);
#pragma unroll
                for (int q = 0; q < 8; ++q) v[q] += static_cast<float>(bb[q]);
            }
            const int64_t off = (row0 + l) * ld + n;
            if (res) {
                const half8_t rr = *reinterpret_cast<const half8_t *>(res + off);
#pragma unroll
                for (int q = 0; q < 8; ++q) v[q] += static_cast<float>(rr[q]);
            }
            half8_t h;
#pragma unroll
            for (int q = 0; q < 8; ++q) h[q] = static_cast<half_t>(conv_act(v[q], act));
            if (y_pre) *reinterpret_cast<half8_t *>(y_pre + off) = h;
            if (a_out) {
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    h[q] = static_cast<half_t>(snake_f16out(static_cast<float>(h[q]), a_out[n + q], r_out[n + q]));
            }
            *reinterpret_cast<half8_t *>(y + off) = h;
        }
    }
    __syncthreads();
}

}  // namespace dtts
