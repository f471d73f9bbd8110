// The channels-last implicit-GEMM conv tile: the staged dilated window, the MFMA main loop, and
// the epilogue.
//
// GEMM view per lane: M = positions, N = output channels, K = k*cin tap-major. A workgroup of
// WM x WN waves owns BM positions x BN channels. Per KC-channel chunk it stages, in LDS:
//   A: the whole dilated window, BM + (k-1)*dil rows x KC channels, loaded once and read by
//      all k taps at row offsets t*dil (the im2col never exists, not even in LDS);
//   B: w[n0 .. n0+BN, t*cin + c0 .. +KC] for every tap t.
// Each wave owns (BM/WM) x (BN/WN) on 32x32x16 f16 MFMAs with f32 accumulation, computed
// transposed (weights as the A operand): a lane's result is one position x 16 channels.
//
// Two ways to fill a stage (the tile's STAGING parameter):
//   kStageRegs:   global -> registers -> ds_write, rows padded by 8 halves so the 16-byte
//                 fragment reads of consecutive rows hit distinct banks; the next chunk is
//                 prefetched into registers while the current one computes.
//   kStageDirect: buffer_load_dwordx4 ... lds, the load unit writing LDS itself. No staging
//                 registers, no per-chunk address arithmetic (a chunk moves only the scalar
//                 offset), and rows of the window outside [0, L) read as zeros through the
//                 buffer range check. A load instruction fills 64 consecutive 16-byte slots,
//                 so rows cannot be padded: the 16-byte segments of a row are XOR-swizzled
//                 instead. NBUF >= 2 stages: chunk c+NBUF-1 lands while chunk c is multiplied,
//                 one barrier per chunk.
#pragma once

#include <type_traits>

#include "conv.hpp"
#include "snake.hpp"

namespace dtts {

enum { kStageRegs = 0, kStageDirect = 1 };

template <int BM_, int BN_, int WM_, int WN_, int KC_, int KMAX_, int HMAX_, int NBUF_ = 1, int STAGING_ = kStageRegs>
struct ConvTile {
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, KC = KC_, KMAX = KMAX_, HMAX = HMAX_;
    static constexpr int STAGING = STAGING_;
    static constexpr int NBUF = STAGING == kStageDirect && NBUF_ < 2 ? 2 : NBUF_;  // LDS stages
    static constexpr int THREADS = 64 * WM * WN;
    static constexpr int NW = WM * WN;
    static constexpr int WTM = BM / WM, WTN = BN / WN;  // per-wave tile
    static constexpr int TM = WTM / 32, TN = WTN / 32;  // 32x32 blocks per wave
    static constexpr int SEGS = KC / 8;                 // 16-byte segments per row chunk
    // register staging: padded rows
    static constexpr int LDA = KC + 8;  // LDS pitch (halves) of A and B rows
    static constexpr int A_SEGS = (BM + HMAX) * SEGS;
    static constexpr int A_PER_T = (A_SEGS + THREADS - 1) / THREADS;
    static constexpr int B_SEGS = KMAX * BN * SEGS;
    static constexpr int B_PER_T = (B_SEGS + THREADS - 1) / THREADS;
    // direct staging: unpadded swizzled rows, 1 KiB per load instruction
    static constexpr int ROW_BYTES = STAGING == kStageDirect ? KC * 2 : LDA * 2;
    static constexpr int RPI = 1024 / (KC * 2);  // rows per load instruction
    static constexpr int A_ROWS = STAGING == kStageDirect ? (BM + HMAX + RPI - 1) / RPI * RPI : BM + HMAX;
    static constexpr int A_INST = A_ROWS / RPI, B_INST = KMAX * BN / RPI;
    static constexpr int A_PER_W = (A_INST + NW - 1) / NW, B_PER_W = (B_INST + NW - 1) / NW;
    static constexpr int A_BYTES = A_ROWS * ROW_BYTES;
    static constexpr int B_BYTES = KMAX * BN * ROW_BYTES;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    static constexpr int MAIN_BYTES = NBUF * STAGE_BYTES;
    // epilogue: each wave stages a 32-row block of its results in f32 through LDS (the stages are
    // free by then); a row pitch of 4 (mod 64) floats keeps the 16-byte writes of 16 consecutive
    // rows on distinct banks
    static constexpr int EPI_PITCH = WTN + 4;
    static constexpr int EPI_BYTES = NW * 32 * EPI_PITCH * 4;
    // the output SnakeBeta table (a/2pi, r per channel of the tile) sits after both
    static constexpr int TAB_OFFSET = MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES;
    static constexpr int LDS_BYTES = TAB_OFFSET + BN * 8;
    // workgroups per CU the register budget is sized for: as many as fit in LDS, at most three
    // (two when the accumulators alone take 96 registers: three would spill)
    static constexpr int WG_BY_LDS = (160 * 1024) / LDS_BYTES;
    static constexpr int MIN_WG = THREADS > 256 ? 1 : (WG_BY_LDS >= 3 && TM * TN <= 4 ? 3 : (WG_BY_LDS >= 2 ? 2 : 1));
    static_assert(WTM % 32 == 0 && WTN % 32 == 0 && KC % 16 == 0, "tile shape");
    static_assert(STAGING != kStageDirect || (KC >= 16 && KC <= 64 && BN % RPI == 0), "direct staging shape");
};

// The demangled name of kernel<ConvTile<...>, ...> as profilers print it; `tail` closes the
// template argument list (", true>", " >").
template <typename Cfg>
inline const char *tile_kernel_name(char *buf, size_t n, const char *kernel, const char *tail) {
    snprintf(buf, n, "%s<dtts::ConvTile<%d, %d, %d, %d, %d, %d, %d, %d, %d>%s", kernel, Cfg::BM, Cfg::BN, Cfg::WM,
             Cfg::WN, Cfg::KC, Cfg::KMAX, Cfg::HMAX, Cfg::NBUF, Cfg::STAGING, tail);
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
    const float *scale;  // [cout] factor on (sum + bias) before the residual, or null
    int L, cin, cout, k, dil, pad_left, act;
    int tiles_m, tiles_n, total_tiles, tiles_per_xcd;
    int tiles_ng;  // N tiles per group of the tile order (a divisor of tiles_n; tiles_n: N fastest)
};

// N tiles per group of the tile order: the largest divisor of tiles_n whose weight slices (each
// BN x k x cin f16) fit `budget` bytes, so a group's weights stay in an XCD's 4 MB L2 while every
// lane's M tiles pass over them. All of tiles_n when the whole weight fits (the plain N-fastest
// order, where an M tile's window is what L2 reuses).
inline int pick_tiles_ng(int tiles_n, int64_t slice_bytes, int64_t budget = int64_t(4) << 20) {
    if (int64_t(tiles_n) * slice_bytes <= budget) return tiles_n;
    int best = 1;
    for (int g = 1; g <= tiles_n; ++g)
        if (tiles_n % g == 0 && int64_t(g) * slice_bytes <= budget) best = g;
    return best;
}

// Host check for direct staging: every byte offset a buffer load forms stays below 2^31, where
// the out-of-range marker sits.
inline bool direct_offsets_fit(int64_t len, int64_t cin, int64_t cout, int64_t k) {
    return len * cin * 2 < (int64_t(1) << 31) && cout * k * cin * 2 < (int64_t(1) << 31);
}

// act 1: tanh; act 2: GELU, erf form (0.5 v (1 + erf(v / sqrt 2))); act 3: clamp to [-1, 1].
__device__ __forceinline__ float conv_act(float v, int act) {
    if (act == 1) return tanhf(v);
    if (act == 2) return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
    if (act == 3) return fminf(fmaxf(v, -1.0f), 1.0f);
    return v;
}

// The epilogue's sum for one element: (acc + bias), times the channel's scale when there is one,
// plus the residual; each step rounded in f32 (no contraction), as the reference's separate ops.
__device__ __forceinline__ float conv_sum(float acc, float bias, const float *scale, int n, float res) {
#pragma clang fp contract(off)
    float t = acc + bias;
    if (scale) t = t * scale[n];
    return t + res;
}

// The same with the scale already in hand (1 when there is none: t * 1 == t exactly).
__device__ __forceinline__ float conv_sum_s(float acc, float bias, float scale, float res) {
#pragma clang fp contract(off)
    float t = acc + bias;
    t = t * scale;
    return t + res;
}

// XCD-aware tile order: dispatch slot b runs on XCD b % 8; each XCD takes a contiguous range of
// tiles ordered (N group, lane, m, n within the group), N fastest within a group. An M tile's
// window is fetched into one L2 and reused by the group's N tiles there, and a group's weight
// slices stay in that L2 while the lanes' M tiles pass (pick_tiles_ng sizes the group to fit;
// with one group this is the plain (lane, m, n) order). Returns false for the padding slots past
// the last tile.
__device__ __forceinline__ bool conv_tile_coords(const ConvArgs &p, int &lane_idx, int &m_tile, int &n_tile) {
    const int tile = (blockIdx.x & 7) * p.tiles_per_xcd + (blockIdx.x >> 3);
    if (tile >= p.total_tiles) return false;
    const int per_group = p.total_tiles / p.tiles_n * p.tiles_ng;  // lanes * tiles_m * tiles_ng
    const int group = tile / per_group;
    const int rest = tile - group * per_group;
    n_tile = group * p.tiles_ng + rest % p.tiles_ng;
    const int mm = rest / p.tiles_ng;  // lane * tiles_m + m
    m_tile = mm % p.tiles_m;
    lane_idx = mm / p.tiles_m;
    return true;
}

// Slot of segment q in row r for direct staging: with 64 banks of 4 bytes a ds_read_b128 serves
// 16 lanes per cycle, and a fragment read has those 16 lanes on 16 consecutive rows at one
// segment. Rows r and r + 128/KC share a 256-byte bank sweep, so the swizzle is (r / (128/KC))
// mod SEGS: the 16 rows land on 16 distinct 16-byte bank groups from any starting row. It only
// looks at row bits below 5, so rows 32 apart (the TM/TN fragments) share it.
template <int KC>
__device__ __forceinline__ int seg_swizzle(int r) {
    constexpr int SHIFT = KC == 16 ? 3 : (KC == 32 ? 2 : 1);  // log2(128 / KC)
    return (static_cast<unsigned>(r) >> SHIFT) & (KC / 8 - 1);
}

typedef __attribute__((address_space(3))) void lds_void_t;
constexpr int kBufferWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, no swizzle
constexpr uint32_t kOutOfRange = 0x80000000u;
typedef unsigned v4u_t __attribute__((ext_vector_type(4)));  // a 16-byte buffer load or store

__device__ __forceinline__ void load_lds_16(__amdgpu_buffer_rsrc_t rs, char *lds, uint32_t voffset,
                                            uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t *)lds, 16, voffset, soffset, 0, 0);
}

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Waits until at most N of this wave's vector-memory operations are in flight.
template <int N>
__device__ __forceinline__ void wait_vmem_le() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The workgroup barrier between pipeline stages. __syncthreads() carries a workgroup release
// fence, which the compiler lowers to s_waitcnt vmcnt(0) before the s_barrier: every vector-memory
// operation of the wave has to finish, the loads of the stages still being prefetched too, so a
// deeper pipeline degenerates into one full memory round trip per chunk. Here the caller has
// already waited (vmcnt) for exactly the loads the barrier publishes -- its share of the next
// stage -- and this waits for the wave's own LDS accesses only; later loads stay in flight.
// The asm is also a compiler barrier for memory: no access moves across it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Load instructions a wave issues per chunk, at least: instruction j of a region belongs to wave
// j % nw, and the region has at least `inst` instructions.
constexpr int loads_of_wave(int wave, int nw, int inst) { return wave < inst ? (inst - wave + nw - 1) / nw : 0; }
constexpr int min_loads_per_wave(int nw, int a_inst, int b_inst) {
    int m = 1 << 30;
    for (int w = 0; w < nw; ++w) {
        const int c = loads_of_wave(w, nw, a_inst) + loads_of_wave(w, nw, b_inst);
        m = c < m ? c : m;
    }
    return m;
}

// The k taps of one staged chunk on the matrix cores. KT > 0 is the tap count known at compile
// time: the loop unrolls into straight-line code, and with PIPE two fragment sets alternate: tap
// t+1's reads are interleaved with tap t's MFMAs, and the wait before an MFMA counts only tap t's
// reads (without PIPE, the compiler schedules one set). KT == 0 takes k at run time.
// frag_a(t, kk, i) / frag_b(t, kk, j) give the 16-byte fragment addresses of 32-row block i (or
// column block j) at k-step kk of tap t.
template <typename Cfg, int KT, bool PIPE, typename FA, typename FB>
__device__ __forceinline__ void mma_taps(int k, FA frag_a, FB frag_b, float16_t (&acc)[Cfg::TM][Cfg::TN]) {
    constexpr int KS = Cfg::KC / 16;
    typedef half8_t FragA[KS][Cfg::TM];
    typedef half8_t FragB[KS][Cfg::TN];
    auto load = [&](int t, FragA &a, FragB &b) {
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
            for (int i = 0; i < Cfg::TM; ++i) a[kk][i] = *frag_a(t, kk, i);
#pragma unroll
            for (int j = 0; j < Cfg::TN; ++j) b[kk][j] = *frag_b(t, kk, j);
        }
    };
    auto mma = [&](const FragA &a, const FragB &b) {
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
#pragma unroll
            for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
                for (int j = 0; j < Cfg::TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[kk][j], a[kk][i], acc[i][j], 0, 0, 0);
    };
    if constexpr (KT > 0 && PIPE) {
        FragA a[2];
        FragB b[2];
        load(0, a[0], b[0]);
#pragma unroll
        for (int t = 0; t < KT; ++t) {
            if (t + 1 < KT) load(t + 1, a[(t + 1) & 1], b[(t + 1) & 1]);
            mma(a[t & 1], b[t & 1]);
            // tap t+1's fragment reads go out one at a time between tap t's MFMAs, so the LDS
            // queue and the matrix pipe stay busy together
#pragma unroll
            for (int m = 0; m < KS * Cfg::TM * Cfg::TN; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    } else if constexpr (KT > 0) {
#pragma unroll
        for (int t = 0; t < KT; ++t) {
            FragA a;
            FragB b;
            load(t, a, b);
            mma(a, b);
        }
    } else {
        for (int t = 0; t < k; ++t) {
            FragA a;
            FragB b;
            load(t, a, b);
            mma(a, b);
        }
    }
}

// acc += window(x) . w over all taps for the workgroup's BM x BN tile, register staging.
template <typename Cfg, bool SNAKE_IN, int KT>
__device__ __forceinline__ void conv_mainloop_regs(const ConvArgs &p, const half_t *xl, int l0, int n0, char *smem,
                                                   float16_t (&acc)[Cfg::TM][Cfg::TN]) {
    constexpr int LDA = Cfg::LDA;
    constexpr int STAGE_H = Cfg::STAGE_BYTES / 2;
    constexpr int A_H = Cfg::A_BYTES / 2;
    half_t *As = reinterpret_cast<half_t *>(smem);
    half_t *Bs = As + A_H;
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
    static_assert(Cfg::THREADS % Cfg::SEGS == 0, "a thread's segments share one channel group");
    auto store_chunk = [&](int c0, half_t *A, half_t *B) {
        float ka[8], kr[8];
        if constexpr (SNAKE_IN) {
            const int c = c0 + (tid % Cfg::SEGS) * 8;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                ka[j] = p.a_in[c + j] * kInv2Pi;
                kr[j] = p.r_in[c + j];
            }
        }
#pragma unroll
        for (int i = 0; i < Cfg::A_PER_T; ++i) {
            const int seg = tid + i * Cfg::THREADS;
            if (seg < Cfg::A_SEGS) {
                const int r = seg / Cfg::SEGS;
                const int q = seg % Cfg::SEGS;
                half8_t v = ra[i];
                if constexpr (SNAKE_IN) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[j] = snake_f16k(v[j], ka[j], kr[j]);
                }
                *reinterpret_cast<half8_t *>(A + r * LDA + q * 8) = v;
            }
        }
#pragma unroll
        for (int i = 0; i < Cfg::B_PER_T; ++i) {
            const int seg = tid + i * Cfg::THREADS;
            if (seg < Cfg::B_SEGS) {
                const int row = seg / Cfg::SEGS;
                const int q = seg % Cfg::SEGS;
                *reinterpret_cast<half8_t *>(B + row * LDA + q * 8) = rb[i];
            }
        }
    };

    const int nchunks = p.cin / Cfg::KC;
    const int arow0 = wm * Cfg::WTM + (lane & 31);
    const int bcol0 = wn * Cfg::WTN + (lane & 31);
    const int koff = (lane >> 5) * 8;
    auto compute = [&](const half_t *A, const half_t *B) {
        const half_t *a0 = A + arow0 * LDA + koff;
        const half_t *b0 = B + bcol0 * LDA + koff;
        mma_taps<Cfg, KT, false>(
            p.k,
            [&](int t, int kk, int i) {
                return reinterpret_cast<const half8_t *>(a0 + (t * p.dil + i * 32) * LDA + kk * 16);
            },
            [&](int t, int kk, int j) {
                return reinterpret_cast<const half8_t *>(b0 + (t * Cfg::BN + j * 32) * LDA + kk * 16);
            },
            acc);
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
            if (c + 1 < nchunks) load_chunk((c + 1) * Cfg::KC);
            compute(As + cur * STAGE_H, Bs + cur * STAGE_H);
            if (c + 1 < nchunks) store_chunk((c + 1) * Cfg::KC, As + (cur ^ 1) * STAGE_H, Bs + (cur ^ 1) * STAGE_H);
            __syncthreads();
        }
    }
}

// acc += window(x) . w over all taps for the workgroup's BM x BN tile, direct staging.
// SPLIT: x holds f32 values as f16 pairs, each row [hi(cs) | lo(cs)] with cs = cin / 3, and the
// reduction runs over K' = 3 cs channels per tap: chunks of the first third read hi, of the
// second lo, of the third hi again, against weights [w_hi | w_hi | w_lo] (so the sum is
// xh.wh + xl.wh + xh.wl); only the window's source offset changes.
template <typename Cfg, bool SNAKE_IN, int KT, bool SPLIT = false>
__device__ __forceinline__ void conv_mainloop_direct(const ConvArgs &p, const half_t *xl, int l0, int n0, char *smem,
                                                     float16_t (&acc)[Cfg::TM][Cfg::TN]) {
    static_assert(!(SPLIT && SNAKE_IN), "split operands take no prologue SnakeBeta");
    constexpr int RB = Cfg::ROW_BYTES;
    constexpr int SEGS = Cfg::SEGS;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: load guards stay scalar
    const int lane = tid & 63;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
    const int rows = Cfg::BM + (p.k - 1) * p.dil;
    const int win0 = l0 - p.pad_left;
    const int K = p.k * p.cin;
    const int cs = SPLIT ? p.cin / 3 : p.cin;    // channels of a stored row (per half when SPLIT)
    const int x_ld = SPLIT ? 2 * cs : p.cin;     // halves per stored row
    // the stored offset of K' chunk c0: hi for the first and third thirds, lo for the second
    auto x_off = [&](int c0) { return SPLIT && c0 >= 2 * cs ? c0 - 2 * cs : c0; };
    const int a_inst = (rows + Cfg::RPI - 1) / Cfg::RPI;
    const int b_inst = (KT > 0 ? KT : p.k) * Cfg::BN / Cfg::RPI;
    const __amdgpu_buffer_rsrc_t rsa =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t *>(xl), 0, p.L * x_ld * 2, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rsb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t *>(p.w), 0, p.cout * K * 2, kBufferWord3);

    // Per-lane byte offsets of the slots this wave's load instructions fill; a chunk adds c0*2.
    // Instruction j covers slots j*64 .. j*64+63 of its region; lane l fills slot j*64+l, which
    // holds segment (slot % SEGS) ^ swizzle(row) of row slot / SEGS.
    uint32_t va[Cfg::A_PER_W], vb[Cfg::B_PER_W];
#pragma unroll
    for (int i = 0; i < Cfg::A_PER_W; ++i) {
        const int slot = (wave + i * Cfg::NW) * 64 + lane;
        const int r = slot / SEGS;
        const int q = (slot % SEGS) ^ seg_swizzle<Cfg::KC>(r);
        const int s = win0 + r;
        va[i] = (r < rows && s >= 0 && s < p.L) ? static_cast<uint32_t>((s * x_ld + q * 8) * 2) : kOutOfRange;
    }
#pragma unroll
    for (int i = 0; i < Cfg::B_PER_W; ++i) {
        const int slot = (wave + i * Cfg::NW) * 64 + lane;
        const int r = slot / SEGS;  // t * BN + n
        const int q = (slot % SEGS) ^ seg_swizzle<Cfg::KC>(r);
        const int t = r / Cfg::BN;
        const int n = r - t * Cfg::BN;
        vb[i] = static_cast<uint32_t>(((n0 + n) * K + t * p.cin + q * 8) * 2);
    }
    auto issue = [&](int c0, int st) {
        char *base = smem + st * Cfg::STAGE_BYTES;
        const uint32_t so = static_cast<uint32_t>(c0 * 2);
        const uint32_t sx = static_cast<uint32_t>(x_off(c0) * 2);
#pragma unroll
        for (int i = 0; i < Cfg::A_PER_W; ++i) {
            const int j = wave + i * Cfg::NW;
            if (j < a_inst) load_lds_16(rsa, base + j * 1024, va[i], sx);
        }
#pragma unroll
        for (int i = 0; i < Cfg::B_PER_W; ++i) {
            const int j = wave + i * Cfg::NW;
            if (j < b_inst) load_lds_16(rsb, base + Cfg::A_BYTES + j * 1024, vb[i], so);
        }
    };
    // SnakeBeta on the window slots this lane loaded (after they landed): rows outside the
    // sequence hold zeros and snake(0) = 0, so they are skipped.
    auto snake_stage = [&](int c0, int st) {
        char *base = smem + st * Cfg::STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < Cfg::A_PER_W; ++i) {
            const int j = wave + i * Cfg::NW;
            if (j < a_inst && va[i] != kOutOfRange) {
                const int slot = j * 64 + lane;
                const int q = (slot % SEGS) ^ seg_swizzle<Cfg::KC>(slot / SEGS);
                half8_t *sp = reinterpret_cast<half8_t *>(base + slot * 16);
                half8_t v = *sp;
                const int c = c0 + q * 8;
                const float4_t a0 = *reinterpret_cast<const float4_t *>(p.a_in + c);
                const float4_t a1 = *reinterpret_cast<const float4_t *>(p.a_in + c + 4);
                const float4_t r0 = *reinterpret_cast<const float4_t *>(p.r_in + c);
                const float4_t r1 = *reinterpret_cast<const float4_t *>(p.r_in + c + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = snake_f16k(v[e], a0[e] * kInv2Pi, r0[e]);
                    v[e + 4] = snake_f16k(v[e + 4], a1[e] * kInv2Pi, r1[e]);
                }
                *sp = v;
            }
        }
    };

    const int nchunks = p.cin / Cfg::KC;
    const int arow0 = wm * Cfg::WTM + (lane & 31);
    const int bcol0 = wn * Cfg::WTN + (lane & 31);
    const int qh = lane >> 5;
    auto compute = [&](int st) {
        const char *A = smem + st * Cfg::STAGE_BYTES;
        const char *B = A + Cfg::A_BYTES;
        mma_taps<Cfg, KT, true>(
            p.k,
            [&](int t, int kk, int i) {
                const int r = arow0 + t * p.dil;
                return reinterpret_cast<const half8_t *>(A + (r + i * 32) * RB +
                                                         (((kk * 2 + qh) ^ seg_swizzle<Cfg::KC>(r)) << 4));
            },
            [&](int t, int kk, int j) {
                const int r = t * Cfg::BN + bcol0;
                return reinterpret_cast<const half8_t *>(B + (r + j * 32) * RB +
                                                         (((kk * 2 + qh) ^ seg_swizzle<Cfg::KC>(r)) << 4));
            },
            acc);
    };
    // NBUF stages: chunk c+NBUF-1 is issued while chunk c is multiplied. vmcnt counts this wave's
    // loads in issue order, so chunk c+1 has landed once no more than the loads of the chunks
    // after it remain; the bound uses the fewest loads any wave issues per chunk (the narrowest
    // window), which can only wait longer, never shorter.
    constexpr int S = Cfg::NBUF;
    constexpr int PMIN = min_loads_per_wave(Cfg::NW, (Cfg::BM + Cfg::RPI - 1) / Cfg::RPI,
                                            (KT > 0 ? KT : 1) * Cfg::BN / Cfg::RPI);
    constexpr int LATER = (S - 2) * PMIN;
    auto wait_for_next = [&](int later_chunks) {
        if (later_chunks >= S - 2)
            wait_vmem_le<LATER>();
        else
            wait_vmem();
    };
#pragma unroll
    for (int st = 0; st < S - 1; ++st)
        if (st < nchunks) issue(st * Cfg::KC, st);
    wait_for_next(nchunks - 1);
    if constexpr (SNAKE_IN) snake_stage(0, 0);
    stage_barrier();
    int st = 0;          // stage holding chunk c
    int st_new = S - 1;  // stage receiving chunk c + S - 1
    if constexpr (!SNAKE_IN && KT >= 3) {
        // The taps of all chunks as one stream: tap t+1's fragment reads go out between tap t's
        // MFMAs, across chunk boundaries too. The barrier sits before the last tap's MFMAs, once
        // that tap's reads are back in registers: every wave has then finished reading the chunk
        // (its stage may be refilled) and the next chunk has landed (its first tap can be read in
        // the shadow of this tap's MFMAs) -- instead of every wave starting each chunk with its
        // first reads exposed behind the barrier. Measured A/B: the k=7 convs 3-5% faster; with
        // one or two taps per chunk (k=1, the transposed convs) the chunk-end barrier is better.
        constexpr int KS = Cfg::KC / 16;
        half8_t fa[2][KS][Cfg::TM], fb[2][KS][Cfg::TN];
        auto load = [&](int s, int t, half8_t (&a)[KS][Cfg::TM], half8_t (&b)[KS][Cfg::TN]) {
            const char *A = smem + s * Cfg::STAGE_BYTES;
            const char *B = A + Cfg::A_BYTES;
            const int ra = arow0 + t * p.dil, rb = t * Cfg::BN + bcol0;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
                for (int i = 0; i < Cfg::TM; ++i)
                    a[kk][i] = *reinterpret_cast<const half8_t *>(
                        A + (ra + i * 32) * RB + (((kk * 2 + qh) ^ seg_swizzle<Cfg::KC>(ra)) << 4));
#pragma unroll
                for (int j = 0; j < Cfg::TN; ++j)
                    b[kk][j] = *reinterpret_cast<const half8_t *>(
                        B + (rb + j * 32) * RB + (((kk * 2 + qh) ^ seg_swizzle<Cfg::KC>(rb)) << 4));
            }
        };
        auto mma = [&](const half8_t (&a)[KS][Cfg::TM], const half8_t (&b)[KS][Cfg::TN]) {
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
#pragma unroll
                for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
                    for (int j = 0; j < Cfg::TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[kk][j], a[kk][i], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int m = 0; m < KS * Cfg::TM * Cfg::TN; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        int c = 0;
        // PAR: the fragment set of the chunk's tap 0 (tap t uses set (t + PAR) & 1); it flips
        // from chunk to chunk when KT is odd, so chunks run in pairs with PAR fixed at compile time
        auto chunk = [&](auto par) {
            constexpr int PAR = decltype(par)::value;
            if (c + S - 1 < nchunks) issue((c + S - 1) * Cfg::KC, st_new);
            const bool more = c + 1 < nchunks;
            const int st_next = st + 1 == S ? 0 : st + 1;
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                const int cur = (t + PAR) & 1;
                if (t + 1 < KT) {
                    load(st, t + 1, fa[cur ^ 1], fb[cur ^ 1]);
                } else if (more) {
                    wait_for_next(nchunks - 2 - c);
                    stage_barrier();
                    load(st_next, 0, fa[cur ^ 1], fb[cur ^ 1]);
                }
                mma(fa[cur], fb[cur]);
            }
            st = st_next;
            st_new = st_new + 1 == S ? 0 : st_new + 1;
            ++c;
        };
        load(st, 0, fa[0], fb[0]);
        while (c + 1 < nchunks) {
            chunk(std::integral_constant<int, 0>{});
            chunk(std::integral_constant<int, KT & 1>{});
        }
        if (c < nchunks) chunk(std::integral_constant<int, 0>{});
        __syncthreads();
        return;
    }
    for (int c = 0; c < nchunks; ++c) {
        if (c + S - 1 < nchunks) issue((c + S - 1) * Cfg::KC, st_new);
        compute(st);
        const int st_next = st + 1 == S ? 0 : st + 1;
        if (c + 1 < nchunks) {
            wait_for_next(nchunks - 2 - c);
            if constexpr (SNAKE_IN) snake_stage((c + 1) * Cfg::KC, st_next);
        }
        stage_barrier();
        st = st_next;
        st_new = st_new + 1 == S ? 0 : st_new + 1;
    }
}

// acc += sum over taps and cin of window(x) . w; ends on a barrier, after which all of smem is
// free. KT: the tap count when the launch fixed it at compile time (== p.k), else 0.
template <typename Cfg, bool SNAKE_IN, int KT>
__device__ __forceinline__ void conv_mainloop(const ConvArgs &p, const half_t *xl, int l0, int n0, char *smem,
                                              float16_t (&acc)[Cfg::TM][Cfg::TN]) {
    if constexpr (Cfg::STAGING == kStageDirect)
        conv_mainloop_direct<Cfg, SNAKE_IN, KT>(p, xl, l0, n0, smem, acc);
    else
        conv_mainloop_regs<Cfg, SNAKE_IN, KT>(p, xl, l0, n0, smem, acc);
}

// Fills the output SnakeBeta table (a/2pi and r for the tile's BN channels) after the stages and
// the epilogue's staging area; the main loop's barriers make it visible before the epilogue.
template <typename Cfg>
__device__ __forceinline__ void conv_snake_table(char *smem, int n0, const float *a_out, const float *r_out) {
    if (!a_out) return;
    float *tab = reinterpret_cast<float *>(smem + Cfg::TAB_OFFSET);
    for (int c = threadIdx.x; c < Cfg::BN; c += Cfg::THREADS) {
        tab[c] = a_out[n0 + c] * kInv2Pi;
        tab[Cfg::BN + c] = r_out[n0 + c];
    }
}

// Orders this wave's LDS accesses before and after it (the LDS executes one wave's instructions
// in issue order, so lanes then see each other's earlier writes; the fence stops the compiler
// from moving accesses across).
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Writes acc (+ bias, + residual, act, rounded; y_pre; SnakeBeta_out; y) for the tile, one 32-row
// block per wave at a time through the wave's own LDS region. The products are transposed
// (D[channel][position]): a lane holds one position and runs of four consecutive channels, which
// go to LDS as 16-byte writes; rows then come back 8 channels per lane, so bias, residual and the
// stores move 16 coalesced bytes per lane. The bias and the first block's residual rows are
// requested up front, each next block's residual rows while the current block is written. The
// residual, y_pre and y rows are reached through buffer resources bounded to the lane's rows
// (lmax * ld halves, under 2^31 bytes: the route's eligibility checks it); a position past the
// sequence gets an offset beyond them, so its loads read zeros and its stores are dropped, and no
// branch splits a block. `ld` is the output row length (cout), `n0` the tile's first output
// channel, `lmax` the lane's length. Called after the main loop's closing barrier (smem free).
// PLAIN: no activation and no scale, known at compile time. The general form reads act and scale
// at run time, but they are uniform over the tile: branching on them per element costs more scalar
// instructions and branches than the epilogue's arithmetic, so the caller picks a form once.
template <typename Cfg, bool PLAIN>
__device__ __forceinline__ void conv_epilogue_form(const float16_t (&acc)[Cfg::TM][Cfg::TN], char *smem, int64_t row0,
                                                   int l0, int n0, int lmax, int ld, const half_t *bias,
                                                   const half_t *res, half_t *y_pre, half_t *y, const float *a_out,
                                                   int act, const float *scale) {
    constexpr int CG = Cfg::WTN / 8;  // 8-channel groups per wave row
    constexpr int NG = 32 * CG / 64;  // groups per lane per 32-row block
    static_assert((32 * CG) % 64 == 0, "a 32-row block splits evenly over the lanes");
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int l32 = lane & 31, hf = lane >> 5;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
    float *E = reinterpret_cast<float *>(smem) + wave * 32 * Cfg::EPI_PITCH;
    const int nw = n0 + wn * Cfg::WTN;
    const float *tab = reinterpret_cast<const float *>(smem + Cfg::TAB_OFFSET);
    // the residual rows of two 32-row blocks are live at a time: block i+1's are requested while
    // block i is written (all TM blocks at once left the 128 x 64 wave tile spilling)
    half8_t rr[2][NG], bb[NG];
#pragma unroll
    for (int u = 0; u < NG; ++u) {
        const int cg = (lane + 64 * u) % CG;
        bb[u] = bias ? *reinterpret_cast<const half8_t *>(bias + nw + cg * 8) : half8_t{};
    }
    const uint32_t lane_bytes = static_cast<uint32_t>(static_cast<int64_t>(lmax) * ld * 2);
    const int64_t base = row0 * ld;
    const __amdgpu_buffer_rsrc_t rs_res =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t *>(res ? res + base : y + base), 0, lane_bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rs_y = __builtin_amdgcn_make_buffer_rsrc(y + base, 0, lane_bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rs_yp =
        __builtin_amdgcn_make_buffer_rsrc(y_pre ? y_pre + base : y + base, 0, lane_bytes, kBufferWord3);
    auto out_off = [&](int l, int n) -> uint32_t {
        return l < lmax ? static_cast<uint32_t>((static_cast<int64_t>(l) * ld + n) * 2) : kOutOfRange;
    };
    auto load_res = [&](int i, half8_t (&dst)[NG]) {
        const int lb = l0 + wm * Cfg::WTM + i * 32;
#pragma unroll
        for (int u = 0; u < NG; ++u) {
            const int g = lane + 64 * u;
            const int mr = g / CG, cg = g - (g / CG) * CG;
            dst[u] = half8_t{};
            if (res)
                dst[u] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(rs_res, out_off(lb + mr, nw + cg * 8), 0, 0));
        }
    };
    load_res(0, rr[0]);
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i) {
        const int lb = l0 + wm * Cfg::WTM + i * 32;
        if (i + 1 < Cfg::TM) load_res(i + 1, rr[(i + 1) & 1]);
        if (i > 0) wave_lds_order();  // the wave's reads of block i-1 precede these writes
        // the bias stays f16 until used: the compiler would otherwise convert it once for all
        // blocks and hold 8 NG f32 registers through the epilogue (A/B with both changes: the
        // 256 x 128 and 128 x 96 transposed convs 4-5% faster, no spills)
#pragma unroll
        for (int u = 0; u < NG; ++u) asm volatile("" : "+v"(bb[u]));
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
            const float4_t *src = reinterpret_cast<const float4_t *>(E + mr * Cfg::EPI_PITCH + cg * 8);
            const float4_t v0 = src[0], v1 = src[1];
            float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            const uint32_t off = out_off(l, n);
            half8_t h;
            if constexpr (PLAIN) {
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    h[q] = static_cast<half_t>(conv_sum_s(v[q], static_cast<float>(bb[u][q]), 1.0f,
                                                          static_cast<float>(rr[i & 1][u][q])));
            } else {
                float sc[8] = {1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f};
                if (scale) {
                    const float4_t s0 = *reinterpret_cast<const float4_t *>(scale + n);
                    const float4_t s1 = *reinterpret_cast<const float4_t *>(scale + n + 4);
                    sc[0] = s0[0], sc[1] = s0[1], sc[2] = s0[2], sc[3] = s0[3];
                    sc[4] = s1[0], sc[5] = s1[1], sc[6] = s1[2], sc[7] = s1[3];
                }
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    v[q] = conv_sum_s(v[q], static_cast<float>(bb[u][q]), sc[q], static_cast<float>(rr[i & 1][u][q]));
                // one branch on the (uniform) activation per eight values
                switch (act) {
                case 1:
#pragma unroll
                    for (int q = 0; q < 8; ++q) h[q] = static_cast<half_t>(conv_act(v[q], 1));
                    break;
                case 2:
#pragma unroll
                    for (int q = 0; q < 8; ++q) h[q] = static_cast<half_t>(conv_act(v[q], 2));
                    break;
                case 3:
#pragma unroll
                    for (int q = 0; q < 8; ++q) h[q] = static_cast<half_t>(conv_act(v[q], 3));
                    break;
                default:
#pragma unroll
                    for (int q = 0; q < 8; ++q) h[q] = static_cast<half_t>(v[q]);
                }
            }
            if (y_pre) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u_t, h), rs_yp, off, 0, 0);
            if (a_out) {
                const int c = n - n0;
                const float4_t ka0 = *reinterpret_cast<const float4_t *>(tab + c);
                const float4_t ka1 = *reinterpret_cast<const float4_t *>(tab + c + 4);
                const float4_t kr0 = *reinterpret_cast<const float4_t *>(tab + Cfg::BN + c);
                const float4_t kr1 = *reinterpret_cast<const float4_t *>(tab + Cfg::BN + c + 4);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    h[q] = snake_f16k(h[q], ka0[q], kr0[q]);
                    h[q + 4] = snake_f16k(h[q + 4], ka1[q], kr1[q]);
                }
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u_t, h), rs_y, off, 0, 0);
        }
    }
}

template <typename Cfg>
__device__ __forceinline__ void conv_epilogue(const float16_t (&acc)[Cfg::TM][Cfg::TN], char *smem, int64_t row0,
                                              int l0, int n0, int lmax, int ld, const half_t *bias, const half_t *res,
                                              half_t *y_pre, half_t *y, const float *a_out, int act,
                                              const float *scale) {
    if (act == 0 && !scale)
        conv_epilogue_form<Cfg, true>(acc, smem, row0, l0, n0, lmax, ld, bias, res, y_pre, y, a_out, 0, nullptr);
    else
        conv_epilogue_form<Cfg, false>(acc, smem, row0, l0, n0, lmax, ld, bias, res, y_pre, y, a_out, act, scale);
}

}  // namespace dtts
