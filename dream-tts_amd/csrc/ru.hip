// The codec's residual unit as one kernel (ResidualUnit::forward, crates/qwen3tts/src/codec.rs:
// 215-229):
//
//   h  = f16(conv_k,dil(SnakeBeta1(u)) + b1)          conv1, the chunked main loop
//   h2 = f16(SnakeBeta2(h))                           in registers
//   y  = f16(conv_1(h2) + b2 + u)                     conv2, from registers
//   out = y, and/or f16(SnakeBeta_next(y))
//
// A workgroup owns BM positions x all C channels, so the k=1 conv's whole reduction (C) is in the
// workgroup after conv1: h and h2 never reach HBM. Per unit the activation traffic is two passes
// (read u with its halo, write y) instead of the unfused chain's five, and every value rounded
// to f16 here is one the unfused chain stores.
//
// The matrix products are computed transposed, D[channel][position] = W . X^T, so the MFMA result
// a lane holds is one position x 16 channels (four runs of four consecutive channels). That makes
// conv2 free of any data movement: the f16-packed h2 values of a lane are exactly the B operand
// conv2 needs at that position, provided conv2's reduction index runs over the channels in the
// same order -- so the A operand (W2) is read in that order, two 8-byte pieces per fragment.
// The epilogues work on four consecutive channels per access, and the biases start the
// accumulators.
//
// Main loop, per KC-channel chunk: the dilated window of u (BM + (k-1)*dil rows) is loaded into
// registers two or three chunks ahead, SnakeBeta'd in f32 (fma_mix reads the f16 directly) and
// written to LDS while the previous chunk is on the matrix cores; W1's slice for the chunk goes straight
// from memory to LDS (buffer_load ... lds), XOR-swizzled rows. Two LDS stages, one barrier per
// chunk.
#include "conv_tile.hpp"

namespace dtts {
namespace {

struct RuArgs {
    const half_t *u;    // [lanes, L, C]: the input and the residual
    const half_t *w1;   // [C, k*C] tap-major
    const half_t *w2;   // [C, C]
    const half_t *b1, *b2;
    const float *a1, *r1, *a2, *r2, *a_out, *r_out;
    half_t *y_pre, *y;
    int L, k, dil, pad_left;
    int tiles_m, total_tiles, tiles_per_xcd;
};

// C channels; a wave owns WP positions x all C channels; NW waves; KC channels per chunk; WPE_:
// waves per SIMD the registers are budgeted for (0: as many as the LDS lets workgroups share a CU).
template <int C_, int WP_, int NW_, int KC_, int WPE_ = 0>
struct RuCfg {
    static constexpr int C = C_, WP = WP_, NW = NW_, KC = KC_;
    static constexpr int BM = WP * NW;  // positions per workgroup
    static constexpr int THREADS = 64 * NW;
    static constexpr int TM = WP / 32;  // 32-position blocks per wave
    static constexpr int TN = C / 32;   // 32-channel blocks
    static constexpr int KMAX = 7, HMAX = 64;
    static constexpr int CHUNKS = C / KC;
    // window: BM + HMAX rows x KC halves, rows padded by 8 halves (16 consecutive rows at one
    // 16-byte segment then hit 16 distinct 4-bank groups)
    static constexpr int ROWS = BM + HMAX;
    static constexpr int SEGS = KC / 8;
    static constexpr int APITCH = KC + 8;
    static constexpr int A_BYTES = ROWS * APITCH * 2;
    static constexpr int A_SEGS = ROWS * SEGS;
    static constexpr int A_PER_T = (A_SEGS + THREADS - 1) / THREADS;
    // W1 slice: KMAX * C rows (tap-major, t * C + channel) x KC halves, direct loads of 1 KiB
    static constexpr int RPI = 1024 / (KC * 2);
    static constexpr int B_BYTES = KMAX * C * KC * 2;
    static constexpr int B_INST = KMAX * C / RPI;
    static constexpr int B_PER_W = (B_INST + NW - 1) / NW;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int TAB_BYTES = 8 * C * 4;
    static constexpr int LDS = 2 * STAGE + TAB_BYTES;
    static constexpr int MIN_WG = 2 * LDS <= 160 * 1024 ? 2 : 1;
    // __launch_bounds__'s second argument is waves per SIMD: workgroups per CU x NW / 4
    static constexpr int WPE = WPE_ > 0 ? WPE_ : (MIN_WG * NW + 3) / 4;
    static constexpr int WPE_ARG = WPE_;
    // W2 in LDS for conv2, written once the main loop is done (both stages are free then):
    // rows padded to C + 8 halves (16 consecutive rows at one 16-byte column hit distinct banks)
    static constexpr int W2_PITCH = C + 8;
    static constexpr int W2_SEGS = C * C / 8;
    static constexpr int W2_PER_T = (W2_SEGS + THREADS - 1) / THREADS;
    static_assert(C % 32 == 0 && C % KC == 0 && WP % 32 == 0 && KC == 16, "residual-unit tile shape");
    static_assert(THREADS % SEGS == 0, "a thread's window segments share one channel group");
    static_assert((KMAX * C) % RPI == 0 && RPI % 32 == 0, "whole direct-load instructions per tap");
    static_assert(C * W2_PITCH * 2 <= 2 * STAGE, "W2 fits the stages");
    // output staging: a 32-row block per wave, rows of C + 4 halves (an odd multiple of 4 bytes
    // over 64 banks puts the 8-byte writes of 32 consecutive rows on distinct bank pairs)
    static constexpr int OPITCH = C + 4;
    static_assert(NW * 32 * OPITCH * 2 <= 2 * STAGE, "output staging fits the stages");
};

// C = 96: two 32-position blocks per wave, two workgroups per CU. C = 192: one block per wave
// (96 accumulator registers either way), eight waves, one workgroup per CU.
typedef RuCfg<96, 64, 4, 16> RuTile96;
typedef RuCfg<192, 32, 8, 16> RuTile192;

typedef _Float16 half4_v __attribute__((ext_vector_type(4)));

// SnakeBeta on an f16 value with ka = alpha / 2pi: the product reads the f16 directly (fma_mix),
// the sine takes revolutions after the fract reduction, and the result is rounded once to f16.
__device__ __forceinline__ half_t snake_h(half_t x, float ka, float r) {
    const float t = __builtin_fmaf(static_cast<float>(x), ka, 0.0f);
    const float s = __builtin_amdgcn_sinf(__builtin_amdgcn_fractf(t));
    return static_cast<half_t>(__builtin_fmaf(r, s * s, static_cast<float>(x)));
}

template <typename Cfg, int KT>
__global__ __launch_bounds__(Cfg::THREADS, Cfg::WPE) void ru_nlc_f16(RuArgs q) {
    constexpr int C = Cfg::C, KC = Cfg::KC, SEGS = Cfg::SEGS, TM = Cfg::TM, TN = Cfg::TN, NW = Cfg::NW;
    constexpr int APITCH = Cfg::APITCH;
    __shared__ __attribute__((aligned(16))) char smem[Cfg::LDS];
    const int tile = (blockIdx.x & 7) * q.tiles_per_xcd + (blockIdx.x >> 3);
    if (tile >= q.total_tiles) return;
    const int m_tile = tile % q.tiles_m;
    const int lane_idx = tile / q.tiles_m;
    const int l0 = m_tile * Cfg::BM;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int l32 = lane & 31, hf = lane >> 5;
    const int k = KT > 0 ? KT : q.k;
    const int rows = Cfg::BM + (k - 1) * q.dil;
    const int win0 = l0 - q.pad_left;
    const half_t *ul = q.u + static_cast<int64_t>(lane_idx) * q.L * C;

    // per-channel constants: ka1 r1 b1 ka2 r2 b2 ka_out r_out, f32
    float *tab = reinterpret_cast<float *>(smem + 2 * Cfg::STAGE);
    for (int c = tid; c < C; c += Cfg::THREADS) {
        tab[c] = q.a1[c] * kInv2Pi;
        tab[C + c] = q.r1[c];
        tab[2 * C + c] = static_cast<float>(q.b1[c]);
        tab[3 * C + c] = q.a2[c] * kInv2Pi;
        tab[4 * C + c] = q.r2[c];
        tab[5 * C + c] = static_cast<float>(q.b2[c]);
        if (q.a_out) {
            tab[6 * C + c] = q.a_out[c] * kInv2Pi;
            tab[7 * C + c] = q.r_out[c];
        }
    }

    // window segments of this thread: s = tid + i * THREADS -> row s / SEGS, segment tid % SEGS.
    // Where the last round of segments runs past the window, a thread takes the segment of a
    // thread that has one (same channel group) and stores the same value there: every load, snake
    // and store is unconditional, so no branch splits the main loop's scheduling regions. Rows
    // outside the window or the sequence read zeros through the buffer range check.
    constexpr int LAST = Cfg::A_SEGS - (Cfg::A_PER_T - 1) * Cfg::THREADS;  // segments of the last round
    static_assert(LAST > 0 && LAST % SEGS == 0, "window segment rounds");
    const __amdgpu_buffer_rsrc_t rsu =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t *>(ul), 0, q.L * C * 2, kBufferWord3);
    const int qd = tid % SEGS;
    uint32_t va[Cfg::A_PER_T];
    int arow[Cfg::A_PER_T];
#pragma unroll
    for (int i = 0; i < Cfg::A_PER_T; ++i) {
        const int s = i + 1 < Cfg::A_PER_T ? tid + i * Cfg::THREADS : (Cfg::A_PER_T - 1) * Cfg::THREADS + tid % LAST;
        const int r = s / SEGS;
        const int src = win0 + r;
        arow[i] = r;
        va[i] = (r < rows && src >= 0 && src < q.L) ? static_cast<uint32_t>((src * C + qd * 8) * 2) : kOutOfRange;
    }
    typedef half8_t WinRegs[Cfg::A_PER_T];
    auto win_load = [&](WinRegs &R, int c0) {
#pragma unroll
        for (int i = 0; i < Cfg::A_PER_T; ++i)
            R[i] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(rsu, va[i], c0 * 2, 0));
    };
    // SnakeBeta on the window registers, element g of the chunk (vector g / 8, lane element g % 8),
    // in place; the per-channel constants of the thread's channel group come from the table
    struct SnakeK {
        float4_t ka0, ka1, r0, r1;
    };
    auto snake_consts = [&](int c0) {
        const int c = c0 + qd * 8;
        return SnakeK{*reinterpret_cast<const float4_t *>(tab + c), *reinterpret_cast<const float4_t *>(tab + c + 4),
                      *reinterpret_cast<const float4_t *>(tab + C + c), *reinterpret_cast<const float4_t *>(tab + C + c + 4)};
    };
    auto snake_elems = [&](WinRegs &R, const SnakeK &kk, int g0, int g1) {
#pragma unroll
        for (int g = g0; g < g1; ++g) {
            const int i = g >> 3, e = g & 7;
            R[i][e] = snake_h(R[i][e], e < 4 ? kk.ka0[e & 3] : kk.ka1[e & 3], e < 4 ? kk.r0[e & 3] : kk.r1[e & 3]);
        }
    };
    auto win_write = [&](const WinRegs &R, char *stage) {
#pragma unroll
        for (int i = 0; i < Cfg::A_PER_T; ++i)
            *reinterpret_cast<half8_t *>(stage + arow[i] * APITCH * 2 + qd * 16) = R[i];
    };
    auto win_store = [&](WinRegs &R, int c0, char *stage) {
        const SnakeK kk = snake_consts(c0);
        snake_elems(R, kk, 0, 8 * Cfg::A_PER_T);
        win_write(R, stage);
    };

    // W1 slice of a chunk, straight to LDS: instruction j fills slots j*64 .. j*64+63; slot ->
    // row slot / SEGS (= t * C + channel), segment (slot % SEGS) ^ swizzle(row)
    const int K = k * C;
    const __amdgpu_buffer_rsrc_t rsw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t *>(q.w1), 0, C * K * 2, kBufferWord3);
    const int b_inst = k * C / Cfg::RPI;
    uint32_t vb[Cfg::B_PER_W];
#pragma unroll
    for (int i = 0; i < Cfg::B_PER_W; ++i) {
        const int slot = (wave + i * NW) * 64 + lane;
        const int r = slot / SEGS;
        const int qq = (slot % SEGS) ^ seg_swizzle<KC>(r);
        const int t = r / C;
        const int n = r - t * C;
        vb[i] = static_cast<uint32_t>((n * K + t * C + qq * 8) * 2);
    }
    auto w_issue = [&](int c0, char *stage) {
        char *base = stage + Cfg::A_BYTES;
#pragma unroll
        for (int i = 0; i < Cfg::B_PER_W; ++i) {
            const int j = wave + i * NW;
            if (j < b_inst) load_lds_16(rsw, base + j * 1024, vb[i], static_cast<uint32_t>(c0 * 2));
        }
    };

    // accumulators start at b1: acc[i][j][4g + e] is channel 32j + 8g + 4hf + e at position
    // 32i + l32 of the wave's block
    float16_t acc[TM][TN];
    __syncthreads();  // the table
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4_t b = *reinterpret_cast<const float4_t *>(tab + 2 * C + 32 * j + 8 * g + 4 * hf);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[i][j][4 * g + e] = b[e];
        }

    // fragments: window (B operand) rows wave*WP + 32i + l32 + t*dil, halves hf*8; W1 (A operand)
    // rows t*C + 32j + l32, segment hf ^ swizzle
    const int prow = wave * Cfg::WP + l32;
    // hook(t) runs in the same scheduling region as tap t's MFMAs, so its VALU work issues in
    // their shadow
    auto compute = [&](const char *stage, auto &&hook) {
        const char *A = stage;
        const char *B = stage + Cfg::A_BYTES;
        auto frag_x = [&](int t, int i) {
            return *reinterpret_cast<const half8_t *>(A + (prow + 32 * i + t * q.dil) * APITCH * 2 + hf * 16);
        };
        auto frag_w = [&](int t, int j) {
            const int r = t * C + 32 * j + l32;
            return *reinterpret_cast<const half8_t *>(B + r * (KC * 2) + ((hf ^ seg_swizzle<KC>(r)) << 4));
        };
        if constexpr (KT > 0) {
            half8_t fx[2][TM], fw[2][TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) fx[0][i] = frag_x(0, i);
#pragma unroll
            for (int j = 0; j < TN; ++j) fw[0][j] = frag_w(0, j);
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                if (t + 1 < KT) {
#pragma unroll
                    for (int i = 0; i < TM; ++i) fx[(t + 1) & 1][i] = frag_x(t + 1, i);
#pragma unroll
                    for (int j = 0; j < TN; ++j) fw[(t + 1) & 1][j] = frag_w(t + 1, j);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fw[t & 1][j], fx[t & 1][i], acc[i][j], 0, 0, 0);
                hook(t);
                // one MFMA, then a few VALU instructions (the hook's), in turn
#pragma unroll
                for (int m = 0; m < TM * TN; ++m) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x402, 4, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            for (int t = 0; t < k; ++t) {
                half8_t fx[TM], fw[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i) fx[i] = frag_x(t, i);
#pragma unroll
                for (int j = 0; j < TN; ++j) fw[j] = frag_w(t, j);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fw[j], fx[i], acc[i][j], 0, 0, 0);
            }
            hook(-1);
        }
    };

    // Pipeline. Chunk c computes from stage c & 1. During chunk c: W1 of chunk c+1 streams into
    // stage (c+1) & 1, the window of chunk c+PD into registers, and the registers holding chunk
    // c+1's window are snaked into stage (c+1) & 1. Stage (c+1) & 1 was last read by chunk c-1,
    // which every wave finished before the barrier that closed it.
    char *stage[2] = {smem, smem + Cfg::STAGE};
    // chunk c's window in R[c % PD], loaded PD chunks ahead: three for the 192-channel unit (one
    // workgroup per CU, so no second workgroup's work covers the loads' latency), two for the
    // 96-channel one (two workgroups per CU; the registers of a third set slowed it)
    constexpr int PD = C == 192 ? 3 : 2;
    WinRegs R[PD];
    // W2 [C][C] in 16-byte segments (8 input channels of one output channel), loaded during the
    // last chunk and stored in the A-fragment order conv2 reads (see below)
    half8_t w2r[Cfg::W2_PER_T];
    auto w2_load = [&] {
#pragma unroll
        for (int i = 0; i < Cfg::W2_PER_T; ++i) {
            const int sg = tid + i * Cfg::THREADS;
            if (Cfg::W2_SEGS % Cfg::THREADS == 0 || sg < Cfg::W2_SEGS)
                w2r[i] = *reinterpret_cast<const half8_t *>(q.w2 + sg * 8);
        }
    };
    w_issue(0, stage[0]);
    win_load(R[0], 0);
    if (Cfg::CHUNKS > 1) win_load(R[1], KC);
    if (PD == 3 && Cfg::CHUNKS > 2) win_load(R[PD - 1], 2 * KC);
    wait_vmem_le<(Cfg::CHUNKS > PD - 1 ? PD - 1 : Cfg::CHUNKS - 1) * Cfg::A_PER_T>();  // W1 and chunk 0's window
    win_store(R[0], 0, stage[0]);
    __syncthreads();
#pragma unroll
    for (int c = 0; c < Cfg::CHUNKS; ++c) {
        const int cur = c & 1, nxt = cur ^ 1;
        if (c + 1 < Cfg::CHUNKS) w_issue((c + 1) * KC, stage[nxt]);
        if (c + PD < Cfg::CHUNKS) win_load(R[c % PD], (c + PD) * KC);
        if (c + 1 == Cfg::CHUNKS) w2_load();
        if (c + 1 < Cfg::CHUNKS) {
            // the window of chunk c+1 (loaded PD-1 chunks ago; the compiler waits for those
            // registers) is snaked in the shadow of chunk c's MFMAs
            const SnakeK kk = snake_consts((c + 1) * KC);
            constexpr int NE = 8 * Cfg::A_PER_T;
            WinRegs &Rn = R[(c + 1) % PD];
            compute(stage[cur], [&](int t) {
                if constexpr (KT > 0) {
                    snake_elems(Rn, kk, t * NE / KT, (t + 1) * NE / KT);
                } else {
                    if (t < 0) snake_elems(Rn, kk, 0, NE);
                }
            });
        } else {
            compute(stage[cur], [](int) {});
        }
        // W1 of chunk c+1 has landed (only the newest window loads, chunk c+PD's, may be in flight)
        if (c + PD < Cfg::CHUNKS)
            wait_vmem_le<Cfg::A_PER_T>();
        else if (c + 1 < Cfg::CHUNKS)
            wait_vmem();
        if (c + 1 < Cfg::CHUNKS) win_write(R[(c + 1) % PD], stage[nxt]);
        stage_barrier();
    }

    // the residual rows of this lane's positions, four channels per load (consumed at the end)
    half4_v ures[TM][TN][4];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int pos = l0 + prow + 32 * i;
        const half_t *urow = ul + static_cast<int64_t>(pos < q.L ? pos : 0) * C + 4 * hf;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) ures[i][j][g] = *reinterpret_cast<const half4_v *>(urow + 32 * j + 8 * g);
    }
    // W2 into LDS, permuted within each 16-channel group so that one 16-byte read is an A
    // fragment: row co holds, at 16kk + 8h + 4m + e, W2[co][16kk + 8m + 4h + e]
    half_t *W2s = reinterpret_cast<half_t *>(smem);
#pragma unroll
    for (int i = 0; i < Cfg::W2_PER_T; ++i) {
        const int sg = tid + i * Cfg::THREADS;
        if (Cfg::W2_SEGS % Cfg::THREADS == 0 || sg < Cfg::W2_SEGS) {
            const int co = sg / (C / 8), s8 = sg % (C / 8);  // channels 8*s8 .. +8: kk = s8/2, m = s8&1
            half_t *dst = W2s + co * Cfg::W2_PITCH + 16 * (s8 >> 1) + 4 * (s8 & 1);
            const half8_t v = w2r[i];
            *reinterpret_cast<half4_v *>(dst) = half4_v{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<half4_v *>(dst + 8) = half4_v{v[4], v[5], v[6], v[7]};
        }
    }

    // h2 = f16(SnakeBeta2(f16(acc))), packed as conv2's B fragments: fragment kk of position block
    // i holds channels 16kk + {0..3, 8..11} + 4hf, in that order (accumulator block j gives
    // fragments 2j and 2j+1)
    half8_t h2[TM][C / 16];
    auto make_h2 = [&](int j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int ch = 32 * j + 8 * g + 4 * hf;
            const float4_t ka = *reinterpret_cast<const float4_t *>(tab + 3 * C + ch);
            const float4_t rr = *reinterpret_cast<const float4_t *>(tab + 4 * C + ch);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    h2[i][2 * j + (g >> 1)][(g & 1) * 4 + e] = snake_h(static_cast<half_t>(acc[i][j][4 * g + e]), ka[e], rr[e]);
        }
    };
    auto b2_init = [&](int j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4_t b = *reinterpret_cast<const float4_t *>(tab + 5 * C + 32 * j + 8 * g + 4 * hf);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[i][j][4 * g + e] = b[e];
        }
    };
    const half_t *w2l = W2s + l32 * Cfg::W2_PITCH + 8 * hf;
    auto conv2_step = [&](int j, int kk) {
        const half8_t a = *reinterpret_cast<const half8_t *>(w2l + 32 * j * Cfg::W2_PITCH + 16 * kk);
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, h2[i][kk], acc[i][j], 0, 0, 0);
    };
    // conv2: acc = b2 + W2 . h2, each output block's k-steps summed in order
    if constexpr (TN >= 6) {
        // block s's accumulators restart at b2 once its fragments exist and take k-steps
        // 0 .. 2s+1, the blocks before it k-steps 2s and 2s+1: block s+1's SnakeBeta runs in the
        // shadow of step s's MFMAs
        make_h2(0);
        __syncthreads();  // W2 in LDS
#pragma unroll
        for (int s2 = 0; s2 < TN; ++s2) {
            b2_init(s2);
#pragma unroll
            for (int kk = 0; kk < 2 * s2 + 2; ++kk) {
                conv2_step(s2, kk);
                if (kk >= 2 * s2)
#pragma unroll
                    for (int j = 0; j < s2; ++j) conv2_step(j, kk);
            }
            if (s2 + 1 < TN) make_h2(s2 + 1);
        }
    } else {
#pragma unroll
        for (int j = 0; j < TN; ++j) make_h2(j);
#pragma unroll
        for (int j = 0; j < TN; ++j) b2_init(j);
        __syncthreads();  // W2 in LDS
#pragma unroll
        for (int kk = 0; kk < C / 16; ++kk)
#pragma unroll
            for (int j = 0; j < TN; ++j) conv2_step(j, kk);
    }

    // y = f16(acc + u), y_pre, SnakeBeta_out. The values are made in the transposed layout (a
    // lane: one position, runs of four channels) and go out through the wave's own LDS block, so
    // every store moves 16 coalesced bytes of a row (a store of the 8-byte runs would touch 32
    // rows per instruction). The stages are free once every wave's conv2 has read W2.
    __syncthreads();
    half_t *O = reinterpret_cast<half_t *>(smem) + wave * 32 * Cfg::OPITCH;
    constexpr int RSEG = C / 8;                 // 16-byte segments per row
    constexpr int NSEG = 32 * RSEG / 64;        // per lane per 32-row block
    static_assert((32 * RSEG) % 64 == 0, "row segments split evenly over the lanes");
    auto flush = [&](int i, half_t *dst) {      // the block's rows from O to dst, 16 bytes a lane
        wave_lds_order();
        // four segments in flight at a time: the values of the block are still live here
#pragma unroll 1
        for (int u0 = 0; u0 < NSEG; u0 += 4) {
#pragma unroll
            for (int u = u0; u < u0 + 4 && u < NSEG; ++u) {
                const int sgi = lane + 64 * u;
                const int r = sgi / RSEG, c8 = sgi - (sgi / RSEG) * RSEG;
                const int pos = l0 + wave * Cfg::WP + 32 * i + r;
                const half8_t v = *reinterpret_cast<const half8_t *>(O + r * Cfg::OPITCH + c8 * 8);
                if (pos < q.L)
                    *reinterpret_cast<half8_t *>(dst + (static_cast<int64_t>(lane_idx) * q.L + pos) * C + c8 * 8) = v;
            }
        }
        wave_lds_order();  // the reads precede the next block's writes
    };
    // y_pre = f16(acc + u) of run (i, j, g), and y = SnakeBeta_out(y_pre) (or y_pre)
    auto y_run = [&](int i, int j, int g, bool snake) {
        const half4_v uu = ures[i][j][g];
        half4_v yv;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            yv[e] = static_cast<half_t>(__builtin_fmaf(static_cast<float>(uu[e]), 1.0f, acc[i][j][4 * g + e]));
        if (snake) {
            const int ch = 32 * j + 8 * g + 4 * hf;
            const float4_t ka = *reinterpret_cast<const float4_t *>(tab + 6 * C + ch);
            const float4_t rr = *reinterpret_cast<const float4_t *>(tab + 7 * C + ch);
#pragma unroll
            for (int e = 0; e < 4; ++e) yv[e] = snake_h(yv[e], ka[e], rr[e]);
        }
        *reinterpret_cast<half4_v *>(O + l32 * Cfg::OPITCH + 32 * j + 8 * g + 4 * hf) = yv;
    };
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        if (q.y_pre) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) y_run(i, j, g, false);
            flush(i, q.y_pre);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) y_run(i, j, g, q.a_out != nullptr);
        flush(i, q.y);
    }
}

template <typename Cfg>
hipError_t launch_ru(RuArgs q, int64_t lanes, hipStream_t stream) {
    q.tiles_m = (q.L + Cfg::BM - 1) / Cfg::BM;
    const int64_t total = lanes * q.tiles_m;
    q.total_tiles = static_cast<int>(total);
    q.tiles_per_xcd = static_cast<int>((total + 7) / 8);
    const unsigned grid = static_cast<unsigned>(int64_t(q.tiles_per_xcd) * 8);
    if (q.k == Cfg::KMAX)
        ru_nlc_f16<Cfg, Cfg::KMAX><<<grid, Cfg::THREADS, 0, stream>>>(q);
    else
        ru_nlc_f16<Cfg, 0><<<grid, Cfg::THREADS, 0, stream>>>(q);
    return hipGetLastError();
}

bool ru_shape_ok(const dtts_ru_desc *d) {
    const int64_t halo = (d->k - 1) * d->dilation;
    return (d->channels == 96 || d->channels == 192) && d->k >= 1 && d->k <= 7 && d->dilation >= 1 && halo <= 64 &&
           direct_offsets_fit(d->len, d->channels, d->channels, d->k);
}

template <typename Cfg>
const char *ru_name(char *buf, size_t n, int k) {
    snprintf(buf, n, "ru_nlc_f16<dtts::(anonymous namespace)::RuCfg<%d, %d, %d, %d, %d>, %d>", Cfg::C, Cfg::WP, Cfg::NW,
             Cfg::KC, Cfg::WPE_ARG, k == Cfg::KMAX ? Cfg::KMAX : 0);
    return buf;
}

}  // namespace

bool residual_unit_supported(const dtts_ru_desc *d) {
    return d && ru_shape_ok(d) && aligned(d->x, 16) && aligned(d->w1, 16) && aligned(d->w2, 8) && aligned(d->b1, 2) &&
           aligned(d->b2, 2) && aligned(d->y, 8) && (!d->y_pre || aligned(d->y_pre, 8));
}

const char *residual_unit_kernel_name(const dtts_ru_desc *d) {
    static thread_local char buf[128];
    const int k = static_cast<int>(d->k);
    return d->channels == 96 ? ru_name<RuTile96>(buf, sizeof(buf), k) : ru_name<RuTile192>(buf, sizeof(buf), k);
}

int residual_unit_nlc_f16(const dtts_ru_desc *d, hipStream_t stream) {
    const char *name = "dtts_residual_unit_nlc_f16";
    DTTS_REQUIRE(d, "%s: null descriptor", name);
    DTTS_REQUIRE(d->lanes >= 0 && d->len >= 0, "%s: negative shape", name);
    if (d->lanes == 0 || d->len == 0) return DTTS_OK;
    DTTS_REQUIRE(d->x && d->act1_alpha && d->act1_brecip && d->w1 && d->b1 && d->act2_alpha && d->act2_brecip &&
                     d->w2 && d->b2 && d->y,
                 "%s: every operand but y_pre and the output SnakeBeta is required", name);
    DTTS_REQUIRE((d->out_alpha == nullptr) == (d->out_brecip == nullptr), "%s: out_alpha and out_brecip go together",
                 name);
    if (!residual_unit_supported(d)) {
        set_error("%s: channels %lld, k %lld, dilation %lld (or alignment) not supported; compose two convs", name,
                  (long long)d->channels, (long long)d->k, (long long)d->dilation);
        return DTTS_ERR_UNSUPPORTED;
    }
    DTTS_REQUIRE(d->len < (int64_t(1) << 30) && d->lanes * d->len < (int64_t(1) << 36), "%s: shape too large", name);
    RuArgs q{};
    q.u = reinterpret_cast<const half_t *>(d->x);
    q.w1 = reinterpret_cast<const half_t *>(d->w1);
    q.w2 = reinterpret_cast<const half_t *>(d->w2);
    q.b1 = reinterpret_cast<const half_t *>(d->b1);
    q.b2 = reinterpret_cast<const half_t *>(d->b2);
    q.a1 = d->act1_alpha;
    q.r1 = d->act1_brecip;
    q.a2 = d->act2_alpha;
    q.r2 = d->act2_brecip;
    q.a_out = d->out_alpha;
    q.r_out = d->out_brecip;
    q.y_pre = reinterpret_cast<half_t *>(d->y_pre);
    q.y = reinterpret_cast<half_t *>(d->y);
    q.L = static_cast<int>(d->len);
    q.k = static_cast<int>(d->k);
    q.dil = static_cast<int>(d->dilation);
    q.pad_left = static_cast<int>((d->k - 1) * d->dilation);
    const hipError_t e = d->channels == 96 ? launch_ru<RuTile96>(q, d->lanes, stream) : launch_ru<RuTile192>(q, d->lanes, stream);
    DTTS_HIP_CHECK(e, name);
    return DTTS_OK;
}

}  // namespace dtts

extern "C" int dtts_residual_unit_nlc_f16(const dtts_ru_desc *desc, hipStream_t stream) {
    return dtts::residual_unit_nlc_f16(desc, stream);
}

extern "C" int dtts_residual_unit_supported(const dtts_ru_desc *desc) {
    return dtts::residual_unit_supported(desc) ? 1 : 0;
}
