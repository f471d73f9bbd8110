// The codec's residual unit as one kernel (ResidualUnit::forward, crates/qwen3tts/src/codec.rs:
// 215-229):
//
//   h  = f16(conv_k,dil(SnakeBeta1(u)) + b1)          conv1, the tile main loop
//   h2 = f16(SnakeBeta2(h))                           epilogue 1, into LDS
//   y  = f16(conv_1(h2) + b2 + u)                     conv2 on the matrix cores from LDS
//   out = y, and/or f16(SnakeBeta_next(y))            epilogue 2
//
// A workgroup owns BM positions x all C channels, so the k=1 conv's whole reduction (C) is in the
// workgroup after conv1: h and h2 never reach HBM. Per unit the activation traffic drops from
// five passes (read u; write h; read h; read u; write y) to two (read u with its halo, write y),
// and every value rounded to f16 here is one the unfused chain stores. W2 (C x C) is read as
// MFMA B fragments straight from L2.
#include "conv_tile.hpp"

namespace dtts {
namespace {

struct RuArgs {
    ConvArgs c1;        // conv1: x = u, w = w1, bias = b1, a_in/r_in = act1; cin = cout = C
    const half_t *u;    // the residual
    const float *a2, *r2;
    const half_t *w2, *b2;
    half_t *y_pre, *y;
    const float *a_out, *r_out;
};

template <typename Cfg, int KT>
__global__ __launch_bounds__(Cfg::THREADS, Cfg::MIN_WG) void ru_nlc_f16(RuArgs q) {
    constexpr int C = Cfg::BN;
    constexpr int HP = C + 8;  // h2 row pitch (halves)
    constexpr int H_BYTES = Cfg::BM * HP * 2;
    constexpr int LDS0 = Cfg::MAIN_BYTES > Cfg::EPI_TOTAL ? Cfg::MAIN_BYTES : Cfg::EPI_TOTAL;
    constexpr int LDS = LDS0 > H_BYTES ? LDS0 : H_BYTES;
    __shared__ __attribute__((aligned(16))) char smem[LDS];
    const ConvArgs &p = q.c1;
    int lane_idx, m_tile, n_tile;
    if (!conv_tile_coords(p, lane_idx, m_tile, n_tile)) return;
    const int l0 = m_tile * Cfg::BM;
    const half_t *xl = p.x + static_cast<int64_t>(lane_idx) * p.L * p.cin;
    float16_t acc[Cfg::TM][Cfg::TN];
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::TN; ++j) acc[i][j] = float16_t{};
    conv_mainloop<Cfg, true, KT>(p, xl, l0, 0, smem, acc);  // ends on a barrier

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
    half_t *H = reinterpret_cast<half_t *>(smem);
    // epilogue 1: h = f16(acc + b1), h2 = f16(SnakeBeta2(h)) -> H[row][channel]
#pragma unroll
    for (int j = 0; j < Cfg::TN; ++j) {
        const int n = wn * Cfg::WTN + j * 32 + (lane & 31);
        const float b1 = static_cast<float>(p.bias[n]);
        const float ka2 = q.a2[n] * kInv2Pi, r2 = q.r2[n];
#pragma unroll
        for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = wm * Cfg::WTM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                H[m * HP + n] = snake_f16k(static_cast<half_t>(acc[i][j][r] + b1), ka2, r2);
            }
    }
    __syncthreads();
    // conv2 (k = 1): acc = H[rows] . W2^T over K = C
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::TN; ++j) acc[i][j] = float16_t{};
    const int koff = (lane >> 5) * 8;
    const half_t *ha = H + (wm * Cfg::WTM + (lane & 31)) * HP + koff;
    const half_t *wb = q.w2 + static_cast<int64_t>(wn * Cfg::WTN + (lane & 31)) * C + koff;
#pragma unroll 2
    for (int kk = 0; kk < C; kk += 16) {
        half8_t af[Cfg::TM], bf[Cfg::TN];
#pragma unroll
        for (int j = 0; j < Cfg::TN; ++j) bf[j] = *reinterpret_cast<const half8_t *>(wb + j * 32 * C + kk);
#pragma unroll
        for (int i = 0; i < Cfg::TM; ++i) af[i] = *reinterpret_cast<const half8_t *>(ha + i * 32 * HP + kk);
#pragma unroll
        for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    // epilogue 2 (starts with a barrier, so H is no longer read when E overwrites it)
    conv_epilogue<Cfg>(acc, smem, static_cast<int64_t>(lane_idx) * p.L, l0, 0, p.L, C, q.b2, q.u, q.y_pre, q.y,
                       q.a_out, q.r_out, 0);
}

// C = 96 is bound by the SnakeBeta VALU work, which register staging overlaps across two
// workgroups per CU; C = 192 is matrix-bound and takes direct staging with eight waves.
typedef ConvTile<256, 96, 4, 1, 32, 7, 64> RuTile96;
typedef ConvTile<256, 192, 4, 2, 16, 7, 64, 2, kStageDirect> RuTile192;

template <typename Cfg>
hipError_t launch_ru(RuArgs q, int64_t lanes, hipStream_t stream) {
    ConvArgs &p = q.c1;
    p.tiles_m = (p.L + Cfg::BM - 1) / Cfg::BM;
    p.tiles_n = 1;
    const int64_t total = lanes * p.tiles_m;
    p.total_tiles = static_cast<int>(total);
    p.tiles_per_xcd = static_cast<int>((total + 7) / 8);
    const unsigned grid = static_cast<unsigned>(int64_t(p.tiles_per_xcd) * 8);
    if (p.k == Cfg::KMAX)
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

}  // namespace

bool residual_unit_supported(const dtts_ru_desc *d) {
    return d && ru_shape_ok(d) && aligned(d->x, 16) && aligned(d->w1, 16) && aligned(d->w2, 16) && aligned(d->b1, 2) &&
           aligned(d->b2, 16) && aligned(d->y, 16) && (!d->y_pre || aligned(d->y_pre, 16));
}

const char *residual_unit_kernel_name(const dtts_ru_desc *d) {
    static thread_local char buf[128];
    const char *tail = d->k == 7 ? ", 7>" : ", 0>";
    return d->channels == 96 ? tile_kernel_name<RuTile96>(buf, sizeof(buf), "ru_nlc_f16", tail)
                             : tile_kernel_name<RuTile192>(buf, sizeof(buf), "ru_nlc_f16", tail);
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
    ConvArgs &p = q.c1;
    p.x = reinterpret_cast<const half_t *>(d->x);
    p.w = reinterpret_cast<const half_t *>(d->w1);
    p.bias = reinterpret_cast<const half_t *>(d->b1);
    p.a_in = d->act1_alpha;
    p.r_in = d->act1_brecip;
    p.L = static_cast<int>(d->len);
    p.cin = p.cout = static_cast<int>(d->channels);
    p.k = static_cast<int>(d->k);
    p.dil = static_cast<int>(d->dilation);
    p.pad_left = static_cast<int>((d->k - 1) * d->dilation);
    q.u = reinterpret_cast<const half_t *>(d->x);
    q.a2 = d->act2_alpha;
    q.r2 = d->act2_brecip;
    q.w2 = reinterpret_cast<const half_t *>(d->w2);
    q.b2 = reinterpret_cast<const half_t *>(d->b2);
    q.y_pre = reinterpret_cast<half_t *>(d->y_pre);
    q.y = reinterpret_cast<half_t *>(d->y);
    q.a_out = d->out_alpha;
    q.r_out = d->out_brecip;
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
