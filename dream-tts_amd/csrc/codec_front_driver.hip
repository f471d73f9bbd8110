// The codec's front half as one call: codes -> the latent the waveform stack takes.
//
// Reference: Codec::forward up to `head_conv` (crates/qwen3tts/src/codec.rs:401-424): the split
// RVQ (Rvq::decode twice, summed), pre_conv (causal, k = 3), pre_transformer.input_proj, the
// 8-layer sliding-window transformer (Stack::forward's prefill branch over the chunk, qwen3.rs:
// 294-467, with LayerScale and no QK-norm), output_proj, then per upsampling ratio a TransConv
// (kernel = stride) and a ConvNext block (codec.rs:160-196). All lanes at once; the projections
// and convs run on the channels-last conv kernel (k = 1 for a projection); the RVQ lookup,
// norms, SwiGLU, windowed attention and depthwise+LayerNorm have kernels of their own
// (codec_front.hip). Activations are f16 in HBM, f32 inside every kernel.
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "conv.hpp"

struct dtts_codec_front {
    dtts_codec_front_geometry geo;
    dtts_codec_front_weights w;
    float *cos_t = nullptr, *sin_t = nullptr;  // [max_frames, tf_head_dim / 2]
    // Pinned staging for the host's codes: the host fills it, an async copy on the caller's stream
    // reads it, and `staged` marks that copy's end, so the next call waits for it before refilling
    // (calls on one front half from several host threads at once race on it).
    mutable int32_t *pinned = nullptr;
    mutable size_t pinned_n = 0;
    mutable hipEvent_t staged = nullptr;
};

namespace dtts {
namespace {

inline size_t round256(size_t v) { return (v + 255) & ~size_t(255); }

dtts_conv_desc pointwise(int64_t lanes, int64_t len, int64_t cin, int64_t cout, const void *x, const void *w,
                         const void *b, void *y) {
    dtts_conv_desc d{};
    d.lanes = lanes;
    d.len = len;
    d.cin = cin;
    d.cout = cout;
    d.k = 1;
    d.dilation = 1;
    d.pad_left = 0;
    d.x = x;
    d.w = w;
    d.bias = b;
    d.y = y;
    return d;
}

struct FrontPlan {
    size_t codes, s, q, lat_a, lat_b, h, a, qkv, att, gu, t, dn, p, total;
};

FrontPlan front_plan(const dtts_codec_front_geometry &g, int64_t lanes, int64_t frames) {
    FrontPlan pl{};
    const int64_t rows = lanes * frames;
    int64_t up = 1;
    for (int64_t i = 0; i < g.n_up; ++i) up *= g.up_ratios[i];
    const int64_t rows_out = rows * up;
    const int64_t qkvw = (g.tf_heads + 2 * g.tf_n_kv) * g.tf_head_dim, qw = g.tf_heads * g.tf_head_dim;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += round256(bytes);
        return at;
    };
    pl.codes = take(sizeof(int32_t) * rows * g.n_books);
    pl.s = take(2 * rows * 2 * g.book_dim);
    pl.q = take(2 * rows * g.codebook_dim);
    // latent-width tensors at every length up to the output's; the last stage writes the caller's
    int64_t lat_rows = rows;
    for (int64_t i = 0; i + 1 < g.n_up; ++i) lat_rows *= g.up_ratios[i];
    const int64_t lat = (g.n_up > 0 ? lat_rows * g.up_ratios[g.n_up - 1] : rows) * g.latent_dim;
    pl.lat_a = take(2 * lat);
    pl.lat_b = take(2 * lat);
    pl.h = take(2 * rows * g.tf_dim);
    pl.a = take(2 * rows * g.tf_dim);
    pl.qkv = take(2 * rows * qkvw);
    pl.att = take(2 * rows * qw);
    pl.gu = take(2 * rows * 2 * g.tf_ffn);
    pl.t = take(2 * rows * g.tf_ffn);
    pl.dn = take(2 * rows_out * g.latent_dim);
    pl.p = take(2 * rows_out * 4 * g.latent_dim);
    pl.total = off;
    return pl;
}

#define FRONT_STEP(expr)                 \
    do {                                 \
        const int rc_ = (expr);          \
        if (rc_ != DTTS_OK) return rc_;  \
    } while (0)

}  // namespace
}  // namespace dtts

extern "C" int dtts_codec_front_create(const dtts_codec_front_geometry *geo, const dtts_codec_front_weights *w,
                                       dtts_codec_front **out) {
    const char *name = "dtts_codec_front_create";
    DTTS_REQUIRE(geo && w && out, "%s: null argument", name);
    *out = nullptr;
    const dtts_codec_front_geometry &g = *geo;
    DTTS_REQUIRE(g.n_books > 1 && g.n_first > 0 && g.n_first < g.n_books && g.book_size > 0 && g.book_dim > 0 &&
                     g.book_dim % 4 == 0 && g.codebook_dim > 0,
                 "%s: bad quantizer geometry", name);
    DTTS_REQUIRE(g.latent_dim > 0 && g.pre_kernel > 0 && g.tf_dim > 0 && g.tf_layers > 0 &&
                     g.tf_layers <= DTTS_FRONT_MAX_LAYERS && g.tf_heads > 0 && g.tf_n_kv > 0 &&
                     g.tf_heads % g.tf_n_kv == 0 && g.tf_head_dim == 64 && g.tf_ffn > 0 && g.tf_window >= 1 &&
                     g.tf_window <= 192 && g.max_frames > 0 && g.max_frames < (int64_t(1) << 24),
                 "%s: bad transformer geometry (head_dim 64, window 1..192, up to %d layers)", name,
                 DTTS_FRONT_MAX_LAYERS);
    DTTS_REQUIRE(g.tf_dim % 8 == 0 && g.tf_ffn % 8 == 0 && g.latent_dim % 8 == 0 && g.latent_dim <= 2048,
                 "%s: widths must be multiples of 8 (latent up to 2048)", name);
    DTTS_REQUIRE(g.n_up >= 0 && g.n_up <= DTTS_FRONT_MAX_UP && g.dw_kernel > 0 && g.dw_kernel <= 64, "%s: bad upsampling",
                 name);
    for (int64_t i = 0; i < g.n_up; ++i) DTTS_REQUIRE(g.up_ratios[i] > 0, "%s: up_ratios[%lld]", name, (long long)i);
    DTTS_REQUIRE(w->codebooks && w->out_proj && w->pre_w && w->in_w && w->tf_norm && w->out_w,
                 "%s: missing weights", name);
    for (int64_t i = 0; i < g.tf_layers; ++i) {
        const dtts_codec_front_layer &L = w->layers[i];
        DTTS_REQUIRE(L.attn_norm && L.attn_scale && L.ffn_norm && L.mlp_scale && L.wqkv && L.wo && L.w_gateup &&
                         L.wdown,
                     "%s: layer %lld incomplete", name, (long long)i);
    }
    for (int64_t i = 0; i < g.n_up; ++i) {
        const dtts_codec_front_up &U = w->up[i];
        DTTS_REQUIRE(U.up_w && U.dw_taps && U.dw_bias && U.ln_weight && U.ln_bias && U.pw1_w && U.pw2_w && U.gamma,
                     "%s: upsampling stage %lld incomplete", name, (long long)i);
    }
    dtts_codec_front *f = new (std::nothrow) dtts_codec_front();
    DTTS_REQUIRE(f, "%s: out of host memory", name);
    f->geo = g;
    f->w = *w;
    const int64_t half = g.tf_head_dim / 2;
    std::vector<float> c(static_cast<size_t>(g.max_frames * half)), s(c.size());
    int rc = dtts_rope_table_f32(g.max_frames, g.tf_head_dim, g.tf_rope_base, c.data(), s.data());
    hipError_t e = hipSuccess;
    if (rc == DTTS_OK) {
        e = hipMalloc(&f->cos_t, sizeof(float) * c.size());
        if (e == hipSuccess) e = hipMalloc(&f->sin_t, sizeof(float) * c.size());
        if (e == hipSuccess) e = hipMemcpy(f->cos_t, c.data(), sizeof(float) * c.size(), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(f->sin_t, s.data(), sizeof(float) * c.size(), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&f->staged, hipEventDisableTiming);
    }
    if (rc != DTTS_OK || e != hipSuccess) {
        dtts_codec_front_destroy(f);
        if (e != hipSuccess) dtts::set_error("%s: %s", name, hipGetErrorString(e));
        return rc != DTTS_OK ? rc : DTTS_ERR_HIP;
    }
    *out = f;
    return DTTS_OK;
}

extern "C" void dtts_codec_front_destroy(dtts_codec_front *f) {
    if (!f) return;
    if (f->cos_t) (void)hipFree(f->cos_t);
    if (f->sin_t) (void)hipFree(f->sin_t);
    if (f->staged) {
        (void)hipEventSynchronize(f->staged);
        (void)hipEventDestroy(f->staged);
    }
    if (f->pinned) (void)hipHostFree(f->pinned);
    delete f;
}

extern "C" size_t dtts_codec_front_workspace_bytes(const dtts_codec_front *f, int64_t lanes, int64_t frames) {
    if (!f || lanes <= 0 || frames <= 0) return 0;
    return dtts::front_plan(f->geo, lanes, frames).total;
}

namespace dtts {
namespace {

// The pinned staging buffer, holding at least n codes, once the previous call's copy out of it
// has ended; nullptr (error set) on failure.
int32_t *stage_codes(const dtts_codec_front *f, size_t n, const char *name) {
    hipError_t e = hipEventSynchronize(f->staged);
    if (e == hipSuccess && f->pinned_n < n) {
        if (f->pinned) e = hipHostFree(f->pinned);
        f->pinned = nullptr;
        f->pinned_n = 0;
        if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void **>(&f->pinned), sizeof(int32_t) * n, 0);
        if (e == hipSuccess) f->pinned_n = n;
    }
    if (e != hipSuccess) {
        set_error("%s: staging codes: %s", name, hipGetErrorString(e));
        return nullptr;
    }
    return f->pinned;
}

// The front half over codes already in the pinned staging buffer ([lanes, frames, n_books]).
int front_decode_staged(const dtts_codec_front *f, dtts_f16 *latent, int64_t lanes, int64_t frames,
                        void *workspace, size_t ws_bytes, hipStream_t stream, const char *name) {
    const dtts_codec_front_geometry &g = f->geo;
    const dtts_codec_front_weights &W = f->w;
    const FrontPlan pl = front_plan(g, lanes, frames);
    DTTS_REQUIRE(ws_bytes >= pl.total, "%s: workspace %zu bytes < %zu needed", name, ws_bytes, pl.total);
    DTTS_REQUIRE(aligned(workspace, 256) && aligned(latent, 16), "%s: misaligned workspace or latent", name);
    const int64_t rows = lanes * frames;
    const int32_t *codes = f->pinned;
    // Rvq::decode's index_select refuses codes outside the book (codec.rs:303-305)
    for (int64_t i = 0; i < rows * g.n_books; ++i)
        DTTS_REQUIRE(codes[i] >= 0 && codes[i] < g.book_size, "%s: code %d at %lld outside [0, %lld)", name, codes[i],
                     (long long)i, (long long)g.book_size);
    char *ws = static_cast<char *>(workspace);
    auto at = [&](size_t off) { return static_cast<void *>(ws + off); };
    DTTS_HIP_CHECK(hipMemcpyAsync(at(pl.codes), codes, sizeof(int32_t) * rows * g.n_books, hipMemcpyHostToDevice, stream),
                   name);
    DTTS_HIP_CHECK(hipEventRecord(f->staged, stream), name);
    // split RVQ: both stacks' lookups side by side, then one projection over the joined width
    FRONT_STEP(dtts_rvq_lookup_sum_f16(static_cast<const int32_t *>(at(pl.codes)), W.codebooks, g.n_books, g.n_first,
                                       g.book_size, g.book_dim, static_cast<dtts_f16 *>(at(pl.s)), rows, stream));
    dtts_conv_desc d = pointwise(lanes, frames, 2 * g.book_dim, g.codebook_dim, at(pl.s), W.out_proj, nullptr, at(pl.q));
    FRONT_STEP(dtts::conv1d_nlc_f16(&d, stream));
    // pre_conv (causal) and the transformer's input projection
    d = pointwise(lanes, frames, g.codebook_dim, g.latent_dim, at(pl.q), W.pre_w, W.pre_b, at(pl.lat_a));
    d.k = g.pre_kernel;
    d.pad_left = g.pre_kernel - 1;
    FRONT_STEP(dtts::conv1d_nlc_f16(&d, stream));
    d = pointwise(lanes, frames, g.latent_dim, g.tf_dim, at(pl.lat_a), W.in_w, W.in_b, at(pl.h));
    FRONT_STEP(dtts::conv1d_nlc_f16(&d, stream));
    // the sliding-window transformer over the chunk
    const int64_t qkvw = (g.tf_heads + 2 * g.tf_n_kv) * g.tf_head_dim, qw = g.tf_heads * g.tf_head_dim;
    const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(g.tf_head_dim)));
    dtts_f16 *h = static_cast<dtts_f16 *>(at(pl.h)), *a = static_cast<dtts_f16 *>(at(pl.a));
    for (int64_t li = 0; li < g.tf_layers; ++li) {
        const dtts_codec_front_layer &L = W.layers[li];
        FRONT_STEP(dtts_rms_norm_rows_f16(h, L.attn_norm, a, rows, g.tf_dim, g.tf_eps, stream));
        d = pointwise(lanes, frames, g.tf_dim, qkvw, a, L.wqkv, nullptr, at(pl.qkv));
        FRONT_STEP(dtts::conv1d_nlc_f16(&d, stream));
        FRONT_STEP(dtts_window_attention_prefill_f16(static_cast<const dtts_f16 *>(at(pl.qkv)), f->cos_t, f->sin_t,
                                                     g.max_frames, static_cast<dtts_f16 *>(at(pl.att)), lanes, frames,
                                                     g.tf_heads, g.tf_n_kv, g.tf_head_dim, g.tf_window, scale, stream));
        d = pointwise(lanes, frames, qw, g.tf_dim, at(pl.att), L.wo, nullptr, h);
        d.residual = h;  // h + attn * attn_scale, in place (each element read, then written, by one thread)
        d.out_scale = L.attn_scale;
        FRONT_STEP(dtts::conv1d_nlc_f16(&d, stream));
        FRONT_STEP(dtts_rms_norm_rows_f16(h, L.ffn_norm, a, rows, g.tf_dim, g.tf_eps, stream));
        d = pointwise(lanes, frames, g.tf_dim, 2 * g.tf_ffn, a, L.w_gateup, nullptr, at(pl.gu));
        FRONT_STEP(dtts::conv1d_nlc_f16(&d, stream));
        FRONT_STEP(dtts_swiglu_rows_f16(static_cast<const dtts_f16 *>(at(pl.gu)), static_cast<dtts_f16 *>(at(pl.t)), rows,
                                        g.tf_ffn, stream));
        d = pointwise(lanes, frames, g.tf_ffn, g.tf_dim, at(pl.t), L.wdown, nullptr, h);
        d.residual = h;
        d.out_scale = L.mlp_scale;
        FRONT_STEP(dtts::conv1d_nlc_f16(&d, stream));
    }
    FRONT_STEP(dtts_rms_norm_rows_f16(h, W.tf_norm, a, rows, g.tf_dim, g.tf_eps, stream));
    void *x = g.n_up > 0 ? at(pl.lat_a) : static_cast<void *>(latent);
    d = pointwise(lanes, frames, g.tf_dim, g.latent_dim, a, W.out_w, W.out_b, x);
    FRONT_STEP(dtts::conv1d_nlc_f16(&d, stream));
    // upsampling: TransConv (one tap over r phases) then ConvNeXt, the last one into `latent`
    int64_t len = frames;
    for (int64_t i = 0; i < g.n_up; ++i) {
        const dtts_codec_front_up &U = W.up[i];
        const int64_t r = g.up_ratios[i];
        void *u = x == at(pl.lat_a) ? at(pl.lat_b) : at(pl.lat_a);
        d = pointwise(lanes, len, g.latent_dim, r * g.latent_dim, x, U.up_w, U.up_b, u);
        FRONT_STEP(dtts::conv1d_nlc_f16(&d, stream));
        len *= r;  // [lanes, len, r C] is [lanes, r len, C]
        FRONT_STEP(dtts_depthwise_layernorm_nlc_f16(static_cast<const dtts_f16 *>(u), U.dw_taps, U.dw_bias, U.ln_weight,
                                                    U.ln_bias, g.ln_eps, static_cast<dtts_f16 *>(at(pl.dn)), lanes, len,
                                                    g.latent_dim, g.dw_kernel, stream));
        d = pointwise(lanes, len, g.latent_dim, 4 * g.latent_dim, at(pl.dn), U.pw1_w, U.pw1_b, at(pl.p));
        d.act = 2;
        FRONT_STEP(dtts::conv1d_nlc_f16(&d, stream));
        void *y = i + 1 == g.n_up ? static_cast<void *>(latent) : x;
        d = pointwise(lanes, len, 4 * g.latent_dim, g.latent_dim, at(pl.p), U.pw2_w, U.pw2_b, y);
        d.residual = u;
        d.out_scale = U.gamma;
        FRONT_STEP(dtts::conv1d_nlc_f16(&d, stream));
        x = y;
    }
    return DTTS_OK;
}

}  // namespace
}  // namespace dtts

extern "C" int dtts_codec_front_decode(const dtts_codec_front *f, const int32_t *codes, dtts_f16 *latent,
                                       int64_t lanes, int64_t frames, void *workspace, size_t ws_bytes,
                                       hipStream_t stream) {
    const char *name = "dtts_codec_front_decode";
    DTTS_REQUIRE(f, "%s: null front half", name);
    DTTS_REQUIRE(lanes >= 0 && frames >= 0, "%s: bad shape", name);
    if (lanes == 0 || frames == 0) return DTTS_OK;
    DTTS_REQUIRE(codes && latent && workspace, "%s: null pointer", name);
    DTTS_REQUIRE(frames <= f->geo.max_frames, "%s: %lld frames exceed max_frames %lld", name, (long long)frames,
                 (long long)f->geo.max_frames);
    DTTS_REQUIRE(lanes * frames < (int64_t(1) << 30), "%s: too many frames", name);
    const size_t n = static_cast<size_t>(lanes * frames * f->geo.n_books);
    int32_t *pin = dtts::stage_codes(f, n, name);
    if (!pin) return DTTS_ERR_HIP;
    std::memcpy(pin, codes, sizeof(int32_t) * n);
    return dtts::front_decode_staged(f, latent, lanes, frames, workspace, ws_bytes, stream, name);
}

// ------------------------------------------------------------------ Codec::decode, chunked

namespace dtts {
namespace {

struct DocPlan {
    int64_t lanes, frames, spf;  // windows run as lanes, each `frames` long; samples per frame
    bool f32;                    // an f32 waveform stack: its latent widened from the front half's f16
    size_t front, latent, latent32, codec, audio, total;
};

bool doc_plan(const dtts_codec_front *f, const dtts_codec *c, int64_t n, int64_t chunk, int64_t context, DocPlan &p) {
    if (!f || !c || n <= 0 || chunk <= 0 || context < 0) return false;
    // Every window is one lane of one length: the span when n >= span (the reference pads to it);
    // otherwise n, the first window's length, with the later, shorter windows padded on the right
    // by their last frame too -- the decoder is causal, so frames after the kept ones change nothing.
    const int64_t span = chunk + context;
    p.lanes = (n + chunk - 1) / chunk;
    p.frames = n >= span ? span : n;
    int64_t up = 1;
    for (int64_t i = 0; i < f->geo.n_up; ++i) up *= f->geo.up_ratios[i];
    p.spf = up * dtts_codec_hop(c);
    p.f32 = codec_is_f32(c);
    const size_t es = p.f32 ? 4 : 2;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += round256(bytes);
        return at;
    };
    p.front = take(dtts_codec_front_workspace_bytes(f, p.lanes, p.frames));
    p.latent = take(2 * static_cast<size_t>(p.lanes * p.frames * up * f->geo.latent_dim));
    p.latent32 = take(p.f32 ? 4 * static_cast<size_t>(p.lanes * p.frames * up * f->geo.latent_dim) : 0);
    p.codec = take(dtts_codec_workspace_bytes(c, p.lanes, p.frames * up));
    p.audio = take(es * static_cast<size_t>(p.lanes * p.frames * p.spf));
    p.total = off;
    return true;
}

// out[o] = window w's sample at o - w's chunk start + its context's length, w = (o / spf) / chunk
template <typename T>
__global__ __launch_bounds__(256) void doc_gather_kernel(const T *audio, float *out, int64_t total, int64_t spf,
                                                         int64_t chunk, int64_t context, int64_t win_len) {
    for (int64_t o = blockIdx.x * int64_t(256) + threadIdx.x; o < total; o += int64_t(gridDim.x) * 256) {
        const int64_t w = (o / spf) / chunk;
        const int64_t start = w * chunk;
        const int64_t from = start > context ? start - context : 0;
        out[o] = static_cast<float>(audio[w * win_len + (start - from) * spf + (o - start * spf)]);
    }
}

__global__ __launch_bounds__(256) void widen_f16_kernel(const half_t *x, float *y, int64_t n) {
    for (int64_t i = blockIdx.x * int64_t(256) + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256)
        y[i] = static_cast<float>(x[i]);
}

}  // namespace
}  // namespace dtts

extern "C" size_t dtts_codec_document_workspace_bytes(const dtts_codec_front *f, const dtts_codec *c, int64_t n,
                                                      int64_t chunk, int64_t context) {
    dtts::DocPlan p{};
    return dtts::doc_plan(f, c, n, chunk, context, p) ? p.total : 0;
}

extern "C" int dtts_codec_decode_document(const dtts_codec_front *f, const dtts_codec *c, const int32_t *codes,
                                          int64_t n, int64_t chunk, int64_t context, float *audio, void *workspace,
                                          size_t ws_bytes, hipStream_t stream) {
    const char *name = "dtts_codec_decode_document";
    DTTS_REQUIRE(f && c, "%s: null front half or codec", name);
    DTTS_REQUIRE(n >= 0 && chunk > 0 && context >= 0, "%s: bad sizes (n %lld, chunk %lld, context %lld)", name,
                 (long long)n, (long long)chunk, (long long)context);
    if (n == 0) return DTTS_OK;
    DTTS_REQUIRE(codes && audio && workspace, "%s: null pointer", name);
    dtts::DocPlan p{};
    DTTS_REQUIRE(dtts::doc_plan(f, c, n, chunk, context, p), "%s: bad plan", name);
    DTTS_REQUIRE(ws_bytes >= p.total, "%s: workspace %zu bytes < %zu needed", name, ws_bytes, p.total);
    DTTS_REQUIRE(dtts::aligned(workspace, 256), "%s: misaligned workspace", name);
    const int64_t nb = f->geo.n_books;
    DTTS_REQUIRE(p.frames <= f->geo.max_frames, "%s: %lld-frame windows exceed max_frames %lld", name,
                 (long long)p.frames, (long long)f->geo.max_frames);
    DTTS_REQUIRE(p.lanes * p.frames < (int64_t(1) << 30), "%s: too many frames", name);
    // the windows' codes, each right-padded with its last frame (codec.rs:585-593)
    int32_t *win = dtts::stage_codes(f, static_cast<size_t>(p.lanes * p.frames * nb), name);
    if (!win) return DTTS_ERR_HIP;
    for (int64_t w = 0; w < p.lanes; ++w) {
        const int64_t start = w * chunk;
        const int64_t from = start > context ? start - context : 0;
        const int64_t to = from + p.frames < n ? from + p.frames : n;
        for (int64_t t = 0; t < p.frames; ++t) {
            const int64_t src = from + t < to ? from + t : to - 1;
            for (int64_t b = 0; b < nb; ++b) win[(w * p.frames + t) * nb + b] = codes[src * nb + b];
        }
    }
    char *ws = static_cast<char *>(workspace);
    dtts_f16 *latent = reinterpret_cast<dtts_f16 *>(ws + p.latent);
    FRONT_STEP(dtts::front_decode_staged(f, latent, p.lanes, p.frames, ws + p.front, p.latent - p.front, stream, name));
    int64_t up = 1;
    for (int64_t i = 0; i < f->geo.n_up; ++i) up *= f->geo.up_ratios[i];
    const int64_t total = n * p.spf;
    if (p.f32) {
        // the reference's own precision for the waveform stack: the latent widened exactly
        float *latent32 = reinterpret_cast<float *>(ws + p.latent32);
        float *wav = reinterpret_cast<float *>(ws + p.audio);
        const int64_t ne = p.lanes * p.frames * up * f->geo.latent_dim;
        dtts::widen_f16_kernel<<<dtts::grid_for(ne, 256), 256, 0, stream>>>(
            reinterpret_cast<const dtts::half_t *>(latent), latent32, ne);
        DTTS_LAUNCH_CHECK(name);
        FRONT_STEP(dtts_codec_decode_f32(c, latent32, wav, p.lanes, p.frames * up, ws + p.codec, p.audio - p.codec,
                                         stream));
        dtts::doc_gather_kernel<float><<<dtts::grid_for(total, 256), 256, 0, stream>>>(wav, audio, total, p.spf, chunk,
                                                                                      context, p.frames * p.spf);
    } else {
        dtts_f16 *wav = reinterpret_cast<dtts_f16 *>(ws + p.audio);
        FRONT_STEP(dtts_codec_decode(c, latent, wav, p.lanes, p.frames * up, ws + p.codec, p.audio - p.codec, stream));
        dtts::doc_gather_kernel<dtts::half_t><<<dtts::grid_for(total, 256), 256, 0, stream>>>(
            reinterpret_cast<const dtts::half_t *>(wav), audio, total, p.spf, chunk, context, p.frames * p.spf);
    }
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}
