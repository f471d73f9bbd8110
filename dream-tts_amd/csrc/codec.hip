// The qwen3tts codec's waveform stack (head conv, upsampling blocks, output conv) as a sequence
// of fused channels-last convs over all lanes at once.
//
// Reference: Codec::forward's tail, crates/qwen3tts/src/codec.rs:426-436, with DecoderBlock
// (codec.rs:252-258), ResidualUnit (codec.rs:215-229), TransConv (codec.rs:153-158) and SnakeBeta
// (codec.rs:55-73). Every SnakeBeta is folded into a conv:
//   head conv           epilogue: block 0's SnakeBeta, only the snaked tensor is stored
//   block i TransConv   prologue: nothing (its input arrives snaked); epilogue: stores u and,
//                       when u is wide, also SnakeBeta_{unit 0, act1}(u)
//   unit j conv1 (k7)   prologue: act1 when u was stored unsnaked; epilogue: act2, stored snaked
//   unit j conv2 (k1)   epilogue: + u (residual), then the next activation: unit j+1's act1
//                       (stored both ways when wide), or the next block's / the output SnakeBeta
//   output conv         tanh in the epilogue
// Every tensor stored is one the unfused chain would store (f16), so the arithmetic matches the
// composed form up to summation order.
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "conv.hpp"

struct dtts_codec {
    dtts_codec_geometry geo;
    dtts_codec_weights w;
    bool f32;  // made by dtts_codec_create_f32: every tensor and sum at f32 accuracy
    // An f32 codec whose convs all fit the split tiles runs them on the f16 matrix cores with
    // split operands (conv_split.hip): activations stored as f16 hi/lo pairs, each conv weight
    // converted once here. Otherwise (or with DTTS_F32_CODEC_KERNEL=f32 set at create) every
    // tensor is plain f32 and every conv the f32 matrix-core kernel.
    bool split = false;
    struct SplitW {
        const void *src;      // the caller's f32 weight
        dtts::half_t *w3;     // [cout, k * 3 cin]
        float inv;            // 2^-s
    };
    std::vector<SplitW> splitw;
    // A decode runs its lanes as two halves, one on the caller's stream and one on `side`, forked
    // and joined with the two events: each launch of one half fills the ramp and tail of the
    // other's (measured: 19.58 -> 19.06 ms for config 5).
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    // Held from the fork record through the join wait, so that decodes from several host threads
    // each wait on their own fork and join: without it one thread's record could land between
    // another's record and wait, and that decode's second half would start on the wrong
    // stream's work.
    mutable std::mutex split_lock;
    // act1 of unit 0 of each block, repeated over the TransConv's `rate` output phases (the
    // TransConv's output channel p*C + c is channel c of phase p).
    std::vector<float *> phase_alpha, phase_brecip;
};

namespace dtts {
namespace {

// Stages whose residual-unit input is wider than this store it snaked as well: the unit's k7 conv
// then reads the snaked copy instead of recomputing SnakeBeta once per output tile. An f32 codec
// stores it at every width: its SnakeBeta is the full-precision sine, which costs the matrix-bound
// k7 conv more than the extra store costs the producer.
constexpr int64_t kStoreSnakedAbove = 96;
inline bool stores_snaked(bool f32, int64_t cout) { return f32 || cout > kStoreSnakedAbove; }

inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

int64_t stage_elems(const dtts_codec_geometry &g, int64_t frames, bool split = false) {
    int64_t m = frames * g.channels[0];
    if (split && frames * g.latent_dim > m) m = frames * g.latent_dim;  // the latent, split
    int64_t len = frames;
    for (int64_t i = 0; i < g.n_blocks; ++i) {
        len *= g.rates[i];
        const int64_t e = len * g.channels[i + 1];
        if (e > m) m = e;
    }
    return m;
}

int64_t hop_of(const dtts_codec_geometry &g) {
    int64_t h = 1;
    for (int64_t i = 0; i < g.n_blocks; ++i) h *= g.rates[i];
    return h;
}

dtts_conv_desc desc(int64_t lanes, int64_t len, int64_t cin, int64_t cout, int64_t k, int64_t dil,
                    const void *x, const void *w, const void *b, void *y) {
    dtts_conv_desc d{};
    d.lanes = lanes;
    d.len = len;
    d.cin = cin;
    d.cout = cout;
    d.k = k;
    d.dilation = dil;
    d.pad_left = (k - 1) * dil;
    d.x = x;
    d.w = w;
    d.bias = b;
    d.y = y;
    return d;
}

}  // namespace
}  // namespace dtts

using dtts::set_error;

namespace dtts {
namespace {
// Every conv of an f32 codec as (weight, cin, cout, k, dilation), the output conv excluded.
template <typename F>
void for_each_conv(const dtts_codec_geometry &g, const dtts_codec_weights &w, F &&f) {
    f(w.head_w, g.latent_dim, g.channels[0], g.head_kernel, int64_t(1));
    for (int64_t i = 0; i < g.n_blocks; ++i) {
        const int64_t cin = g.channels[i], cout = g.channels[i + 1];
        f(w.blocks[i].up_w, cin, g.rates[i] * cout, int64_t(2), int64_t(1));
        for (int j = 0; j < 3; ++j) {
            f(w.blocks[i].units[j].conv1_w, cout, cout, g.ru_kernel, g.ru_dilations[j]);
            f(w.blocks[i].units[j].conv2_w, cout, cout, int64_t(1), int64_t(1));
        }
    }
}

// Converts an f32 codec's conv weights to the split form when every conv (and the output conv's
// split-input window kernel) takes its shape; leaves c->split false otherwise.
int split_codec_weights(dtts_codec *c) {
    const char *env = std::getenv("DTTS_F32_CODEC_KERNEL");
    if (env && std::strcmp(env, "f32") == 0) return DTTS_OK;
    const dtts_codec_geometry &g = c->geo;
    bool ok = g.latent_dim % 8 == 0;
    for_each_conv(g, c->w, [&](const void *, int64_t cin, int64_t cout, int64_t k, int64_t dil) {
        ok = ok && conv_split_supported(1, 1, cin, cout, k, dil);
    });
    dtts_conv_desc od{};
    od.lanes = od.len = 1;
    od.cin = g.channels[g.n_blocks];
    od.cout = 1;
    od.k = g.out_kernel;
    od.dilation = 1;
    od.x = reinterpret_cast<const void *>(uintptr_t(256));  // at decode: a workspace buffer (256-byte aligned)
    ok = ok && conv_f32_narrow_split_eligible(&od);
    if (!ok) return DTTS_OK;
    int rc = DTTS_OK;
    for_each_conv(g, c->w, [&](const void *w, int64_t cin, int64_t cout, int64_t k, int64_t) {
        if (rc != DTTS_OK) return;
        dtts_codec::SplitW sw{w, nullptr, 1.0f};
        const hipError_t e = hipMalloc(&sw.w3, sizeof(half_t) * static_cast<size_t>(3 * k * cin * cout));
        if (e != hipSuccess) {
            set_error("dtts_codec_create_f32: %s", hipGetErrorString(e));
            rc = DTTS_ERR_HIP;
            return;
        }
        c->splitw.push_back(sw);
        rc = split_weight(static_cast<const float *>(w), cout, k, cin, sw.w3, c->splitw.back().inv, nullptr);
    });
    if (rc == DTTS_OK) c->split = true;
    return rc;
}

const dtts_codec::SplitW *split_of(const dtts_codec *c, const void *w) {
    for (const auto &sw : c->splitw)
        if (sw.src == w) return &sw;
    return nullptr;
}

int codec_create(const dtts_codec_geometry *geo, const dtts_codec_weights *w, bool f32, dtts_codec **out) {
    DTTS_REQUIRE(geo && w && out, "dtts_codec_create: null argument");
    *out = nullptr;
    const dtts_codec_geometry &g = *geo;
    DTTS_REQUIRE(g.n_blocks >= 1 && g.n_blocks <= DTTS_CODEC_MAX_BLOCKS, "dtts_codec_create: n_blocks %lld",
                 (long long)g.n_blocks);
    DTTS_REQUIRE(g.latent_dim > 0 && g.head_kernel > 0 && g.ru_kernel > 0 && g.out_kernel > 0,
                 "dtts_codec_create: bad kernel sizes");
    for (int64_t i = 0; i <= g.n_blocks; ++i)
        DTTS_REQUIRE(g.channels[i] > 0, "dtts_codec_create: channels[%lld] = %lld", (long long)i,
                     (long long)g.channels[i]);
    for (int64_t i = 0; i < g.n_blocks; ++i) DTTS_REQUIRE(g.rates[i] > 0, "dtts_codec_create: rates[%lld]", (long long)i);
    for (int j = 0; j < 3; ++j) DTTS_REQUIRE(g.ru_dilations[j] > 0, "dtts_codec_create: ru_dilations[%d]", j);
    DTTS_REQUIRE(w->head_w && w->out_w, "dtts_codec_create: missing head or output weights");
    for (int64_t i = 0; i < g.n_blocks; ++i) {
        const dtts_codec_block &b = w->blocks[i];
        DTTS_REQUIRE(b.act_alpha && b.act_brecip && b.up_w, "dtts_codec_create: block %lld incomplete", (long long)i);
        for (int j = 0; j < 3; ++j) {
            const dtts_codec_unit &u = b.units[j];
            DTTS_REQUIRE(u.act1_alpha && u.act1_brecip && u.conv1_w && u.act2_alpha && u.act2_brecip && u.conv2_w,
                         "dtts_codec_create: block %lld unit %d incomplete", (long long)i, j);
        }
    }
    DTTS_REQUIRE(w->out_alpha && w->out_brecip, "dtts_codec_create: missing output SnakeBeta");

    dtts_codec *c = new (std::nothrow) dtts_codec();
    DTTS_REQUIRE(c, "dtts_codec_create: out of host memory");
    c->geo = g;
    c->w = *w;
    c->f32 = f32;
    {
        hipError_t e = hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&c->fork, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&c->join, hipEventDisableTiming);
        if (e != hipSuccess) {
            dtts_codec_destroy(c);
            set_error("dtts_codec_create: %s", hipGetErrorString(e));
            return DTTS_ERR_HIP;
        }
    }
    if (f32) {
        int rc = split_codec_weights(c);
        if (rc != DTTS_OK) {
            dtts_codec_destroy(c);
            return rc;
        }
    }
    for (int64_t i = 0; i < g.n_blocks; ++i) {
        const int64_t cout = g.channels[i + 1];
        const int64_t rate = g.rates[i];
        float *pa = nullptr, *pr = nullptr;
        if (dtts::stores_snaked(f32, cout)) {
            const size_t bytes = sizeof(float) * static_cast<size_t>(rate * cout);
            hipError_t e = hipMalloc(&pa, bytes);
            if (e == hipSuccess) e = hipMalloc(&pr, bytes);
            for (int64_t p = 0; p < rate && e == hipSuccess; ++p) {
                e = hipMemcpy(pa + p * cout, w->blocks[i].units[0].act1_alpha, sizeof(float) * cout, hipMemcpyDeviceToDevice);
                if (e == hipSuccess)
                    e = hipMemcpy(pr + p * cout, w->blocks[i].units[0].act1_brecip, sizeof(float) * cout, hipMemcpyDeviceToDevice);
            }
            if (e != hipSuccess) {
                if (pa) (void)hipFree(pa);
                if (pr) (void)hipFree(pr);
                dtts_codec_destroy(c);
                set_error("dtts_codec_create: %s", hipGetErrorString(e));
                return DTTS_ERR_HIP;
            }
        }
        c->phase_alpha.push_back(pa);
        c->phase_brecip.push_back(pr);
    }
    *out = c;
    return DTTS_OK;
}
}  // namespace
}  // namespace dtts

extern "C" int dtts_codec_create(const dtts_codec_geometry *geo, const dtts_codec_weights *w, dtts_codec **out) {
    return dtts::codec_create(geo, w, false, out);
}

extern "C" int dtts_codec_create_f32(const dtts_codec_geometry *geo, const dtts_codec_weights *w, dtts_codec **out) {
    return dtts::codec_create(geo, w, true, out);
}

extern "C" void dtts_codec_destroy(dtts_codec *c) {
    if (!c) return;
    if (c->side) (void)hipStreamDestroy(c->side);
    if (c->fork) (void)hipEventDestroy(c->fork);
    if (c->join) (void)hipEventDestroy(c->join);
    for (float *p : c->phase_alpha)
        if (p) (void)hipFree(p);
    for (float *p : c->phase_brecip)
        if (p) (void)hipFree(p);
    for (const auto &sw : c->splitw)
        if (sw.w3) (void)hipFree(sw.w3);
    delete c;
}

extern "C" int64_t dtts_codec_hop(const dtts_codec *c) { return c ? dtts::hop_of(c->geo) : 0; }

bool dtts::codec_is_f32(const dtts_codec *c) { return c && c->f32; }

namespace dtts {
namespace {
// One plan's workspace: four ping-pong buffers of `lanes` x the widest stage.
size_t plan_bytes(const dtts_codec *c, int64_t lanes, int64_t frames) {
    if (lanes <= 0) return 0;
    const size_t esize = c->f32 ? 4 : 2;
    return 4 * round_up(static_cast<size_t>(lanes * stage_elems(c->geo, frames, c->split)) * esize, 256);
}
// The decode's two halves: lanes [0, first) and [first, lanes).
int64_t first_half(int64_t lanes) { return (lanes + 1) / 2; }
}  // namespace
}  // namespace dtts

extern "C" size_t dtts_codec_workspace_bytes(const dtts_codec *c, int64_t lanes, int64_t frames) {
    if (!c || lanes <= 0 || frames <= 0) return 0;
    // room for both halves' plans side by side; a plan over all lanes (the profile) fits too
    const int64_t h0 = dtts::first_half(lanes);
    return dtts::plan_bytes(c, h0, frames) + dtts::plan_bytes(c, lanes - h0, frames);
}

namespace dtts {
namespace {

struct Stage {
    bool ru;           // a fused residual unit (r) rather than one conv (d)
    bool split_in;     // split codec: the latent (d.x, f32) stored split at d.y (rows lanes * len, d.cin wide)
    dtts_conv_desc d;
    dtts_ru_desc r;
    int64_t cv;        // channels of the output's rows: d.cout, or cout / rate for a TransConv
    char name[32];
};

int run_stage(const Stage &st, const dtts_codec *c, hipStream_t stream) {
    if (st.ru) return residual_unit_nlc_f16(&st.r, stream);
    if (!c->split) return c->f32 ? conv1d_nlc_f32(&st.d, stream) : conv1d_nlc_f16(&st.d, stream);
    const dtts_conv_desc &d = st.d;
    if (st.split_in)
        return split_activations(static_cast<const float *>(d.x), static_cast<half_t *>(d.y), d.lanes * d.len, d.cin,
                                 stream);
    if (d.cout == 1) return conv1d_nlc_f32_narrow_split(&d, stream);
    const dtts_codec::SplitW *sw = split_of(c, d.w);
    DTTS_REQUIRE(sw, "dtts_codec (split): a conv weight was not converted at create");
    SplitConv s{};
    s.lanes = d.lanes;
    s.len = d.len;
    s.cs = d.cin;
    s.cout = d.cout;
    s.k = d.k;
    s.dil = d.dilation;
    s.pad_left = d.pad_left;
    s.cv = st.cv;
    s.x = static_cast<const half_t *>(d.x);
    s.w = sw->w3;
    s.w_inv = sw->inv;
    s.bias = static_cast<const float *>(d.bias);
    s.res = static_cast<const half_t *>(d.residual);
    s.y_pre = static_cast<half_t *>(d.y_pre);
    s.y = static_cast<half_t *>(d.y);
    s.a_out = d.out_alpha;
    s.r_out = d.out_brecip;
    return conv1d_nlc_split(s, stream);
}

const char *stage_kernel_name(const Stage &st, const dtts_codec *c) {
    if (st.ru) return residual_unit_kernel_name(&st.r);
    if (!c->split) return c->f32 ? conv_f32_kernel_name(&st.d) : conv_kernel_name(&st.d);
    if (st.split_in) return "split_act_kernel";
    if (st.d.cout == 1) return "conv_nlc_f32_narrow<true>";
    return conv_split_kernel_name(st.d.lanes, st.d.len, st.d.cin, st.d.cout, st.d.k, st.d.dilation);
}

// The decode of `lanes` lanes as a list of conv launches over four buffers of one plan's
// workspace (plan_bytes). The caller has checked the pointers, the workspace's size and alignment.
int build_plan(const dtts_codec *c, const void *latent, void *audio, int64_t lanes, int64_t frames,
               void *workspace, std::vector<Stage> &plan) {
    const dtts_codec_geometry &g = c->geo;
    const dtts_codec_weights &w = c->w;
    const size_t one = plan_bytes(c, lanes, frames) / 4;
    char *buf[4];
    for (int i = 0; i < 4; ++i) buf[i] = static_cast<char *>(workspace) + i * one;
    auto pick = [&](const void *a, const void *b, const void *d) -> char * {
        for (char *p : buf)
            if (p != a && p != b && p != d) return p;
        return nullptr;
    };
    auto push = [&](const dtts_conv_desc &d, const char *fmt, long long a, long long b, int64_t cv = 0) {
        Stage st{};
        st.d = d;
        st.cv = cv > 0 ? cv : d.cout;
        snprintf(st.name, sizeof(st.name), fmt, a, b);
        plan.push_back(st);
    };
    auto push_ru = [&](const dtts_ru_desc &r, long long a, long long b) {
        Stage st{};
        st.ru = true;
        st.r = r;
        snprintf(st.name, sizeof(st.name), "block%lld.unit%lld", a, b);
        plan.push_back(st);
    };

    // head conv, then block 0's SnakeBeta in the epilogue
    char *x = buf[0];
    if (c->split) {  // the latent, stored split for the head conv
        char *lat = pick(x, nullptr, nullptr);
        Stage st{};
        st.split_in = true;
        st.d = desc(lanes, frames, g.latent_dim, g.latent_dim, 1, 1, latent, nullptr, nullptr, lat);
        st.cv = g.latent_dim;
        snprintf(st.name, sizeof(st.name), "latent");
        plan.push_back(st);
        latent = lat;
    }
    {
        dtts_conv_desc d = desc(lanes, frames, g.latent_dim, g.channels[0], g.head_kernel, 1, latent, w.head_w, w.head_b, x);
        d.out_alpha = w.blocks[0].act_alpha;
        d.out_brecip = w.blocks[0].act_brecip;
        push(d, "head%.0lld%.0lld", 0, 0);
    }
    int64_t len = frames;
    for (int64_t i = 0; i < g.n_blocks; ++i) {
        const dtts_codec_block &blk = w.blocks[i];
        const int64_t cin = g.channels[i], cout = g.channels[i + 1], rate = g.rates[i];
        // residual units that fit one workgroup's channel width run fused (ru.hip); the others
        // are two convs, and wide ones read a snaked copy of their input stored beside it
        dtts_ru_desc probe{};
        probe.channels = cout;
        probe.k = g.ru_kernel;
        probe.x = probe.w1 = probe.w2 = probe.b1 = probe.b2 = probe.y = buf[0];
        const bool fused = !c->f32 && [&] {
            for (int j = 0; j < 3; ++j) {
                probe.dilation = g.ru_dilations[j];
                const dtts_codec_unit &un = blk.units[j];
                probe.w1 = un.conv1_w;
                probe.w2 = un.conv2_w;
                probe.b1 = un.conv1_b;
                probe.b2 = un.conv2_b;
                if (!un.conv1_b || !un.conv2_b || !residual_unit_supported(&probe)) return false;
            }
            return true;
        }();
        const bool wide = !fused && stores_snaked(c->f32, cout);
        // TransConv: one causal conv of 2 taps over the snaked input, rate*cout phase columns
        char *u = pick(x, nullptr, nullptr);
        char *su = wide ? pick(x, u, nullptr) : nullptr;
        {
            dtts_conv_desc d = desc(lanes, len, cin, rate * cout, 2, 1, x, blk.up_w, blk.up_b, wide ? su : u);
            if (wide) {
                d.y_pre = u;
                d.out_alpha = c->phase_alpha[i];
                d.out_brecip = c->phase_brecip[i];
            }
            push(d, "block%lld.up%.0lld", (long long)i, 0, cout);
        }
        len *= rate;
        for (int j = 0; j < 3 && fused; ++j) {
            const dtts_codec_unit &un = blk.units[j];
            dtts_ru_desc r{};
            r.lanes = lanes;
            r.len = len;
            r.channels = cout;
            r.k = g.ru_kernel;
            r.dilation = g.ru_dilations[j];
            r.x = u;
            r.act1_alpha = un.act1_alpha;
            r.act1_brecip = un.act1_brecip;
            r.w1 = un.conv1_w;
            r.b1 = un.conv1_b;
            r.act2_alpha = un.act2_alpha;
            r.act2_brecip = un.act2_brecip;
            r.w2 = un.conv2_w;
            r.b2 = un.conv2_b;
            char *y = pick(u, nullptr, nullptr);
            r.y = y;
            if (j == 2) {
                const bool last = i + 1 == g.n_blocks;
                r.out_alpha = last ? w.out_alpha : w.blocks[i + 1].act_alpha;
                r.out_brecip = last ? w.out_brecip : w.blocks[i + 1].act_brecip;
            }
            push_ru(r, (long long)i, j);
            if (j == 2)
                x = y;  // snaked input of the next TransConv (or of the output conv)
            else
                u = y;
        }
        for (int j = 0; j < 3 && !fused; ++j) {
            const dtts_codec_unit &un = blk.units[j];
            char *h = pick(u, su, nullptr);
            {
                dtts_conv_desc d = desc(lanes, len, cout, cout, g.ru_kernel, g.ru_dilations[j], wide ? su : u, un.conv1_w,
                                        un.conv1_b, h);
                if (!wide) {
                    d.in_alpha = un.act1_alpha;
                    d.in_brecip = un.act1_brecip;
                }
                d.out_alpha = un.act2_alpha;
                d.out_brecip = un.act2_brecip;
                push(d, "block%lld.unit%lld.conv1", (long long)i, j);
            }
            // conv2 (k=1) + residual, then the next activation
            char *y = pick(u, h, su);
            dtts_conv_desc d = desc(lanes, len, cout, cout, 1, 1, h, un.conv2_w, un.conv2_b, y);
            d.residual = u;
            if (j < 2) {
                const dtts_codec_unit &nx = blk.units[j + 1];
                if (wide) {
                    // su is dead once conv1 has read it: the snaked copy of y goes there
                    d.y_pre = y;
                    d.y = su;
                    d.out_alpha = nx.act1_alpha;
                    d.out_brecip = nx.act1_brecip;
                }
                push(d, "block%lld.unit%lld.conv2", (long long)i, j);
                u = y;
            } else {
                const bool last = i + 1 == g.n_blocks;
                d.out_alpha = last ? w.out_alpha : w.blocks[i + 1].act_alpha;
                d.out_brecip = last ? w.out_brecip : w.blocks[i + 1].act_brecip;
                push(d, "block%lld.unit%lld.conv2", (long long)i, j);
                x = y;  // snaked input of the next TransConv (or of the output conv)
            }
        }
    }
    dtts_conv_desc d = desc(lanes, len, g.channels[g.n_blocks], 1, g.out_kernel, 1, x, w.out_w, w.out_b, audio);
    d.act = g.out_clamp ? 3 : 1;
    push(d, "out%.0lld%.0lld", 0, 0);
    return DTTS_OK;
}

}  // namespace
}  // namespace dtts

namespace dtts {
namespace {
int check_call(const char *name, const dtts_codec *c, const void *latent, void *audio, int64_t lanes, int64_t frames,
               void *workspace, size_t ws_bytes) {
    DTTS_REQUIRE(c, "%s: null codec", name);
    DTTS_REQUIRE(latent && audio && workspace, "%s: null pointer", name);
    const size_t need = dtts_codec_workspace_bytes(c, lanes, frames);
    DTTS_REQUIRE(ws_bytes >= need, "%s: workspace %zu bytes < %zu needed", name, ws_bytes, need);
    DTTS_REQUIRE(aligned(workspace, 256), "%s: workspace must be 256-byte aligned", name);
    return DTTS_OK;
}

int codec_decode(const char *name, const dtts_codec *c, bool f32, const void *latent, void *audio, int64_t lanes,
                 int64_t frames, void *workspace, size_t ws_bytes, hipStream_t stream) {
    DTTS_REQUIRE(lanes >= 0 && frames >= 0, "%s: negative shape", name);
    if (lanes == 0 || frames == 0) return DTTS_OK;
    DTTS_REQUIRE(c, "%s: null codec", name);
    DTTS_REQUIRE(c->f32 == f32, "%s: the codec was made by %s", name,
                 c->f32 ? "dtts_codec_create_f32 (decode it with dtts_codec_decode_f32)"
                        : "dtts_codec_create (decode it with dtts_codec_decode)");
    int rc = check_call(name, c, latent, audio, lanes, frames, workspace, ws_bytes);
    if (rc != DTTS_OK) return rc;
    const size_t es = c->f32 ? 4 : 2;
    const int64_t h0 = first_half(lanes), h1 = lanes - h0;
    std::vector<Stage> a, b;
    rc = build_plan(c, latent, audio, h0, frames, workspace, a);
    if (rc == DTTS_OK && h1 > 0)
        rc = build_plan(c, static_cast<const char *>(latent) + h0 * frames * c->geo.latent_dim * es,
                        static_cast<char *>(audio) + h0 * frames * hop_of(c->geo) * es, h1, frames,
                        static_cast<char *>(workspace) + plan_bytes(c, h0, frames), b);
    if (rc != DTTS_OK) return rc;
    if (b.empty()) {
        for (const Stage &st : a)
            if ((rc = run_stage(st, c, stream)) != DTTS_OK) return rc;
        return DTTS_OK;
    }
    std::lock_guard<std::mutex> hold(c->split_lock);
    // fork: the side stream starts after everything the caller enqueued before this decode
    DTTS_HIP_CHECK(hipEventRecord(c->fork, stream), name);
    DTTS_HIP_CHECK(hipStreamWaitEvent(c->side, c->fork, 0), name);
    for (size_t i = 0; i < a.size() && rc == DTTS_OK; ++i) {
        rc = run_stage(a[i], c, stream);
        if (rc == DTTS_OK) rc = run_stage(b[i], c, c->side);
    }
    // join, whatever was enqueued: the caller's stream then orders after all of the side's work
    const hipError_t e1 = hipEventRecord(c->join, c->side);
    const hipError_t e2 = e1 == hipSuccess ? hipStreamWaitEvent(stream, c->join, 0) : e1;
    if (rc != DTTS_OK) return rc;
    DTTS_HIP_CHECK(e2, name);
    return DTTS_OK;
}
}  // namespace
}  // namespace dtts

extern "C" int dtts_codec_decode(const dtts_codec *c, const dtts_f16 *latent, dtts_f16 *audio, int64_t lanes,
                                 int64_t frames, void *workspace, size_t ws_bytes, hipStream_t stream) {
    return dtts::codec_decode("dtts_codec_decode", c, false, latent, audio, lanes, frames, workspace, ws_bytes, stream);
}

extern "C" int dtts_codec_decode_f32(const dtts_codec *c, const float *latent, float *audio, int64_t lanes,
                                     int64_t frames, void *workspace, size_t ws_bytes, hipStream_t stream) {
    return dtts::codec_decode("dtts_codec_decode_f32", c, true, latent, audio, lanes, frames, workspace, ws_bytes,
                              stream);
}

extern "C" int dtts_codec_profile(const dtts_codec *c, const void *latent, void *audio, int64_t lanes,
                                  int64_t frames, void *workspace, size_t ws_bytes, hipStream_t stream,
                                  dtts_codec_stage *stages, int max_stages, int *n_stages) {
    DTTS_REQUIRE(stages && n_stages && max_stages > 0, "dtts_codec_profile: no stage table");
    DTTS_REQUIRE(lanes > 0 && frames > 0, "dtts_codec_profile: empty shape");
    int rc = dtts::check_call("dtts_codec_profile", c, latent, audio, lanes, frames, workspace, ws_bytes);
    if (rc != DTTS_OK) return rc;
    std::vector<dtts::Stage> plan;  // all lanes in one plan on one stream: each launch timed alone
    rc = dtts::build_plan(c, latent, audio, lanes, frames, workspace, plan);
    if (rc != DTTS_OK) return rc;
    DTTS_REQUIRE(static_cast<int>(plan.size()) <= max_stages, "dtts_codec_profile: %zu stages > table of %d",
                 plan.size(), max_stages);
    std::vector<hipEvent_t> ev(plan.size() + 1);
    for (auto &e : ev) DTTS_HIP_CHECK(hipEventCreate(&e), "dtts_codec_profile: hipEventCreate");
    int status = DTTS_OK;
    hipError_t he = hipEventRecord(ev[0], stream);
    for (size_t i = 0; i < plan.size() && he == hipSuccess && status == DTTS_OK; ++i) {
        status = dtts::run_stage(plan[i], c, stream);
        if (status == DTTS_OK) he = hipEventRecord(ev[i + 1], stream);
    }
    if (he == hipSuccess && status == DTTS_OK) he = hipEventSynchronize(ev.back());
    for (size_t i = 0; i < plan.size() && he == hipSuccess && status == DTTS_OK; ++i) {
        dtts_codec_stage &s = stages[i];
        std::memset(&s, 0, sizeof(s));
        snprintf(s.name, sizeof(s.name), "%s", plan[i].name);
        if (plan[i].ru) {
            const dtts_ru_desc &r = plan[i].r;
            snprintf(s.kernel, sizeof(s.kernel), "%s", dtts::residual_unit_kernel_name(&r));
            s.lanes = r.lanes;
            s.len = r.len;
            s.cin = s.cout = r.channels;
            s.k = r.k;
            s.dilation = r.dilation;
            const double c = static_cast<double>(r.channels);
            s.flops = 2.0 * r.lanes * r.len * c * c * (r.k + 1);
            s.bytes = 2.0 * r.lanes * r.len * c * (r.y_pre ? 3.0 : 2.0) + 2.0 * c * c * (r.k + 1);
        } else {
            const dtts_conv_desc &d = plan[i].d;
            snprintf(s.kernel, sizeof(s.kernel), "%s", dtts::stage_kernel_name(plan[i], c));
            s.lanes = d.lanes;
            s.len = d.len;
            s.cin = d.cin;
            s.cout = d.cout;
            s.k = d.k;
            s.dilation = d.dilation;
            s.flops = 2.0 * d.lanes * d.len * d.cin * d.cout * d.k;
            const double outs = (d.y_pre ? 2.0 : 1.0) + (d.residual ? 1.0 : 0.0);
            const double es = c->f32 ? 4.0 : 2.0;
            s.bytes = es * d.lanes * d.len * (d.cin + d.cout * outs) + es * d.cout * d.k * d.cin;
            if (plan[i].split_in) {  // a conversion: f32 in, the split pair out
                s.flops = 0.0;
                s.bytes = 8.0 * d.lanes * d.len * d.cin;
            }
        }
        he = hipEventElapsedTime(&s.ms, ev[i], ev[i + 1]);
    }
    for (auto &e : ev) (void)hipEventDestroy(e);
    if (status != DTTS_OK) return status;
    DTTS_HIP_CHECK(he, "dtts_codec_profile");
    *n_stages = static_cast<int>(plan.size());
    return DTTS_OK;
}
