// Codec::load (crates/qwen3tts/src/codec.rs:347-399) from a checkpoint: the reference's tensor
// names, checked against the geometries, converted on the device into one arena in the layouts
// dtts_codec_front_create and dtts_codec_create take.
//
// Two passes over one plan: the first only looks tensors up and checks their shapes and dtypes
// (so a bad checkpoint fails before anything is allocated) while counting the arena's bytes; the
// second uploads each raw tensor once into a device copy of the file's byte buffer, runs the
// conversion into the arena, and fills the weight tables.
#include <new>
#include <string>
#include <unordered_set>

#include "common.hpp"

struct dtts_codec_model {
    void *arena = nullptr;
    size_t bytes = 0;
    dtts_codec_front *front = nullptr;
    dtts_codec *wave = nullptr;
};

namespace dtts {
namespace {

constexpr float kClusterUsageEps = 1e-5f;  // CLUSTER_USAGE_EPSILON (cfg.rs:224) as the f32 clamp

inline size_t round256(size_t v) { return (v + 255) & ~size_t(255); }

struct Build {
    const dtts_checkpoint *ck = nullptr;
    hipStream_t stream = nullptr;
    bool dry = true;
    char *arena = nullptr;       // second pass: the weights
    char *raw = nullptr;         // second pass: device copy of the file's byte buffer
    const char *host0 = nullptr; // first byte of the file's byte buffer (host mapping)
    size_t used = 0;
    std::unordered_set<size_t> sent;  // byte offsets of the raw tensors uploaded
    int rc = DTTS_OK;

    bool fail(int code) {
        if (rc == DTTS_OK) rc = code;
        return false;
    }
    bool ok(int code) { return code == DTTS_OK || fail(code); }

    // The tensor `name` of a float dtype, with exactly `shape` (when `shape` is empty: any shape
    // of `numel` elements).
    bool need(const std::string &name, std::initializer_list<int64_t> shape, dtts_tensor_info &t,
              int64_t numel = 0) {
        if (rc != DTTS_OK) return false;
        if (dtts_checkpoint_get(ck, name.c_str(), &t) != DTTS_OK) return fail(DTTS_ERR_INVALID);
        if (t.dtype != DTTS_DT_F32 && t.dtype != DTTS_DT_F16 && t.dtype != DTTS_DT_BF16 && t.dtype != DTTS_DT_F64) {
            set_error("dtts_codec_model_load: %s: dtype %d is not a float type", name.c_str(), t.dtype);
            return fail(DTTS_ERR_INVALID);
        }
        bool match;
        if (shape.size() == 0) {
            int64_t n = 1;
            for (int i = 0; i < t.ndim; ++i) n *= t.shape[i];
            match = n == numel;
        } else {
            match = static_cast<int>(shape.size()) == t.ndim;
            int i = 0;
            for (int64_t d : shape) match = match && t.shape[i++] == d;
        }
        if (!match) {
            std::string got, want;
            for (int i = 0; i < t.ndim; ++i) got += (i ? ", " : "") + std::to_string(t.shape[i]);
            if (shape.size() == 0) {
                want = std::to_string(numel) + " elements";
            } else {
                int i = 0;
                for (int64_t d : shape) want += (i++ ? ", " : "") + std::to_string(d);
                want = "[" + want + "]";
            }
            set_error("dtts_codec_model_load: %s: shape [%s], expected %s", name.c_str(), got.c_str(), want.c_str());
            return fail(DTTS_ERR_INVALID);
        }
        return true;
    }

    // The raw tensor on the device, uploaded on first use (second pass only).
    const void *src(const dtts_tensor_info &t) {
        const size_t off = static_cast<size_t>(static_cast<const char *>(t.data) - host0);
        if (sent.insert(off).second && t.bytes) {
            const hipError_t e = hipMemcpyAsync(raw + off, t.data, t.bytes, hipMemcpyHostToDevice, stream);
            if (e != hipSuccess) {
                set_error("dtts_codec_model_load: uploading %s: %s", t.name, hipGetErrorString(e));
                fail(DTTS_ERR_HIP);
            }
        }
        return raw + off;
    }

    template <typename T>
    T *alloc(int64_t n) {
        const size_t at = used;
        used += round256(sizeof(T) * static_cast<size_t>(n));
        return dry ? nullptr : reinterpret_cast<T *>(arena + at);
    }

    // --- the conversions the plan uses; each returns the arena pointer (nullptr on the first pass)
    dtts_f16 *f16(const dtts_tensor_info &t, int64_t n) {
        dtts_f16 *d = alloc<dtts_f16>(n);
        if (!dry && rc == DTTS_OK) ok(dtts_convert_f16(src(t), t.dtype, d, n, stream));
        return d;
    }
    float *f32(const dtts_tensor_info &t, int64_t n) {
        float *d = alloc<float>(n);
        if (!dry && rc == DTTS_OK) ok(dtts_convert_f32(src(t), t.dtype, d, n, stream));
        return d;
    }
    dtts_f16 *tap(const dtts_tensor_info &t, int64_t cout, int64_t cin, int64_t k) {
        dtts_f16 *d = alloc<dtts_f16>(cout * cin * k);
        if (!dry && rc == DTTS_OK) ok(dtts_convert_tap_major_f16(src(t), t.dtype, d, cout, cin, k, stream));
        return d;
    }
    dtts_f16 *ttap(const dtts_tensor_info &t, int64_t cin, int64_t cout, int64_t kernel, int64_t stride) {
        dtts_f16 *d = alloc<dtts_f16>(cin * cout * kernel);
        if (!dry && rc == DTTS_OK)
            ok(dtts_convert_transpose_tap_major_f16(src(t), t.dtype, d, cin, cout, kernel, stride, stream));
        return d;
    }
    dtts_f16 *repeat(const dtts_tensor_info &t, int64_t n, int64_t times) {
        dtts_f16 *d = alloc<dtts_f16>(n * times);
        if (!dry && rc == DTTS_OK) ok(dtts_convert_repeat_f16(src(t), t.dtype, d, n, times, stream));
        return d;
    }
    // rows of `t` ([rows, cols]) into rows [row0, row0 + rows) of `d` ([*, cols])
    void rows_into(const dtts_tensor_info &t, dtts_f16 *d, int64_t row0, int64_t rows, int64_t cols) {
        if (!dry && rc == DTTS_OK) ok(dtts_convert_f16(src(t), t.dtype, d + row0 * cols, rows * cols, stream));
    }
    void cols_into(const dtts_tensor_info &t, dtts_f16 *d, int64_t rows, int64_t cols, int64_t ld, int64_t col0) {
        if (!dry && rc == DTTS_OK) ok(dtts_convert_f16_cols(src(t), t.dtype, d, rows, cols, ld, col0, stream));
    }
    void snake(const std::string &prefix, int64_t c, const float *&alpha, const float *&brecip) {
        dtts_tensor_info a, b;
        if (!need(prefix + ".alpha", {}, a, c) || !need(prefix + ".beta", {}, b, c)) return;
        if (a.dtype != b.dtype) {
            set_error("dtts_codec_model_load: %s.alpha and .beta differ in dtype", prefix.c_str());
            fail(DTTS_ERR_INVALID);
            return;
        }
        float *pa = alloc<float>(c), *pb = alloc<float>(c);
        if (!dry && rc == DTTS_OK) {
            const void *sa = src(a), *sb = src(b);
            ok(dtts_convert_snake_fold(sa, sb, a.dtype, pa, pb, c, stream));
        }
        alpha = pa;
        brecip = pb;
    }
};

// The whole plan: front half (codec.rs:401-424's modules) and waveform stack (codec.rs:426-436's).
void plan(Build &b, const dtts_codec_front_geometry &fg, const dtts_codec_geometry &wg, dtts_codec_front_weights &fw,
          dtts_codec_weights &ww) {
    dtts_tensor_info t, u;
    const std::string q = "decoder.quantizer.", tf = "decoder.pre_transformer.";
    // split RVQ: codebooks folded, the two output projections side by side along the input
    float *books = b.alloc<float>(fg.n_books * fg.book_size * fg.book_dim);
    for (int64_t i = 0; i < fg.n_books; ++i) {
        const bool first = i < fg.n_first;
        const std::string p = q + (first ? "rvq_first" : "rvq_rest") + ".vq.layers." +
                              std::to_string(first ? i : i - fg.n_first) + "._codebook.";
        if (!b.need(p + "embedding_sum", {fg.book_size, fg.book_dim}, t) || !b.need(p + "cluster_usage", {fg.book_size}, u))
            return;
        if (t.dtype != u.dtype) {
            set_error("dtts_codec_model_load: %s: embedding_sum and cluster_usage differ in dtype", p.c_str());
            b.fail(DTTS_ERR_INVALID);
            return;
        }
        if (!b.dry && b.rc == DTTS_OK) {
            const void *ss = b.src(t), *su = b.src(u);
            b.ok(dtts_convert_codebook_fold(ss, su, t.dtype, kClusterUsageEps, books + i * fg.book_size * fg.book_dim,
                                            fg.book_size, fg.book_dim, b.stream));
        }
    }
    fw.codebooks = books;
    dtts_f16 *outp = b.alloc<dtts_f16>(fg.codebook_dim * 2 * fg.book_dim);
    for (int s = 0; s < 2; ++s) {
        if (!b.need(q + (s ? "rvq_rest" : "rvq_first") + ".output_proj.weight", {fg.codebook_dim, fg.book_dim, 1}, t))
            return;
        b.cols_into(t, outp, fg.codebook_dim, fg.book_dim, 2 * fg.book_dim, s * fg.book_dim);
    }
    fw.out_proj = outp;
    if (!b.need("decoder.pre_conv.conv.weight", {fg.latent_dim, fg.codebook_dim, fg.pre_kernel}, t)) return;
    fw.pre_w = b.tap(t, fg.latent_dim, fg.codebook_dim, fg.pre_kernel);
    if (!b.need("decoder.pre_conv.conv.bias", {fg.latent_dim}, t)) return;
    fw.pre_b = b.f16(t, fg.latent_dim);
    if (!b.need(tf + "input_proj.weight", {fg.tf_dim, fg.latent_dim}, t)) return;
    fw.in_w = b.f16(t, fg.tf_dim * fg.latent_dim);
    if (!b.need(tf + "input_proj.bias", {fg.tf_dim}, t)) return;
    fw.in_b = b.f16(t, fg.tf_dim);
    // the windowed transformer (Layer::load, qwen3.rs:61-119): q|k|v and gate|up rows joined
    const int64_t D = fg.tf_head_dim, qw = fg.tf_heads * D, kvw = fg.tf_n_kv * D, dim = fg.tf_dim;
    for (int64_t i = 0; i < fg.tf_layers; ++i) {
        const std::string p = tf + "layers." + std::to_string(i) + ".";
        dtts_codec_front_layer &L = fw.layers[i];
        if (!b.need(p + "input_layernorm.weight", {dim}, t)) return;
        L.attn_norm = b.f32(t, dim);
        if (!b.need(p + "post_attention_layernorm.weight", {dim}, t)) return;
        L.ffn_norm = b.f32(t, dim);
        if (!b.need(p + "self_attn_layer_scale.scale", {dim}, t)) return;
        L.attn_scale = b.f32(t, dim);
        if (!b.need(p + "mlp_layer_scale.scale", {dim}, t)) return;
        L.mlp_scale = b.f32(t, dim);
        dtts_f16 *qkv = b.alloc<dtts_f16>((qw + 2 * kvw) * dim);
        if (!b.need(p + "self_attn.q_proj.weight", {qw, dim}, t)) return;
        b.rows_into(t, qkv, 0, qw, dim);
        if (!b.need(p + "self_attn.k_proj.weight", {kvw, dim}, t)) return;
        b.rows_into(t, qkv, qw, kvw, dim);
        if (!b.need(p + "self_attn.v_proj.weight", {kvw, dim}, t)) return;
        b.rows_into(t, qkv, qw + kvw, kvw, dim);
        L.wqkv = qkv;
        if (!b.need(p + "self_attn.o_proj.weight", {dim, qw}, t)) return;
        L.wo = b.f16(t, dim * qw);
        dtts_f16 *gu = b.alloc<dtts_f16>(2 * fg.tf_ffn * dim);
        if (!b.need(p + "mlp.gate_proj.weight", {fg.tf_ffn, dim}, t)) return;
        b.rows_into(t, gu, 0, fg.tf_ffn, dim);
        if (!b.need(p + "mlp.up_proj.weight", {fg.tf_ffn, dim}, t)) return;
        b.rows_into(t, gu, fg.tf_ffn, fg.tf_ffn, dim);
        L.w_gateup = gu;
        if (!b.need(p + "mlp.down_proj.weight", {dim, fg.tf_ffn}, t)) return;
        L.wdown = b.f16(t, dim * fg.tf_ffn);
    }
    if (!b.need(tf + "norm.weight", {dim}, t)) return;
    fw.tf_norm = b.f32(t, dim);
    if (!b.need(tf + "output_proj.weight", {fg.latent_dim, dim}, t)) return;
    fw.out_w = b.f16(t, fg.latent_dim * dim);
    if (!b.need(tf + "output_proj.bias", {fg.latent_dim}, t)) return;
    fw.out_b = b.f16(t, fg.latent_dim);
    // upsampling: TransConv (kernel = stride = r) and ConvNext (codec.rs:124-196)
    const int64_t C = fg.latent_dim;
    for (int64_t i = 0; i < fg.n_up; ++i) {
        const int64_t r = fg.up_ratios[i];
        const std::string p = "decoder.upsample." + std::to_string(i) + ".";
        dtts_codec_front_up &U = fw.up[i];
        if (!b.need(p + "0.conv.weight", {C, C, r}, t)) return;
        U.up_w = b.ttap(t, C, C, r, r);
        if (!b.need(p + "0.conv.bias", {C}, t)) return;
        U.up_b = b.repeat(t, C, r);
        if (!b.need(p + "1.dwconv.conv.weight", {C, 1, fg.dw_kernel}, t)) return;
        U.dw_taps = b.f32(t, C * fg.dw_kernel);
        if (!b.need(p + "1.dwconv.conv.bias", {C}, t)) return;
        U.dw_bias = b.f32(t, C);
        if (!b.need(p + "1.norm.weight", {C}, t)) return;
        U.ln_weight = b.f32(t, C);
        if (!b.need(p + "1.norm.bias", {C}, t)) return;
        U.ln_bias = b.f32(t, C);
        if (!b.need(p + "1.pwconv1.weight", {4 * C, C}, t)) return;
        U.pw1_w = b.f16(t, 4 * C * C);
        if (!b.need(p + "1.pwconv1.bias", {4 * C}, t)) return;
        U.pw1_b = b.f16(t, 4 * C);
        if (!b.need(p + "1.pwconv2.weight", {C, 4 * C}, t)) return;
        U.pw2_w = b.f16(t, 4 * C * C);
        if (!b.need(p + "1.pwconv2.bias", {C}, t)) return;
        U.pw2_b = b.f16(t, C);
        if (!b.need(p + "1.gamma", {C}, t)) return;
        U.gamma = b.f32(t, C);
    }
    // the waveform stack: decoder.decoder is [head conv, blocks..., SnakeBeta, out conv]
    const std::string d = "decoder.decoder.";
    if (!b.need(d + "0.conv.weight", {wg.channels[0], wg.latent_dim, wg.head_kernel}, t)) return;
    ww.head_w = b.tap(t, wg.channels[0], wg.latent_dim, wg.head_kernel);
    if (!b.need(d + "0.conv.bias", {wg.channels[0]}, t)) return;
    ww.head_b = b.f16(t, wg.channels[0]);
    for (int64_t i = 0; i < wg.n_blocks; ++i) {
        const int64_t cin = wg.channels[i], c = wg.channels[i + 1], rate = wg.rates[i];
        const std::string p = d + std::to_string(i + 1) + ".block.";
        dtts_codec_block &B = ww.blocks[i];
        b.snake(p + "0", cin, B.act_alpha, B.act_brecip);
        if (!b.need(p + "1.conv.weight", {cin, c, 2 * rate}, t)) return;
        B.up_w = b.ttap(t, cin, c, 2 * rate, rate);
        if (!b.need(p + "1.conv.bias", {c}, t)) return;
        B.up_b = b.repeat(t, c, rate);
        for (int j = 0; j < 3; ++j) {
            const std::string pu = p + std::to_string(j + 2) + ".";
            dtts_codec_unit &Un = B.units[j];
            b.snake(pu + "act1", c, Un.act1_alpha, Un.act1_brecip);
            if (!b.need(pu + "conv1.conv.weight", {c, c, wg.ru_kernel}, t)) return;
            Un.conv1_w = b.tap(t, c, c, wg.ru_kernel);
            if (!b.need(pu + "conv1.conv.bias", {c}, t)) return;
            Un.conv1_b = b.f16(t, c);
            b.snake(pu + "act2", c, Un.act2_alpha, Un.act2_brecip);
            if (!b.need(pu + "conv2.conv.weight", {c, c, 1}, t)) return;
            Un.conv2_w = b.tap(t, c, c, 1);
            if (!b.need(pu + "conv2.conv.bias", {c}, t)) return;
            Un.conv2_b = b.f16(t, c);
        }
    }
    const int64_t n = wg.n_blocks, cl = wg.channels[n];
    b.snake(d + std::to_string(n + 1), cl, ww.out_alpha, ww.out_brecip);
    if (!b.need(d + std::to_string(n + 2) + ".conv.weight", {1, cl, wg.out_kernel}, t)) return;
    ww.out_w = b.tap(t, 1, cl, wg.out_kernel);
    if (!b.need(d + std::to_string(n + 2) + ".conv.bias", {1}, t)) return;
    ww.out_b = b.f16(t, 1);
}

}  // namespace
}  // namespace dtts

extern "C" int dtts_codec_model_load(const dtts_checkpoint *ck, const dtts_codec_front_geometry *front,
                                     const dtts_codec_geometry *wave, hipStream_t stream, dtts_codec_model **out) {
    const char *name = "dtts_codec_model_load";
    DTTS_REQUIRE(ck && front && wave && out, "%s: null argument", name);
    *out = nullptr;
    DTTS_REQUIRE(front->latent_dim == wave->latent_dim, "%s: front half latent %lld != waveform stack latent %lld",
                 name, (long long)front->latent_dim, (long long)wave->latent_dim);
    DTTS_REQUIRE(front->tf_layers >= 0 && front->tf_layers <= DTTS_FRONT_MAX_LAYERS && front->n_up >= 0 &&
                     front->n_up <= DTTS_FRONT_MAX_UP && wave->n_blocks >= 1 && wave->n_blocks <= DTTS_CODEC_MAX_BLOCKS &&
                     front->n_first > 0 && front->n_first < front->n_books,
                 "%s: bad geometry", name);
    dtts_codec_front_weights fw{};
    dtts_codec_weights ww{};
    dtts::Build b;
    b.ck = ck;
    b.stream = stream;
    dtts::plan(b, *front, *wave, fw, ww);  // first pass: checks and sizes
    if (b.rc != DTTS_OK) return b.rc;
    dtts_codec_model *m = new (std::nothrow) dtts_codec_model();
    DTTS_REQUIRE(m, "%s: out of host memory", name);
    m->bytes = b.used;
    // the raw buffer spans the file's byte buffer; offsets into it are the file's own
    dtts_tensor_info t0{};
    size_t raw_bytes = 0;
    const char *host0 = nullptr;
    for (int64_t i = 0; i < dtts_checkpoint_count(ck); ++i) {
        if (dtts_checkpoint_at(ck, i, &t0) != DTTS_OK) continue;
        const char *p = static_cast<const char *>(t0.data);
        if (!host0 || p < host0) host0 = p;
    }
    for (int64_t i = 0; i < dtts_checkpoint_count(ck); ++i) {
        if (dtts_checkpoint_at(ck, i, &t0) != DTTS_OK) continue;
        const size_t end = static_cast<size_t>(static_cast<const char *>(t0.data) - host0) + t0.bytes;
        if (end > raw_bytes) raw_bytes = end;
    }
    hipError_t e = hipMalloc(&m->arena, m->bytes);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&b.raw), raw_bytes ? raw_bytes : 1);
    if (e != hipSuccess) {
        if (b.raw) (void)hipFree(b.raw);
        dtts_codec_model_destroy(m);
        dtts::set_error("%s: allocating %zu + %zu bytes: %s", name, b.used, raw_bytes, hipGetErrorString(e));
        return DTTS_ERR_HIP;
    }
    b.dry = false;
    b.arena = static_cast<char *>(m->arena);
    b.host0 = host0;
    b.used = 0;
    dtts::plan(b, *front, *wave, fw, ww);  // second pass: upload and convert
    e = hipStreamSynchronize(stream);      // the raw copies are read by now; the staging can go
    (void)hipFree(b.raw);
    int rc = b.rc;
    if (rc == DTTS_OK && e != hipSuccess) {
        dtts::set_error("%s: %s", name, hipGetErrorString(e));
        rc = DTTS_ERR_HIP;
    }
    if (rc == DTTS_OK) rc = dtts_codec_front_create(front, &fw, &m->front);
    if (rc == DTTS_OK) rc = dtts_codec_create(wave, &ww, &m->wave);
    if (rc != DTTS_OK) {
        dtts_codec_model_destroy(m);
        return rc;
    }
    *out = m;
    return DTTS_OK;
}

extern "C" void dtts_codec_model_destroy(dtts_codec_model *m) {
    if (!m) return;
    if (m->wave) dtts_codec_destroy(m->wave);
    if (m->front) dtts_codec_front_destroy(m->front);
    if (m->arena) (void)hipFree(m->arena);
    delete m;
}

extern "C" const dtts_codec_front *dtts_codec_model_front(const dtts_codec_model *m) { return m ? m->front : nullptr; }
extern "C" const dtts_codec *dtts_codec_model_wave(const dtts_codec_model *m) { return m ? m->wave : nullptr; }
extern "C" size_t dtts_codec_model_bytes(const dtts_codec_model *m) { return m ? m->bytes : 0; }
