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

#include "loader.hpp"

struct dtts_codec_model {
    void *arena = nullptr;
    size_t bytes = 0;
    dtts_codec_front *front = nullptr;
    dtts_codec *wave = nullptr;
};

namespace dtts {
namespace {

constexpr float kClusterUsageEps = 1e-5f;  // CLUSTER_USAGE_EPSILON (cfg.rs:224) as the f32 clamp

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
    b.who = name;
    b.ck = ck;
    b.stream = stream;
    dtts::plan(b, *front, *wave, fw, ww);  // first pass: checks and sizes
    if (b.rc != DTTS_OK) return b.rc;
    dtts_codec_model *m = new (std::nothrow) dtts_codec_model();
    DTTS_REQUIRE(m, "%s: out of host memory", name);
    m->bytes = b.used;
    const char *host0 = nullptr;
    const size_t raw_bytes = dtts::Build::raw_span(ck, host0);
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
