// Stack::load (crates/qwen3tts/src/qwen3.rs:61-119, 226-250) from a checkpoint: each layer's
// norms, projections and optional QK-norm / LayerScale tensors under "<prefix>layers.<i>.",
// checked against the geometry, converted into one device arena in dtts_stack_create's layouts.
#include <cmath>
#include <new>
#include <string>
#include <vector>

#include "loader.hpp"

struct dtts_stack_model {
    void *arena = nullptr;
    size_t bytes = 0;
    dtts_stack *stack = nullptr;
};

namespace dtts {
namespace {

void stack_plan(Build &b, const std::string &prefix, const dtts_stack_geometry &g, dtts_stack_layer *layers,
                const float *&final_norm) {
    dtts_tensor_info t;
    const int64_t D = g.head_dim, qw = g.heads * D, kvw = g.n_kv * D, dim = g.dim;
    // q's norm weight times 1/sqrt(head_dim) in f32, as the host path folds it
    const float qscale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(D)));
    for (int64_t i = 0; i < g.layers; ++i) {
        const std::string p = prefix + "layers." + std::to_string(i) + ".";
        dtts_stack_layer &L = layers[i];
        if (!b.need(p + "input_layernorm.weight", {dim}, t)) return;
        L.attn_norm = b.f32(t, dim);
        if (!b.need(p + "post_attention_layernorm.weight", {dim}, t)) return;
        L.ffn_norm = b.f32(t, dim);
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
        dtts_f16 *gu = b.alloc<dtts_f16>(2 * g.ffn * dim);
        if (!b.need(p + "mlp.gate_proj.weight", {g.ffn, dim}, t)) return;
        b.rows_into(t, gu, 0, g.ffn, dim);
        if (!b.need(p + "mlp.up_proj.weight", {g.ffn, dim}, t)) return;
        b.rows_into(t, gu, g.ffn, g.ffn, dim);
        L.w_gateup = gu;
        if (!b.need(p + "mlp.down_proj.weight", {dim, g.ffn}, t)) return;
        L.wdown = b.f16(t, dim * g.ffn);
        L.qk_norms = nullptr;
        if (g.qk_norm) {
            float *qk = b.alloc<float>(2 * D);
            if (!b.need(p + "self_attn.q_norm.weight", {D}, t)) return;
            if (!b.dry && b.rc == DTTS_OK) b.ok(dtts_convert_f32_scaled(b.src(t), t.dtype, qk, D, qscale, b.stream));
            if (!b.need(p + "self_attn.k_norm.weight", {D}, t)) return;
            if (!b.dry && b.rc == DTTS_OK) b.ok(dtts_convert_f32(b.src(t), t.dtype, qk ? qk + D : nullptr, D, b.stream));
            L.qk_norms = qk;
        }
        L.attn_scale = L.mlp_scale = nullptr;
        if (g.layer_scale) {
            if (!b.need(p + "self_attn_layer_scale.scale", {dim}, t)) return;
            L.attn_scale = b.f32(t, dim);
            if (!b.need(p + "mlp_layer_scale.scale", {dim}, t)) return;
            L.mlp_scale = b.f32(t, dim);
        }
    }
    if (!b.need(prefix + "norm.weight", {dim}, t)) return;
    final_norm = b.f32(t, dim);
}

}  // namespace
}  // namespace dtts

extern "C" int dtts_stack_model_load(const dtts_checkpoint *ck, const char *prefix, const dtts_stack_geometry *geo,
                                     hipStream_t stream, dtts_stack_model **out) {
    const char *name = "dtts_stack_model_load";
    DTTS_REQUIRE(ck && prefix && geo && out, "%s: null argument", name);
    *out = nullptr;
    DTTS_REQUIRE(geo->layers > 0 && geo->layers <= 1024 && geo->dim > 0 && geo->heads > 0 && geo->n_kv > 0 &&
                     geo->head_dim > 0 && geo->ffn > 0,
                 "%s: bad geometry", name);
    std::vector<dtts_stack_layer> layers(static_cast<size_t>(geo->layers));
    const float *final_norm = nullptr;
    dtts::Build b;
    b.who = name;
    b.ck = ck;
    b.stream = stream;
    dtts::stack_plan(b, prefix, *geo, layers.data(), final_norm);
    if (b.rc != DTTS_OK) return b.rc;
    dtts_stack_model *m = new (std::nothrow) dtts_stack_model();
    DTTS_REQUIRE(m, "%s: out of host memory", name);
    m->bytes = b.used;
    const char *host0 = nullptr;
    const size_t raw_bytes = dtts::Build::raw_span(ck, host0);
    hipError_t e = hipMalloc(&m->arena, m->bytes);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&b.raw), raw_bytes ? raw_bytes : 1);
    if (e != hipSuccess) {
        if (b.raw) (void)hipFree(b.raw);
        dtts_stack_model_destroy(m);
        dtts::set_error("%s: allocating %zu + %zu bytes: %s", name, b.used, raw_bytes, hipGetErrorString(e));
        return DTTS_ERR_HIP;
    }
    b.dry = false;
    b.arena = static_cast<char *>(m->arena);
    b.host0 = host0;
    b.used = 0;
    dtts::stack_plan(b, prefix, *geo, layers.data(), final_norm);
    e = hipStreamSynchronize(stream);
    (void)hipFree(b.raw);
    int rc = b.rc;
    if (rc == DTTS_OK && e != hipSuccess) {
        dtts::set_error("%s: %s", name, hipGetErrorString(e));
        rc = DTTS_ERR_HIP;
    }
    if (rc == DTTS_OK) rc = dtts_stack_create(geo, layers.data(), final_norm, &m->stack);
    if (rc != DTTS_OK) {
        dtts_stack_model_destroy(m);
        return rc;
    }
    *out = m;
    return DTTS_OK;
}

extern "C" void dtts_stack_model_destroy(dtts_stack_model *m) {
    if (!m) return;
    if (m->stack) dtts_stack_destroy(m->stack);
    if (m->arena) (void)hipFree(m->arena);
    delete m;
}

extern "C" dtts_stack *dtts_stack_model_stack(const dtts_stack_model *m) { return m ? m->stack : nullptr; }
extern "C" size_t dtts_stack_model_bytes(const dtts_stack_model *m) { return m ? m->bytes : 0; }
