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

// A projection of the stack's weight kind, built from one or more [rows, cols] source tensors
// stacked along rows (Layer::load's q|k|v cat, gate|up): f16 or f32 rows converted in place; Q8_0
// rows quantized into a staging buffer of GGML blocks (QTensor::quantize_onto, bit for bit the
// host quantizer) and repacked into the arena once the projection is whole.
struct Proj {
    Build &b;
    int32_t how;
    int64_t rows, cols;
    void *dst = nullptr;
    Proj(Build &b_, int32_t how_, int64_t rows_, int64_t cols_) : b(b_), how(how_), rows(rows_), cols(cols_) {
        if (how == DTTS_WEIGHT_F16) dst = b.alloc<dtts_f16>(rows * cols);
        else if (how == DTTS_WEIGHT_F32) dst = b.alloc<float>(rows * cols);
        else {
            dst = b.alloc<uint8_t>(static_cast<int64_t>(dtts_q8_0_packed_bytes(rows, cols)));
            const size_t staging = static_cast<size_t>(rows * (cols / 32) * 34);
            if (staging > b.q8max) b.q8max = staging;
        }
    }
    void put(const dtts_tensor_info &t, int64_t row0, int64_t n) {
        if (b.dry || b.rc != DTTS_OK) return;
        if (how == DTTS_WEIGHT_F16)
            b.rows_into(t, static_cast<dtts_f16 *>(dst), row0, n, cols);
        else if (how == DTTS_WEIGHT_F32)
            b.ok(dtts_convert_f32(b.src(t), t.dtype, static_cast<float *>(dst) + row0 * cols, n * cols, b.stream));
        else
            b.ok(dtts_convert_q8_0(b.src(t), t.dtype, b.q8tmp + row0 * (cols / 32) * 34, n, cols, b.stream));
    }
    const void *done() {
        if (!b.dry && b.rc == DTTS_OK && how != DTTS_WEIGHT_F16 && how != DTTS_WEIGHT_F32)
            b.ok(dtts_q8_0_repack(b.q8tmp, dst, rows, cols, b.stream));
        return dst;
    }
};

void stack_plan(Build &b, const std::string &prefix, const dtts_stack_geometry &g, int32_t how,
                dtts_stack_layer *layers, const float *&final_norm) {
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
        Proj qkv(b, how, qw + 2 * kvw, dim);
        if (!b.need(p + "self_attn.q_proj.weight", {qw, dim}, t)) return;
        qkv.put(t, 0, qw);
        if (!b.need(p + "self_attn.k_proj.weight", {kvw, dim}, t)) return;
        qkv.put(t, qw, kvw);
        if (!b.need(p + "self_attn.v_proj.weight", {kvw, dim}, t)) return;
        qkv.put(t, qw + kvw, kvw);
        L.wqkv = qkv.done();
        Proj wo(b, how, dim, qw);
        if (!b.need(p + "self_attn.o_proj.weight", {dim, qw}, t)) return;
        wo.put(t, 0, dim);
        L.wo = wo.done();
        Proj gu(b, how, 2 * g.ffn, dim);
        if (!b.need(p + "mlp.gate_proj.weight", {g.ffn, dim}, t)) return;
        gu.put(t, 0, g.ffn);
        if (!b.need(p + "mlp.up_proj.weight", {g.ffn, dim}, t)) return;
        gu.put(t, g.ffn, g.ffn);
        L.w_gateup = gu.done();
        Proj down(b, how, dim, g.ffn);
        if (!b.need(p + "mlp.down_proj.weight", {dim, g.ffn}, t)) return;
        down.put(t, 0, dim);
        L.wdown = down.done();
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
    return dtts_stack_model_load_as(ck, prefix, geo, DTTS_WEIGHT_F16, stream, out);
}

extern "C" int dtts_stack_model_load_as(const dtts_checkpoint *ck, const char *prefix, const dtts_stack_geometry *geo,
                                        int32_t how, hipStream_t stream, dtts_stack_model **out) {
    const char *name = "dtts_stack_model_load";
    DTTS_REQUIRE(ck && prefix && geo && out, "%s: null argument", name);
    *out = nullptr;
    DTTS_REQUIRE(geo->layers > 0 && geo->layers <= 1024 && geo->dim > 0 && geo->heads > 0 && geo->n_kv > 0 &&
                     geo->head_dim > 0 && geo->ffn > 0,
                 "%s: bad geometry", name);
    DTTS_REQUIRE(how == DTTS_WEIGHT_F16 || how == DTTS_WEIGHT_F32 || how == DTTS_WEIGHT_Q8_0 ||
                     how == DTTS_WEIGHT_Q8_0_A32,
                 "%s: weight kind %d unknown", name, how);
    if (how == DTTS_WEIGHT_Q8_0 || how == DTTS_WEIGHT_Q8_0_A32)
        DTTS_REQUIRE(geo->dim % 256 == 0 && (geo->heads * geo->head_dim) % 256 == 0 && geo->ffn % 256 == 0,
                     "%s: Q8_0 layers need dim, heads*head_dim and ffn multiples of 256", name);
    std::vector<dtts_stack_layer> layers(static_cast<size_t>(geo->layers));
    const float *final_norm = nullptr;
    dtts::Build b;
    b.who = name;
    b.ck = ck;
    b.stream = stream;
    dtts::stack_plan(b, prefix, *geo, how, layers.data(), final_norm);
    if (b.rc != DTTS_OK) return b.rc;
    dtts_stack_model *m = new (std::nothrow) dtts_stack_model();
    DTTS_REQUIRE(m, "%s: out of host memory", name);
    m->bytes = b.used;
    const char *host0 = nullptr;
    const size_t raw_bytes = dtts::Build::raw_span(ck, host0);
    hipError_t e = hipMalloc(&m->arena, m->bytes);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void **>(&b.raw), raw_bytes ? raw_bytes : 1);
    if (e == hipSuccess && b.q8max) e = hipMalloc(reinterpret_cast<void **>(&b.q8tmp), b.q8max);
    if (e != hipSuccess) {
        if (b.raw) (void)hipFree(b.raw);
        if (b.q8tmp) (void)hipFree(b.q8tmp);
        dtts_stack_model_destroy(m);
        dtts::set_error("%s: allocating %zu + %zu + %zu bytes: %s", name, b.used, raw_bytes, b.q8max,
                        hipGetErrorString(e));
        return DTTS_ERR_HIP;
    }
    b.dry = false;
    b.arena = static_cast<char *>(m->arena);
    b.host0 = host0;
    b.used = 0;
    dtts::stack_plan(b, prefix, *geo, how, layers.data(), final_norm);
    e = hipStreamSynchronize(stream);
    (void)hipFree(b.raw);
    if (b.q8tmp) (void)hipFree(b.q8tmp);
    int rc = b.rc;
    if (rc == DTTS_OK && e != hipSuccess) {
        dtts::set_error("%s: %s", name, hipGetErrorString(e));
        rc = DTTS_ERR_HIP;
    }
    if (rc == DTTS_OK) rc = dtts_stack_create_as(geo, layers.data(), final_norm, how, &m->stack);
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
