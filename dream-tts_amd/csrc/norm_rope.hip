// Per-step norm and position ops of the decode layer: the entry points, the plain RoPE and KV
// append kernels. RMSNorm and the fused QK-norm + RoPE + append kernels are in norm_rope.hpp.
#include "norm_rope.hpp"

#pragma clang fp contract(off)

namespace dtts {
namespace {

// x, y [rows, heads, D]; thread per (row, head, i < D/2).
template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(const T *x, const float *cos_t, const float *sin_t, T *y, Positions pos,
                                                   int rows, int heads, int hd) {
    const int half = hd / 2;
    const int64_t total = static_cast<int64_t>(rows) * heads * half;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int i = static_cast<int>(e % half);
        const int64_t rh = e / half;
        const int row = static_cast<int>(rh / heads);
        const int64_t base = rh * hd;
        const int p = pos.at(row);
        const float c = cos_t[static_cast<int64_t>(p) * half + i];
        const float s = sin_t[static_cast<int64_t>(p) * half + i];
        float o1, o2;
        rope_pair(static_cast<float>(x[base + i]), static_cast<float>(x[base + i + half]), c, s, o1, o2);
        y[base + i] = static_cast<T>(o1);
        y[base + i + half] = static_cast<T>(o2);
    }
}

// ---------------------------------------------------------------- plain append

// k, v [b, n_kv, D] -> caches [b, n_kv, cap, D] at pos[b]; thread per element.
template <typename T>
__global__ __launch_bounds__(256) void kv_append_kernel(const T *k, const T *v, Positions pos, half_t *kc, half_t *vc,
                                                        int b, int n_kv, int hd, int cap) {
    const int64_t total = static_cast<int64_t>(b) * n_kv * hd;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int d = static_cast<int>(e % hd);
        const int64_t bh = e / hd;
        const int bi = static_cast<int>(bh / n_kv);
        const int64_t dst = (bh * cap + pos.p[bi]) * hd + d;
        kc[dst] = static_cast<half_t>(static_cast<float>(k[e]));
        vc[dst] = static_cast<half_t>(static_cast<float>(v[e]));
    }
}

int load_positions(const char *name, const int32_t *pos, int64_t b, int64_t cap, Positions &out) {
    DTTS_REQUIRE(pos, "%s: null positions", name);
    DTTS_REQUIRE(b <= kMaxLanes, "%s: %lld lanes > %d", name, (long long)b, kMaxLanes);
    for (int64_t i = 0; i < b; ++i) {
        DTTS_REQUIRE(pos[i] >= 0 && pos[i] < cap, "%s: lane %lld position %d outside the cache capacity %lld",
                     name, (long long)i, pos[i], (long long)cap);
        out.p[i] = pos[i];
    }
    return DTTS_OK;
}

template <typename T>
int rms_norm(const char *name, const T *x, const T *gamma, T *y, int64_t rows, int64_t dim, float eps,
             hipStream_t stream) {
    DTTS_REQUIRE(rows >= 0 && dim > 0 && dim < (int64_t(1) << 31), "%s: bad shape (%lld, %lld)", name,
                 (long long)rows, (long long)dim);
    if (rows == 0) return DTTS_OK;
    DTTS_REQUIRE(x && gamma && y, "%s: null pointer", name);
    DTTS_REQUIRE(rows < (int64_t(1) << 31), "%s: too many rows", name);
    const unsigned blocks = static_cast<unsigned>((rows + 3) / 4);
    constexpr int64_t row_vec = 64 * (16 / sizeof(T));  // one 16-byte vector per lane
    const int64_t nv = dim / row_vec;
    if (dim % row_vec == 0 && nv <= 8 && aligned(x, 16) && aligned(gamma, 16) && aligned(y, 16)) {
        const int r = static_cast<int>(rows), d = static_cast<int>(dim);
        if (nv <= 2)
            rms_norm_vec_kernel<T, 2><<<blocks, 256, 0, stream>>>(x, gamma, y, r, d, eps);
        else if (nv <= 4)
            rms_norm_vec_kernel<T, 4><<<blocks, 256, 0, stream>>>(x, gamma, y, r, d, eps);
        else
            rms_norm_vec_kernel<T, 8><<<blocks, 256, 0, stream>>>(x, gamma, y, r, d, eps);
    } else {
        rms_norm_kernel<T><<<blocks, 256, 0, stream>>>(x, gamma, y, static_cast<int>(rows), static_cast<int>(dim), eps);
    }
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

template <typename T>
int rope(const char *name, const T *x, const float *cos_t, const float *sin_t, const int32_t *pos, T *y, int64_t rows,
         int64_t heads, int64_t hd, int64_t table_len, hipStream_t stream) {
    DTTS_REQUIRE(rows >= 0 && heads > 0 && hd > 0 && hd % 2 == 0 && table_len > 0, "%s: bad shape", name);
    if (rows == 0) return DTTS_OK;
    DTTS_REQUIRE(x && y && cos_t && sin_t, "%s: null pointer", name);
    Positions p{};
    int rc = load_positions(name, pos, rows, table_len, p);
    if (rc != DTTS_OK) return rc;
    const int64_t total = rows * heads * hd / 2;
    rope_kernel<T><<<grid_for(total, 256), 256, 0, stream>>>(x, cos_t, sin_t, y, p, static_cast<int>(rows),
                                                             static_cast<int>(heads), static_cast<int>(hd));
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

template <typename T>
int qk_rope(const char *name, const T *qkv, const float *norms, const float *cos_t, const float *sin_t,
            const int32_t *pos, T *q_out, float *k_out, dtts_f16 *kc, dtts_f16 *vc, int64_t b, int64_t heads,
            int64_t n_kv, int64_t hd, int64_t cap, int64_t table_len, float eps, hipStream_t stream) {
    DTTS_REQUIRE(b >= 0 && heads > 0 && n_kv > 0 && hd > 0 && hd % 2 == 0 && hd <= 128 && cap > 0 && table_len > 0,
                 "%s: bad shape (b %lld, heads %lld, n_kv %lld, head_dim %lld, cap %lld)", name, (long long)b,
                 (long long)heads, (long long)n_kv, (long long)hd, (long long)cap);
    if (b == 0) return DTTS_OK;
    DTTS_REQUIRE(qkv && norms && cos_t && sin_t && q_out && kc && vc, "%s: null pointer", name);
    Positions p{};
    int rc = load_positions(name, pos, b, cap < table_len ? cap : table_len, p);
    if (rc != DTTS_OK) return rc;
    const int64_t waves = b * (heads + n_kv);
    qk_rope_kernel<T, Positions><<<static_cast<unsigned>((waves + 3) / 4), 256, 0, stream>>>(
        qkv, norms, cos_t, sin_t, p, q_out, k_out, reinterpret_cast<half_t *>(kc), reinterpret_cast<half_t *>(vc),
        static_cast<int>(b), static_cast<int>(heads), static_cast<int>(n_kv), static_cast<int>(hd),
        static_cast<int>(cap), eps, 1.0f, 1, 0, false);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

// qkrope::apply: t positions per lane from one start, optional f32 k/v side outputs.
int qkrope_apply(const char *name, const float *qkv, const float *norms, const float *cos_t, const float *sin_t,
                 dtts_f16 *kc, dtts_f16 *vc, int64_t heads, int64_t start, float eps, float *q_out, float *k_f32,
                 float *v_f32, int64_t b, int64_t t, int64_t n_kv, int64_t hd, int64_t cap, int64_t table_len,
                 hipStream_t stream) {
    DTTS_REQUIRE(b >= 0 && t >= 0 && start >= 0 && heads > 0 && n_kv > 0 && hd > 0 && hd % 2 == 0 && hd <= 128 &&
                     cap > 0 && table_len > 0,
                 "%s: bad shape (b %lld, t %lld, start %lld, heads %lld, n_kv %lld, head_dim %lld, cap %lld)", name,
                 (long long)b, (long long)t, (long long)start, (long long)heads, (long long)n_kv, (long long)hd,
                 (long long)cap);
    // qkrope.rs:40-44: the new positions must fit the cache (and here the RoPE table too)
    DTTS_REQUIRE(start + t <= cap, "%s: %lld positions exceed %lld", name, (long long)(start + t), (long long)cap);
    DTTS_REQUIRE(start + t <= table_len, "%s: %lld positions exceed the RoPE table's %lld", name,
                 (long long)(start + t), (long long)table_len);
    if (b == 0 || t == 0) return DTTS_OK;
    DTTS_REQUIRE(qkv && norms && cos_t && sin_t && q_out && kc && vc, "%s: null pointer", name);
    DTTS_REQUIRE((k_f32 == nullptr) == (v_f32 == nullptr), "%s: f32 k and v come together (f32_kv)", name);
    const int64_t waves = b * t * (heads + n_kv);
    DTTS_REQUIRE(waves < (int64_t(1) << 31) && cap < (int64_t(1) << 31), "%s: too many rows", name);
    qk_rope_span_kernel<float><<<static_cast<unsigned>((waves + 3) / 4), 256, 0, stream>>>(
        qkv, norms, cos_t, sin_t, q_out, k_f32, v_f32, reinterpret_cast<half_t *>(kc), reinterpret_cast<half_t *>(vc),
        static_cast<int>(b * t), static_cast<int>(t), static_cast<int>(start), static_cast<int>(heads),
        static_cast<int>(n_kv), static_cast<int>(hd), static_cast<int>(cap), eps, 1, 0, false);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

template <typename T>
int kv_append(const char *name, const T *k, const T *v, const int32_t *pos, dtts_f16 *kc, dtts_f16 *vc, int64_t b,
              int64_t n_kv, int64_t hd, int64_t cap, hipStream_t stream) {
    DTTS_REQUIRE(b >= 0 && n_kv > 0 && hd > 0 && cap > 0, "%s: bad shape", name);
    if (b == 0) return DTTS_OK;
    DTTS_REQUIRE(k && v && kc && vc, "%s: null pointer", name);
    Positions p{};
    int rc = load_positions(name, pos, b, cap, p);
    if (rc != DTTS_OK) return rc;
    const int64_t total = b * n_kv * hd;
    kv_append_kernel<T><<<grid_for(total, 256), 256, 0, stream>>>(k, v, p, reinterpret_cast<half_t *>(kc),
                                                                 reinterpret_cast<half_t *>(vc), static_cast<int>(b),
                                                                 static_cast<int>(n_kv), static_cast<int>(hd),
                                                                 static_cast<int>(cap));
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

}  // namespace
}  // namespace dtts

using dtts::half_t;

extern "C" int dtts_rms_norm_f32(const float *x, const float *gamma, float *y, int64_t rows, int64_t dim, float eps,
                                 hipStream_t stream) {
    return dtts::rms_norm<float>("dtts_rms_norm_f32", x, gamma, y, rows, dim, eps, stream);
}

extern "C" int dtts_rms_norm_f16(const dtts_f16 *x, const dtts_f16 *gamma, dtts_f16 *y, int64_t rows, int64_t dim,
                                 float eps, hipStream_t stream) {
    return dtts::rms_norm<half_t>("dtts_rms_norm_f16", reinterpret_cast<const half_t *>(x),
                                  reinterpret_cast<const half_t *>(gamma), reinterpret_cast<half_t *>(y), rows, dim, eps,
                                  stream);
}

extern "C" int dtts_rope_table_f32(int64_t len, int64_t head_dim, double base, float *cos_out, float *sin_out) {
    DTTS_REQUIRE(len >= 0 && head_dim > 0 && head_dim % 2 == 0 && base > 0.0, "dtts_rope_table_f32: bad arguments");
    DTTS_REQUIRE(len == 0 || (cos_out && sin_out), "dtts_rope_table_f32: null output");
    const int64_t half = head_dim / 2;
    for (int64_t t = 0; t < len; ++t)
        for (int64_t i = 0; i < half; ++i) {
            const double freq = 1.0 / std::pow(base, 2.0 * static_cast<double>(i) / static_cast<double>(head_dim));
            const double phase = static_cast<double>(t) * freq;
            cos_out[t * half + i] = static_cast<float>(std::cos(phase));
            sin_out[t * half + i] = static_cast<float>(std::sin(phase));
        }
    return DTTS_OK;
}

extern "C" int dtts_rope_halfsplit_f32(const float *x, const float *cos_t, const float *sin_t, const int32_t *pos,
                                       float *y, int64_t rows, int64_t heads, int64_t head_dim, int64_t table_len,
                                       hipStream_t stream) {
    return dtts::rope<float>("dtts_rope_halfsplit_f32", x, cos_t, sin_t, pos, y, rows, heads, head_dim, table_len,
                             stream);
}

extern "C" int dtts_rope_halfsplit_f16(const dtts_f16 *x, const float *cos_t, const float *sin_t, const int32_t *pos,
                                       dtts_f16 *y, int64_t rows, int64_t heads, int64_t head_dim, int64_t table_len,
                                       hipStream_t stream) {
    return dtts::rope<half_t>("dtts_rope_halfsplit_f16", reinterpret_cast<const half_t *>(x), cos_t, sin_t, pos,
                              reinterpret_cast<half_t *>(y), rows, heads, head_dim, table_len, stream);
}

extern "C" int dtts_qk_norm_rope_kv_append_f32(const float *qkv, const float *norms, const float *cos_t,
                                               const float *sin_t, const int32_t *pos, float *q_out, float *k_out,
                                               dtts_f16 *kcache, dtts_f16 *vcache, int64_t b, int64_t heads,
                                               int64_t n_kv, int64_t head_dim, int64_t cap, int64_t table_len,
                                               float eps, hipStream_t stream) {
    return dtts::qk_rope<float>("dtts_qk_norm_rope_kv_append_f32", qkv, norms, cos_t, sin_t, pos, q_out, k_out, kcache,
                                vcache, b, heads, n_kv, head_dim, cap, table_len, eps, stream);
}

extern "C" int dtts_qk_norm_rope_kv_append_f16(const dtts_f16 *qkv, const float *norms, const float *cos_t,
                                               const float *sin_t, const int32_t *pos, dtts_f16 *q_out, float *k_out,
                                               dtts_f16 *kcache, dtts_f16 *vcache, int64_t b, int64_t heads,
                                               int64_t n_kv, int64_t head_dim, int64_t cap, int64_t table_len,
                                               float eps, hipStream_t stream) {
    return dtts::qk_rope<half_t>("dtts_qk_norm_rope_kv_append_f16", reinterpret_cast<const half_t *>(qkv), norms, cos_t,
                                 sin_t, pos, reinterpret_cast<half_t *>(q_out), k_out, kcache, vcache, b, heads, n_kv,
                                 head_dim, cap, table_len, eps, stream);
}

extern "C" int dtts_qkrope_apply_f32(const float *qkv, const float *norms, const float *cos_t, const float *sin_t,
                                     dtts_f16 *kcache, dtts_f16 *vcache, int64_t heads, int64_t start, float eps,
                                     float *q_out, float *k_f32, float *v_f32, int64_t b, int64_t t, int64_t n_kv,
                                     int64_t head_dim, int64_t cap, int64_t table_len, hipStream_t stream) {
    return dtts::qkrope_apply("dtts_qkrope_apply_f32", qkv, norms, cos_t, sin_t, kcache, vcache, heads, start, eps,
                              q_out, k_f32, v_f32, b, t, n_kv, head_dim, cap, table_len, stream);
}

extern "C" int dtts_kv_append_f32(const float *k, const float *v, const int32_t *pos, dtts_f16 *kcache,
                                  dtts_f16 *vcache, int64_t b, int64_t n_kv, int64_t head_dim, int64_t cap,
                                  hipStream_t stream) {
    return dtts::kv_append<float>("dtts_kv_append_f32", k, v, pos, kcache, vcache, b, n_kv, head_dim, cap, stream);
}

extern "C" int dtts_kv_append_f16(const dtts_f16 *k, const dtts_f16 *v, const int32_t *pos, dtts_f16 *kcache,
                                  dtts_f16 *vcache, int64_t b, int64_t n_kv, int64_t head_dim, int64_t cap,
                                  hipStream_t stream) {
    return dtts::kv_append<half_t>("dtts_kv_append_f16", reinterpret_cast<const half_t *>(k),
                                   reinterpret_cast<const half_t *>(v), pos, kcache, vcache, b, n_kv, head_dim, cap,
                                   stream);
}
