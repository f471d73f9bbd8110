// Decode attention entry points: host-side checks and the launch plan; the kernels are in
// attn.hpp.
#include "attn.hpp"

namespace dtts {
namespace {

template <typename T>
int decode_attention(const char *name, const float *q, const T *kc, const T *vc, float *out, int64_t b, int64_t n_kv,
                     int64_t gqa, int64_t head_dim, int64_t cap, const int32_t *span, const int32_t *window_start,
                     void *workspace, size_t ws_bytes, hipStream_t stream) {
    DTTS_REQUIRE(b >= 0 && n_kv > 0 && cap > 0, "%s: bad shape (b %lld, n_kv %lld, cap %lld)", name, (long long)b,
                 (long long)n_kv, (long long)cap);
    DTTS_REQUIRE(head_dim == 64 || head_dim == 128, "%s: head_dim %lld (64 or 128 supported)", name,
                 (long long)head_dim);
    DTTS_REQUIRE(gqa == 1 || gqa == 2 || gqa == 4 || gqa == 8, "%s: gqa %lld (1, 2, 4 or 8 supported)", name,
                 (long long)gqa);
    DTTS_REQUIRE(b <= kAttnMaxLanes, "%s: %lld lanes > %d", name, (long long)b, kAttnMaxLanes);
    if (b == 0) return DTTS_OK;
    DTTS_REQUIRE(q && kc && vc && out && span, "%s: null pointer", name);
    DTTS_REQUIRE(b * n_kv < (int64_t(1) << 31) && b * n_kv * cap * head_dim < (int64_t(1) << 40), "%s: shape too large",
                 name);
    DTTS_REQUIRE(aligned(q, 16) && aligned(kc, 16) && aligned(vc, 16) && aligned(out, 4), "%s: misaligned operand",
                 name);
    HostSpans sp{};
    int64_t max_window = 0;
    for (int64_t i = 0; i < b; ++i) {
        const int32_t lo = window_start ? window_start[i] : 0;
        DTTS_REQUIRE(span[i] <= cap, "%s: lane %lld span %d exceeds capacity %lld", name, (long long)i, span[i],
                     (long long)cap);
        DTTS_REQUIRE(lo >= 0 && lo < span[i], "%s: lane %lld attends to the empty range [%d, %d)", name,
                     (long long)i, lo, span[i]);
        sp.sp.lo[i] = lo;
        sp.sp.hi[i] = span[i];
        max_window = span[i] - lo > max_window ? span[i] - lo : max_window;
    }
    // split the spans when a workspace holds every chunk's state (and there is more than one)
    const size_t need = attn_workspace_bytes(b, n_kv, gqa, head_dim, max_window);
    float *part = nullptr;
    int max_chunks = 0;
    if (need > 0 && workspace && ws_bytes >= need) {
        DTTS_REQUIRE(aligned(workspace, 16), "%s: misaligned workspace", name);
        part = static_cast<float *>(workspace);
        max_chunks = static_cast<int>((max_window + kChunk - 1) / kChunk);
    }
    const hipError_t e = launch_attention(q, kc, vc, out, part, max_chunks, b, n_kv, gqa, head_dim, cap, sp, stream);
    DTTS_HIP_CHECK(e, name);
    return DTTS_OK;
}

}  // namespace
}  // namespace dtts

extern "C" size_t dtts_decode_attention_workspace_bytes(int64_t b, int64_t n_kv, int64_t gqa, int64_t head_dim,
                                                         int64_t max_window) {
    return dtts::attn_workspace_bytes(b, n_kv, gqa, head_dim, max_window);
}

extern "C" int dtts_decode_attention_f16(const float *q, const dtts_f16 *kcache, const dtts_f16 *vcache, float *out,
                                         int64_t b, int64_t n_kv, int64_t gqa, int64_t head_dim, int64_t cap,
                                         const int32_t *span, const int32_t *window_start, void *workspace,
                                         size_t ws_bytes, hipStream_t stream) {
    return dtts::decode_attention("dtts_decode_attention_f16", q, reinterpret_cast<const dtts::half_t *>(kcache),
                                  reinterpret_cast<const dtts::half_t *>(vcache), out, b, n_kv, gqa, head_dim, cap, span,
                                  window_start, workspace, ws_bytes, stream);
}

extern "C" int dtts_decode_attention_f32(const float *q, const float *kcache, const float *vcache, float *out,
                                         int64_t b, int64_t n_kv, int64_t gqa, int64_t head_dim, int64_t cap,
                                         const int32_t *span, const int32_t *window_start, void *workspace,
                                         size_t ws_bytes, hipStream_t stream) {
    return dtts::decode_attention("dtts_decode_attention_f32", q, kcache, vcache, out, b, n_kv, gqa, head_dim, cap,
                                  span, window_start, workspace, ws_bytes, stream);
}
