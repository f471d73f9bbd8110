// Decode attention over the KV cache in place (attn::decode_attention,
// crates/tts-nn/src/attn.rs:18-73; the CPU path it is held to is Scores, softmax_last_dim and
// Weighted, attn.rs:85-126, 62, 189-226).
//
//   q     [b, n_kv, gqa, D] f32, any scale already folded in
//   cache [b, n_kv, cap, D] f16 or f32 (k and v)
//   out   [b, n_kv, gqa, D] f32
//   lane i attends to positions [window_start[i], span[i]); the reference's single span and
//   window start are the case where every lane has the same ones
//
// One workgroup per (lane, kv head): the cache rows of the span are read once, for all gqa query
// heads that share them. The span is split over groups of 16 lanes (4 per wave), each group
// taking every G-th position; a lane of a group owns D/16 dimensions: the score is a 16-lane
// shuffle reduction, and each group keeps a running softmax state (max m, sum l, weighted sum of
// v) updated position by position, or for f16 caches four positions at a time (online softmax).
// The groups' states are combined through LDS at the end: out = sum_k acc_k e^(m_k - M) /
// sum_k l_k e^(m_k - M), M the largest m_k (exponentials taken in base 2, below). This is the
// reference's exp(s - max) / sum weighting, regrouped; its K and V traffic is one pass.
// HBM-bound: 2 * D * (span - window_start) cache bytes per (lane, kv head).
//
// Long spans are split (flash-decoding): with a workspace, each workgroup takes kChunk positions
// of one (lane, kv head) and leaves its combined state (its max, its sum, its weighted v sum) in
// the workspace, and a second kernel merges a lane's chunks the same way. Without one, a
// workgroup takes the whole span.
#pragma once

#include <cmath>

#include "common.hpp"

namespace dtts {
namespace {

constexpr int kAttnMaxLanes = 256;

struct Spans {
    int32_t lo[kAttnMaxLanes];  // window start
    int32_t hi[kAttnMaxLanes];  // span (exclusive end)
};

// Where a lane's window [lo, hi) comes from: the kernel arguments (checked host arrays), or the
// device-resident position of the token being decoded (hi = pos + 1, the last `window`
// positions of it when a sliding window is set: Stack::forward's wstart, crates/qwen3tts/src/
// qwen3.rs:409-412), which keeps a captured graph valid from step to step.
struct HostSpans {
    Spans sp;
    __device__ __forceinline__ void get(int lane, int &lo, int &hi) const {
        lo = sp.lo[lane];
        hi = sp.hi[lane];
    }
};

struct DevSpans {
    const int32_t *pos;
    int window;  // 0: no window
    __device__ __forceinline__ void get(int lane, int &lo, int &hi) const {
        hi = pos[lane] + 1;
        lo = window > 0 && hi > window ? hi - window : 0;
    }
};

__device__ __forceinline__ void store_out(float *o, float v) { *o = v; }
__device__ __forceinline__ void store_out(half_t *o, float v) { *o = static_cast<half_t>(v); }

template <typename T>
struct CacheRow;  // D/16 consecutive elements of one cache row, as f32

template <>
struct CacheRow<half_t> {
    template <int E>
    __device__ __forceinline__ static void load(const half_t *p, float (&out)[E]) {
        static_assert(E == 8 || E == 4, "row slice");
        if constexpr (E == 8) {
            const half8_t v = *reinterpret_cast<const half8_t *>(p);
#pragma unroll
            for (int e = 0; e < 8; ++e) out[e] = static_cast<float>(v[e]);
        } else {
            const half4_t v = *reinterpret_cast<const half4_t *>(p);
#pragma unroll
            for (int e = 0; e < 4; ++e) out[e] = static_cast<float>(v[e]);
        }
    }
};

template <>
struct CacheRow<float> {
    template <int E>
    __device__ __forceinline__ static void load(const float *p, float (&out)[E]) {
#pragma unroll
        for (int e = 0; e < E; e += 4) {
            const float4_t v = *reinterpret_cast<const float4_t *>(p + e);
            out[e] = v[0];
            out[e + 1] = v[1];
            out[e + 2] = v[2];
            out[e + 3] = v[3];
        }
    }
};

__device__ __forceinline__ float group16_sum(float v) {
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// The softmax runs in base 2: q is scaled by log2(e) as it is loaded, so scores, running maxima
// and the chunk states' m are log2 of the natural-base ones and every weight is one v_exp_f32
// (2^x; the library expf adds a range reduction and overflow checks, ~12 instructions). A weight
// 2^x with x below -126 is under 1e-38 of the running maximum's, whatever the unit rounds it to.
constexpr float kLog2e = 1.44269504088896340736f;
__device__ __forceinline__ float softmax_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr int kChunk = 512;  // positions per workgroup when a span is split

// Chunks of a lane's window [lo, hi) when split.
__device__ __host__ inline int chunks_of(int lo, int hi) { return (hi - lo + kChunk - 1) / kChunk; }

// T: cache element type; D: head dim (64 or 128); GQA: query heads per kv head; NW: waves;
// Src: HostSpans or DevSpans; OutT: float, or half_t for a consumer that casts the result.
// part == nullptr: blockIdx.y is 0 and the workgroup writes out. Otherwise blockIdx.y is a chunk
// of kChunk positions, and the workgroup writes its state to part (rows of D + 2 floats: the
// weighted v sum, the weight sum, the max score) at [(bh * max_chunks + chunk) * GQA + g].
template <typename T, int D, int GQA, int NW, typename Src, typename OutT>
__global__ __launch_bounds__(NW * 64) void decode_attn_kernel(const float *q, const T *kc, const T *vc, OutT *out,
                                                              float *part, int max_chunks, int n_kv, int cap,
                                                              Src sp) {
    constexpr int E = D / 16;     // dimensions per lane
    constexpr int G = NW * 4;     // position groups
    constexpr int UNROLL = 4;     // positions whose rows are in flight per group
    __shared__ float sm_m[G][GQA], sm_l[G][GQA];
    __shared__ __attribute__((aligned(16))) float sm_acc[G][GQA][D];
    const int bh = blockIdx.x;  // lane * n_kv + kv head
    const int lane_idx = bh / n_kv;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int grp = wave * 4 + ((tid & 63) >> 4);
    const int j = tid & 15;
    int lo, hi;
    sp.get(lane_idx, lo, hi);
    if (part) {
        if (static_cast<int>(blockIdx.y) >= chunks_of(lo, hi)) return;  // the whole workgroup
        lo += blockIdx.y * kChunk;
        hi = hi < lo + kChunk ? hi : lo + kChunk;
    }

    float qv[GQA][E];
#pragma unroll
    for (int g = 0; g < GQA; ++g) {
        const float *qp = q + (static_cast<int64_t>(bh) * GQA + g) * D + j * E;
#pragma unroll
        for (int e = 0; e < E; ++e) qv[g][e] = qp[e] * kLog2e;
    }
    float m[GQA], l[GQA], acc[GQA][E];
#pragma unroll
    for (int g = 0; g < GQA; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[g][e] = 0.0f;
    }
    const T *kb = kc + static_cast<int64_t>(bh) * cap * D + j * E;
    const T *vb = vc + static_cast<int64_t>(bh) * cap * D + j * E;
    auto step = [&](const float (&kr)[E], const float (&vr)[E]) {
#pragma unroll
        for (int g = 0; g < GQA; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) s += qv[g][e] * kr[e];
            s = group16_sum(s);
            const float mn = fmaxf(m[g], s);
            const float c = softmax_exp2(m[g] - mn);  // 0 on the group's first position
            const float w = softmax_exp2(s - mn);
            l[g] = l[g] * c + w;
#pragma unroll
            for (int e = 0; e < E; ++e) acc[g][e] = acc[g][e] * c + w * vr[e];
            m[g] = mn;
        }
    };
    // UNROLL positions of the group at a time: their K and V rows are all requested before the
    // first is used (the group's 16 lanes read 16 * E contiguous elements per row). With f16
    // caches the online-softmax state moves once per UNROLL positions: one running maximum over
    // the block, one rescale of l and acc (one exponential for it), then the block's weighted rows
    // in order (decode attention 41.6 -> 39-40 us, the f16 talker step -2%). With f32 caches the
    // per-position update stays: held to four workgroups per CU (below), the block form measured
    // within +-2% there.
    auto step_block = [&](const float (&kr)[UNROLL][E], const float (&vr)[UNROLL][E]) {
#pragma unroll
        for (int g = 0; g < GQA; ++g) {
            float s[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < E; ++e) d += qv[g][e] * kr[u][e];
                s[u] = group16_sum(d);
            }
            float mn = m[g];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) mn = fmaxf(mn, s[u]);
            const float c = softmax_exp2(m[g] - mn);  // 0 on the group's first block
            float w[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) w[u] = softmax_exp2(s[u] - mn);
            float lv = l[g] * c;
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) lv += w[u];
            l[g] = lv;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                float a = acc[g][e] * c;
#pragma unroll
                for (int u = 0; u < UNROLL; ++u) a += w[u] * vr[u][e];
                acc[g][e] = a;
            }
            m[g] = mn;
        }
    };
    int p = lo + grp;
    for (; p + (UNROLL - 1) * G < hi; p += UNROLL * G) {
        float kr[UNROLL][E], vr[UNROLL][E];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            CacheRow<T>::load(kb + static_cast<int64_t>(p + u * G) * D, kr[u]);
            CacheRow<T>::load(vb + static_cast<int64_t>(p + u * G) * D, vr[u]);
        }
        if constexpr (sizeof(T) == 2) {
            step_block(kr, vr);
        } else {
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) step(kr[u], vr[u]);
        }
    }
    for (; p < hi; p += G) {
        float kr[E], vr[E];
        CacheRow<T>::load(kb + static_cast<int64_t>(p) * D, kr);
        CacheRow<T>::load(vb + static_cast<int64_t>(p) * D, vr);
        step(kr, vr);
    }

    // combine the groups' states
#pragma unroll
    for (int g = 0; g < GQA; ++g) {
#pragma unroll
        for (int e = 0; e < E; e += 4)
            *reinterpret_cast<float4_t *>(&sm_acc[grp][g][j * E + e]) =
                float4_t{acc[g][e], acc[g][e + 1], acc[g][e + 2], acc[g][e + 3]};
        if (j == 0) {
            sm_m[grp][g] = m[g];
            sm_l[grp][g] = l[g];
        }
    }
    __syncthreads();
    for (int t = tid; t < GQA * D; t += NW * 64) {
        const int g = t / D, d = t - (t / D) * D;
        float mx = -INFINITY;
#pragma unroll 4
        for (int k = 0; k < G; ++k) mx = fmaxf(mx, sm_m[k][g]);
        float den = 0.0f, num = 0.0f;
#pragma unroll 4
        for (int k = 0; k < G; ++k) {
            const float f = softmax_exp2(sm_m[k][g] - mx);  // 0 for groups that saw no position
            den += sm_l[k][g] * f;
            num += sm_acc[k][g][d] * f;
        }
        if (part) {
            float *pr = part + ((static_cast<int64_t>(bh) * max_chunks + blockIdx.y) * GQA + g) * (D + 2);
            pr[d] = num;
            if (d == 0) {
                pr[D] = den;
                pr[D + 1] = mx;
            }
        } else {
            store_out(out + (static_cast<int64_t>(bh) * GQA + g) * D + d, num / den);
        }
    }
}

// Merges the chunk states of each (lane, kv head): out = sum_c num_c e^(m_c - M) / sum_c den_c
// e^(m_c - M), M the largest m_c, chunks in order (m in log2 units, so 2^(m_c - M)).
template <int D, int GQA, typename Src, typename OutT>
__global__ __launch_bounds__(256) void decode_attn_merge(const float *part, OutT *out, int max_chunks, int n_kv,
                                                         Src sp) {
    const int bh = blockIdx.x;
    const int lane_idx = bh / n_kv;
    int lo, hi;
    sp.get(lane_idx, lo, hi);
    const int nch = chunks_of(lo, hi);
    constexpr int U = 8;  // chunk states requested together (a loop would wait for each in turn)
    for (int t = threadIdx.x; t < GQA * D; t += 256) {
        const int g = t / D, d = t - (t / D) * D;
        const float *pr = part + (static_cast<int64_t>(bh) * max_chunks * GQA + g) * (D + 2);
        const int64_t stride = static_cast<int64_t>(GQA) * (D + 2);
        float num = 0.0f, den = 0.0f;
        if (nch <= U) {
            float mc[U], nc[U], dc[U];
#pragma unroll
            for (int c = 0; c < U; ++c)
                if (c < nch) {
                    mc[c] = pr[c * stride + D + 1];
                    nc[c] = pr[c * stride + d];
                    dc[c] = pr[c * stride + D];
                }
            float mx = -INFINITY;
#pragma unroll
            for (int c = 0; c < U; ++c)
                if (c < nch) mx = fmaxf(mx, mc[c]);
#pragma unroll
            for (int c = 0; c < U; ++c)
                if (c < nch) {
                    const float f = softmax_exp2(mc[c] - mx);
                    num += nc[c] * f;
                    den += dc[c] * f;
                }
        } else {
            float mx = -INFINITY;
            for (int c = 0; c < nch; ++c) mx = fmaxf(mx, pr[c * stride + D + 1]);
            for (int c = 0; c < nch; ++c) {
                const float f = softmax_exp2(pr[c * stride + D + 1] - mx);
                num += pr[c * stride + d] * f;
                den += pr[c * stride + D] * f;
            }
        }
        store_out(out + (static_cast<int64_t>(bh) * GQA + g) * D + d, num / den);
    }
}

// Unused dynamic LDS that holds decode attention to at most 5 workgroups per CU (f16 caches) or
// 4 (f32 caches), one wave per SIMD each: the kernel's registers would let 6 and 5 run, and more
// rows in flight than that measured slower (f32 caches: the F32 and Q8_0 talker steps 5.44 ->
// 5.85 ms at 5; f16 caches: attention 35.5 against 36.0 us at 6). 160 KB of LDS per CU.
template <typename T, int D, int GQA>
constexpr size_t attn_lds_pad() {
    constexpr size_t wg = sizeof(T) == 4 ? 4 : 5;
    constexpr size_t stat = sizeof(float) * (2 * 16 * GQA + 16 * GQA * D);  // the kernel's own LDS
    return stat < 160 * 1024 / wg ? (160 * 1024 / wg - stat) / 512 * 512 : 0;
}

template <typename T, int D, int GQA, typename Src, typename OutT>
hipError_t launch_gqa(const float *q, const T *kc, const T *vc, OutT *out, float *part, int max_chunks, int64_t b,
                      int64_t n_kv, int64_t cap, const Src &sp, hipStream_t stream) {
    const unsigned grid = static_cast<unsigned>(b * n_kv);
    constexpr size_t pad = attn_lds_pad<T, D, GQA>();
    if (!part) {
        decode_attn_kernel<T, D, GQA, 4, Src, OutT><<<grid, 256, pad, stream>>>(
            q, kc, vc, out, nullptr, 0, static_cast<int>(n_kv), static_cast<int>(cap), sp);
        return hipGetLastError();
    }
    decode_attn_kernel<T, D, GQA, 4, Src, OutT><<<dim3(grid, max_chunks), 256, pad, stream>>>(
        q, kc, vc, out, part, max_chunks, static_cast<int>(n_kv), static_cast<int>(cap), sp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    decode_attn_merge<D, GQA, Src, OutT><<<grid, 256, 0, stream>>>(part, out, max_chunks, static_cast<int>(n_kv), sp);
    return hipGetLastError();
}

// gqa in {1, 2, 4, 8} and D in {64, 128}, checked by the caller.
template <typename T, typename Src, typename OutT>
hipError_t launch_attention(const float *q, const T *kc, const T *vc, OutT *out, float *part, int max_chunks,
                            int64_t b, int64_t n_kv, int64_t gqa, int64_t head_dim, int64_t cap, const Src &sp,
                            hipStream_t stream) {
    if (head_dim == 128) {
        switch (gqa) {
            case 1: return launch_gqa<T, 128, 1>(q, kc, vc, out, part, max_chunks, b, n_kv, cap, sp, stream);
            case 2: return launch_gqa<T, 128, 2>(q, kc, vc, out, part, max_chunks, b, n_kv, cap, sp, stream);
            case 4: return launch_gqa<T, 128, 4>(q, kc, vc, out, part, max_chunks, b, n_kv, cap, sp, stream);
            default: return launch_gqa<T, 128, 8>(q, kc, vc, out, part, max_chunks, b, n_kv, cap, sp, stream);
        }
    }
    switch (gqa) {
        case 1: return launch_gqa<T, 64, 1>(q, kc, vc, out, part, max_chunks, b, n_kv, cap, sp, stream);
        case 2: return launch_gqa<T, 64, 2>(q, kc, vc, out, part, max_chunks, b, n_kv, cap, sp, stream);
        case 4: return launch_gqa<T, 64, 4>(q, kc, vc, out, part, max_chunks, b, n_kv, cap, sp, stream);
        default: return launch_gqa<T, 64, 8>(q, kc, vc, out, part, max_chunks, b, n_kv, cap, sp, stream);
    }
}

// Workspace bytes for splitting windows of up to max_window positions (0 when one chunk holds
// them).
inline size_t attn_workspace_bytes(int64_t b, int64_t n_kv, int64_t gqa, int64_t head_dim, int64_t max_window) {
    if (b <= 0 || n_kv <= 0 || gqa <= 0 || head_dim <= 0 || max_window <= kChunk) return 0;
    const int64_t chunks = (max_window + kChunk - 1) / kChunk;
    return static_cast<size_t>(b * n_kv * chunks * gqa * (head_dim + 2)) * sizeof(float);
}

}  // namespace
}  // namespace dtts
