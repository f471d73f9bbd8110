// RMSNorm and the fused QK-norm + RoPE + KV-cache append kernels, shared by the per-op entry
// points and the decoder-stack step.
//
// These are latency-bound at decode shapes (48 lanes): one wave per row (or per (lane, head)),
// a wave-wide shuffle reduction, and no LDS. Per-lane positions come from the host (checked
// against the cache capacity before anything is enqueued, and carried in the kernel arguments)
// or, for the stack step, from a device array the host fills after the same checks, so that a
// captured graph stays valid from step to step.
//
// Rounding: floating-point contraction is off in these kernels, so o = x1*c - x2*s rounds each
// product before the subtraction, as the reference's CPU path does (hipcc would otherwise fuse
// them into an FMA). f32 -> f16 stores round to nearest-even.
#pragma once

#include <cmath>

#include "common.hpp"

namespace dtts {
namespace {

constexpr int kMaxLanes = 256;

struct Positions {  // in the kernel arguments
    int32_t p[kMaxLanes];
    __device__ __forceinline__ int at(int i) const { return p[i]; }
};

struct DevPositions {  // in device memory
    const int32_t *p;
    __device__ __forceinline__ int at(int i) const { return p[i]; }
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ---------------------------------------------------------------- RMSNorm

// One wave per row; lane j owns elements j, j+64, ... TO: the output type; an f32 input with an
// f16 output rounds the f32 result once (the consumer's cast, Proj::forward's x.to_dtype(F16)).

template <typename T, typename TO = T>
__global__ __launch_bounds__(256) void rms_norm_kernel(const T *x, const T *gamma, TO *y, int rows, int dim, float eps) {
#pragma clang fp contract(off)
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const T *xr = x + static_cast<int64_t>(row) * dim;
    TO *yr = y + static_cast<int64_t>(row) * dim;
    float ss = 0.0f;
    for (int i = lane; i < dim; i += 64) {
        const float v = static_cast<float>(xr[i]);
        ss += v * v;
    }
    ss = wave_sum(ss);
    const float m = sqrtf(ss / static_cast<float>(dim) + eps);
    if constexpr (sizeof(T) == 2) {
        // candle's f16 form: m rounded to f16, then (x / m) and (* gamma) each rounded to f16
        const float mh = static_cast<float>(static_cast<half_t>(m));
        for (int i = lane; i < dim; i += 64) {
            const float q = static_cast<float>(static_cast<half_t>(static_cast<float>(xr[i]) / mh));
            yr[i] = static_cast<half_t>(q * static_cast<float>(gamma[i]));
        }
    } else {
        for (int i = lane; i < dim; i += 64) yr[i] = static_cast<TO>((xr[i] / m) * gamma[i]);
    }
}

// The same arithmetic with 16-byte accesses, for rows of a multiple of 64 vectors: lane j owns
// vectors j, j + 64, ... (each 8 f16 or 4 f32), at most NV of them, all loaded before the first
// use, with gamma's loaded beside them. The row stays in registers between the two passes.
template <typename T, int NV>
__global__ __launch_bounds__(256) void rms_norm_vec_kernel(const T *x, const T *gamma, T *y, int rows, int dim,
                                                           float eps) {
#pragma clang fp contract(off)
    constexpr int E = 16 / sizeof(T);  // elements per vector
    typedef T vec_t __attribute__((ext_vector_type(E)));
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int nv = dim / (64 * E);
    const vec_t *xr = reinterpret_cast<const vec_t *>(x + static_cast<int64_t>(row) * dim);
    const vec_t *gr = reinterpret_cast<const vec_t *>(gamma);
    vec_t *yr = reinterpret_cast<vec_t *>(y + static_cast<int64_t>(row) * dim);
    vec_t v[NV], g[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i)
        if (i < nv) {
            v[i] = xr[i * 64 + lane];
            g[i] = gr[i * 64 + lane];
        }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        if (i < nv)
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float f = static_cast<float>(v[i][e]);
                ss += f * f;
            }
    ss = wave_sum(ss);
    const float m = sqrtf(ss / static_cast<float>(dim) + eps);
    const float mh = static_cast<float>(static_cast<half_t>(m));
#pragma unroll
    for (int i = 0; i < NV; ++i)
        if (i < nv) {
            vec_t o;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if constexpr (sizeof(T) == 2) {  // candle's f16 form, as rms_norm_kernel
                    const float q = static_cast<float>(static_cast<half_t>(static_cast<float>(v[i][e]) / mh));
                    o[e] = static_cast<half_t>(q * static_cast<float>(g[i][e]));
                } else {
                    o[e] = (v[i][e] / m) * g[i][e];
                }
            }
            yr[i * 64 + lane] = o;
        }
}

// ---------------------------------------------------------------- RoPE

__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s, float &o1, float &o2) {
#pragma clang fp contract(off)
    const float a = x1 * c, b = x2 * s, e = x2 * c, f = x1 * s;
    o1 = a - b;
    o2 = e + f;
}

// ---------------------------------------------------------------- QK-norm + RoPE + append

// One wave per (lane b, head h) with h < heads (query) or heads <= h < heads + n_kv (key; the
// wave also writes v). Lane j holds dims j and j + 64 when D = 128 (any even D <= 128: lane j
// holds pair j < D/2). norms == nullptr skips the QK-norm (layers without it); q_scale then
// multiplies the roped q (Stack::forward's q * 1/sqrt(D) for such layers, crates/qwen3tts/src/
// qwen3.rs:404-408), and is 1 otherwise. P: Positions or DevPositions. ys > 1: qkv is the sum,
// in order, of ys partial arrays ystride elements apart (a projection's k-split partials);
// round16 rounds that sum to f16 first. CT: the caches' element type (f16, or f32 as Stack::load
// keeps them for f32 and quantized weights, crates/qwen3tts/src/qwen3.rs:242-246).
template <typename T, typename P, typename CT = half_t>
__global__ __launch_bounds__(256) void qk_rope_kernel(const T *qkv, const float *norms, const float *cos_t,
                                                      const float *sin_t, P pos, T *q_out, float *k_out,
                                                      CT *kc, CT *vc, int b, int heads, int n_kv, int hd,
                                                      int cap, float eps, float q_scale, int ys, int64_t ystride,
                                                      bool round16) {
#pragma clang fp contract(off)
    const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int per = heads + n_kv;
    if (wid >= b * per) return;
    const int bi = wid / per;
    const int h = wid - bi * per;
    const int half = hd / 2;
    const int width = (heads + 2 * n_kv) * hd;
    const T *row = qkv + static_cast<int64_t>(bi) * width;
    const T *src = row + h * hd;
    const bool is_q = h < heads;
    const bool act = lane < half;
    auto ld = [&](const T *q) {  // the first 8 partials requested together, summed in order
        float w[8];
#pragma unroll
        for (int y = 0; y < 8; ++y)
            if (y < ys) w[y] = static_cast<float>(q[y * ystride]);
        float v = w[0];
#pragma unroll
        for (int y = 1; y < 8; ++y)
            if (y < ys) v += w[y];
        for (int y = 8; y < ys; ++y) v += static_cast<float>(q[y * ystride]);
        // round16: the projection's output as candle's f16 matmul gives it (one rounding of the sum)
        return round16 ? static_cast<float>(static_cast<half_t>(v)) : v;
    };
    float x1 = 0.0f, x2 = 0.0f;
    if (act) {
        x1 = ld(src + lane);
        x2 = ld(src + lane + half);
    }
    float ss = wave_sum(x1 * x1 + x2 * x2);
    const float m = sqrtf(ss / static_cast<float>(hd) + eps);
    if (!act) return;
    float y1 = x1, y2 = x2;
    if (norms) {  // candle's rms_norm: (x / m) * w
        const float *w = norms + (is_q ? 0 : hd);
        y1 = (x1 / m) * w[lane];
        y2 = (x2 / m) * w[lane + half];
    }
    const int p = pos.at(bi);
    const float c = cos_t[static_cast<int64_t>(p) * half + lane];
    const float s = sin_t[static_cast<int64_t>(p) * half + lane];
    float o1, o2;
    rope_pair(y1, y2, c, s, o1, o2);
    if (is_q) {
        T *dq = q_out + (static_cast<int64_t>(bi) * heads + h) * hd;
        if (q_scale != 1.0f) {
            o1 = o1 * q_scale;
            o2 = o2 * q_scale;
        }
        dq[lane] = static_cast<T>(o1);
        dq[lane + half] = static_cast<T>(o2);
        return;
    }
    const int kh = h - heads;
    const int64_t dst = ((static_cast<int64_t>(bi) * n_kv + kh) * cap + p) * hd;
    kc[dst + lane] = static_cast<CT>(o1);
    kc[dst + lane + half] = static_cast<CT>(o2);
    const T *vs = row + (heads + n_kv + kh) * hd;
    vc[dst + lane] = static_cast<CT>(ld(vs + lane));
    vc[dst + lane + half] = static_cast<CT>(ld(vs + lane + half));
    if (k_out) {
        float *fk = k_out + (static_cast<int64_t>(bi) * n_kv + kh) * hd;
        fk[lane] = o1;
        fk[lane + half] = o2;
    }
}

// QK-norm (when norms is set), RoPE at start + ti and the cache write of t new positions per lane,
// with the reference's optional f32 side outputs (qkrope::apply with f32_kv, qkrope.rs:26-69):
// one wave per (row, head), row = bi * t + ti, the lane holding pair (lane, lane + D/2) as the
// decode kernel does. qkv [rows, (heads + 2 n_kv) D] of T (f32: the sum of ys partials ystride
// apart, a projection's k-split; f16: the f16 matmul's output). Out: q [b, heads, t, D]; kf and
// vf [b, n_kv, t, D] f32 (both or neither); kc, vc [b, n_kv, cap, D] at start .. start + t - 1.
template <typename T>
__global__ __launch_bounds__(256) void qk_rope_span_kernel(const T *qkv, const float *norms, const float *cos_t,
                                                           const float *sin_t, float *q_out, float *kf, float *vf,
                                                           half_t *kc, half_t *vc, int rows, int t, int start, int heads,
                                                           int n_kv, int hd, int cap, float eps, int ys, int64_t ystride,
                                                           bool round16) {
#pragma clang fp contract(off)
    const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int per = heads + n_kv;
    if (wid >= rows * per) return;
    const int row = wid / per;
    const int h = wid - row * per;
    const int bi = row / t, ti = row - (row / t) * t, p = start + ti;
    const int half = hd / 2;
    const T *src_row = qkv + static_cast<int64_t>(row) * (heads + 2 * n_kv) * hd;
    const bool is_q = h < heads;
    const bool act = lane < half;
    auto ld = [&](const T *q) {
        // the first eight ranges' partials requested together, summed in range order
        float w[8];
#pragma unroll
        for (int y = 0; y < 8; ++y)
            if (y < ys) w[y] = static_cast<float>(q[y * ystride]);
        float v = w[0];
#pragma unroll
        for (int y = 1; y < 8; ++y)
            if (y < ys) v += w[y];
        for (int y = 8; y < ys; ++y) v += static_cast<float>(q[y * ystride]);
        return round16 ? static_cast<float>(static_cast<half_t>(v)) : v;
    };
    float x1 = 0.0f, x2 = 0.0f;
    if (act) {
        x1 = ld(src_row + h * hd + lane);
        x2 = ld(src_row + h * hd + lane + half);
    }
    const float ss = wave_sum(x1 * x1 + x2 * x2);
    const float m = sqrtf(ss / static_cast<float>(hd) + eps);
    if (!act) return;
    float y1 = x1, y2 = x2;
    if (norms) {
        const float *w = norms + (is_q ? 0 : hd);
        y1 = (x1 / m) * w[lane];
        y2 = (x2 / m) * w[lane + half];
    }
    const float c = cos_t[static_cast<int64_t>(p) * half + lane];
    const float s = sin_t[static_cast<int64_t>(p) * half + lane];
    float o1, o2;
    rope_pair(y1, y2, c, s, o1, o2);
    if (is_q) {
        float *dq = q_out + ((static_cast<int64_t>(bi) * heads + h) * t + ti) * hd;
        dq[lane] = o1;
        dq[lane + half] = o2;
        return;
    }
    const int kh = h - heads;
    const int64_t dst = ((static_cast<int64_t>(bi) * n_kv + kh) * cap + p) * hd;
    const int64_t fdst = ((static_cast<int64_t>(bi) * n_kv + kh) * t + ti) * hd;
    const T *vs = src_row + (heads + n_kv + kh) * hd;
    const float v1 = ld(vs + lane), v2 = ld(vs + lane + half);
    kc[dst + lane] = static_cast<half_t>(o1);
    kc[dst + lane + half] = static_cast<half_t>(o2);
    vc[dst + lane] = static_cast<half_t>(v1);
    vc[dst + lane + half] = static_cast<half_t>(v2);
    if (kf) {
        kf[fdst + lane] = o1;
        kf[fdst + lane + half] = o2;
        vf[fdst + lane] = v1;
        vf[fdst + lane + half] = v2;
    }
}

}  // namespace
}  // namespace dtts
