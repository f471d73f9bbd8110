// SnakeBeta arithmetic shared by the standalone snake kernels and the conv prologues.
#pragma once

#include "common.hpp"

namespace dtts {

constexpr float kInv2Pi = 0.159154943091895335768883763372514362f;

// sin(2 pi t) through the hardware sine. v_sin_f32 takes its argument in revolutions; taking
// the fractional part first keeps it in [0, 1), where the unit is accurate. Absolute error stays
// near 1e-6 for |2 pi t| up to ~100 (the f32 rounding of t dominates), far inside an f16 ulp, so
// it is used wherever the snake's result is stored as f16.
__device__ __forceinline__ float sin_rev_f16out(float t) { return __builtin_amdgcn_sinf(__builtin_amdgcn_fractf(t)); }

// sin^2(a x) for f32 a and x, within 1.5e-7 of the exact value for |a x| <= 2^20 (measured
// against f64 over 1.2e8 random points). The product a x is carried exactly as the
// pair th + tl (the fma gives the rounding error of th). Cody and Waite's additive reduction
// takes off the nearest multiple k of pi/2, held as three f32 parts P1 + P2 + P3 (P1 = f32(pi/2),
// each next part the f32 rounding of what is left; their sum is pi/2 to 1.1e-23): th - k P1 is
// exact in the fma, the later parts and tl are small. sin r on |r| <= pi/4 is its Taylor series
// through r^9 (truncation under 2e-9), and sin^2(r + k pi/2) is sin^2 r for even k and
// 1 - sin^2 r for odd k, so no cosine is needed. Larger and non-finite arguments take the library
// sinf of the rounded product. The library sinf of the rounded product everywhere loses up to
// 1e-6 to that rounding alone at |a x| ~ 30 (where the codec's convs drive SnakeBeta).
__device__ __forceinline__ bool sin2_f32_reducible(float a, float x) { return __builtin_fabsf(a * x) <= 0x1p20f; }

// The reduction and series alone, for arguments sin2_f32_reducible accepts.
__device__ __forceinline__ float sin2_f32_reduced(float a, float x) {
    const float th = a * x;
    const float tl = __builtin_fmaf(a, x, -th);
    const float k = __builtin_rintf(th * 0x1.45f306p-1f);   // 2/pi
    float r = __builtin_fmaf(-k, 0x1.921fb6p+0f, th);       // P1
    r = __builtin_fmaf(-k, -0x1.777a5cp-25f, r);            // P2
    r = __builtin_fmaf(-k, -0x1.ee59dap-50f, r + tl);       // P3
    const float r2 = r * r;
    float p = __builtin_fmaf(r2, 0x1.71de3ap-19f, -0x1.a01a02p-13f);  // 1/9!, -1/7!
    p = __builtin_fmaf(r2, p, 0x1.111112p-7f);                       // 1/5!
    p = __builtin_fmaf(r2, p, -0x1.555556p-3f);                      // -1/3!
    const float s = __builtin_fmaf(r * r2, p, r);
    const float s2 = s * s;
    return (static_cast<int>(k) & 1) ? 1.0f - s2 : s2;
}

__device__ __forceinline__ float sin2_f32(float a, float x) {
    if (!sin2_f32_reducible(a, x)) {
        const float s = sinf(a * x);
        return s * s;
    }
    return sin2_f32_reduced(a, x);
}

// SnakeBeta over N values (parameters per value): the reduced form for all of them as straight-line
// code, then one branch for the group, taken only when an argument is past the reduction's range.
// A branch per value (as sin2_f32 has) serialises the values and costs more than their arithmetic.
template <int N>
__device__ __forceinline__ void snake_f32_group(float (&v)[N], const float (&a)[N], const float (&r)[N]) {
    float s2[N];
    bool far = false;
#pragma unroll
    for (int q = 0; q < N; ++q) {
        s2[q] = sin2_f32_reduced(a[q], v[q]);
        far |= !sin2_f32_reducible(a[q], v[q]);
    }
    if (far) {
#pragma unroll
        for (int q = 0; q < N; ++q) s2[q] = sin2_f32(a[q], v[q]);
    }
#pragma unroll
    for (int q = 0; q < N; ++q) v[q] = v[q] + r[q] * s2[q];
}

// y = x + r * sin^2(a x). f32 outputs are held to the reference's 1e-6-of-scale accuracy bound
// (crates/tts-nn/src/fused.rs:2356-2391).
__device__ __forceinline__ float snake_f32(float x, float a, float r) { return x + r * sin2_f32(a, x); }

// The f16-storage snake with ka = a / (2 pi) precomputed per channel: x * ka, fract, sin, s*s
// and one fma (which reads x as f16 directly: v_fma_mix_f32) per element.
__device__ __forceinline__ half_t snake_f16k(half_t x, float ka, float r) {
    const float xf = static_cast<float>(x);
    const float s = sin_rev_f16out(xf * ka);
    return static_cast<half_t>(__builtin_fmaf(r, s * s, xf));
}

// The same value from a and an f32 x that holds an f16 (every caller rounds x to f16 first). Fused
// and standalone snakes compute the same formula; where the compiler rounds the final fma to f16
// directly (one rounding) in one kernel and through f32 (two) in another, results within a
// hair of an f16 rounding midpoint differ by one ulp (a few elements per million, measured).
__device__ __forceinline__ float snake_f16out(float x, float a, float r) {
    const float s = sin_rev_f16out(x * (a * kInv2Pi));
    return __builtin_fmaf(r, s * s, x);
}

}  // namespace dtts
