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

// y = x + r * sin^2(a x). The f32 form uses the full-precision library sinf: f32 outputs are
// held to the reference's 1e-6-of-scale accuracy bound (crates/tts-nn/src/fused.rs:2356-2391).
__device__ __forceinline__ float snake_f32(float x, float a, float r) {
    const float s = sinf(a * x);
    return x + r * (s * s);
}

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
