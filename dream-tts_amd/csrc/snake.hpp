// SnakeBeta arithmetic shared by the standalone snake kernels and the conv prologues.
#pragma once

#include "common.hpp"

namespace dtts {

// sin(u) through the hardware sine. v_sin_f32 takes its argument in revolutions; reducing to
// [-1/2, 1/2] revolution first keeps it in the range where the unit is accurate. Absolute error
// stays near 1e-6 for |u| up to ~100 (the f32 rounding of u/(2 pi) dominates), far inside an
// f16 ulp, so it is used wherever the snake's result is stored as f16.
__device__ __forceinline__ float sin_f16out(float u) {
    float t = u * 0.159154943091895335768883763372514362f;
    t = t - __builtin_rintf(t);
    return __builtin_amdgcn_sinf(t);
}

// y = x + r * sin^2(a x). The f32 form uses the full-precision library sinf: f32 outputs are
// held to the reference's 1e-6-of-scale accuracy bound (crates/tts-nn/src/fused.rs:2356-2391).
__device__ __forceinline__ float snake_f32(float x, float a, float r) {
    const float s = sinf(a * x);
    return x + r * (s * s);
}

__device__ __forceinline__ float snake_f16out(float x, float a, float r) {
    const float s = sin_f16out(a * x);
    return x + r * (s * s);
}

}  // namespace dtts
