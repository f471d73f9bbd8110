// The decode-shape projections the decoder stack runs for its non-f16 weight kinds, on the same
// kernels as the per-op entry points: Q8_0 (packed layout, f32 activations; q8_0.hip) and f32
// (gemm_f32.hip). Both split k into ranges whose partials [ranges][m][n] the consumer sums in
// order; with one range the output is written directly.
#pragma once

#include "common.hpp"

namespace dtts {

// k ranges of a Q8_0 projection on packed weights in `mode` (0: shape not supported).
int q8_stack_ranges(int64_t m, int64_t k, int64_t n, int32_t mode);
// x [m, k] f32, packed weights [n, k] (dtts_q8_0_repack's layout); mode DTTS_Q8_W8A8 or _W8A32.
// Partials to `part` when there are several ranges (no merge), else y.
int q8_stack_gemm(const float *x, const void *packed, float *y, float *part, int64_t m, int64_t k, int64_t n,
                  int32_t mode, hipStream_t stream);

// k ranges of an f32 projection (0: shape not supported: m <= 64, k % 32 == 0, n % 64 == 0).
int f32_proj_ranges(int64_t m, int64_t k, int64_t n);
// x [m, k] f32, w [n, k] f32; partials to `part` when there are several ranges (summed into y
// when merge), else y.
hipError_t f32_proj_launch(const float *x, const float *w, float *y, float *part, int64_t m, int64_t k, int64_t n,
                           bool merge, hipStream_t stream);

}  // namespace dtts
