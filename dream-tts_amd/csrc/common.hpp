// Shared pieces of libdtts: the thread-local error slot behind dtts_last_error(), argument
// checks, launch checks, f16 vector types and a division by a launch-time constant.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "dtts.h"

namespace dtts {

// ---------------------------------------------------------------- errors

void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define DTTS_REQUIRE(cond, ...)                                                              \
    do {                                                                                      \
        if (!(cond)) {                                                                        \
            ::dtts::set_error(__VA_ARGS__);                                                   \
            return DTTS_ERR_INVALID;                                                          \
        }                                                                                     \
    } while (0)

#define DTTS_HIP_CHECK(expr, what)                                                           \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess) {                                                               \
            ::dtts::set_error("%s: %s", what, hipGetErrorString(e_));                        \
            return DTTS_ERR_HIP;                                                              \
        }                                                                                     \
    } while (0)

// After a <<<>>> launch: a bad launch configuration surfaces here, not at the next sync.
#define DTTS_LAUNCH_CHECK(what) DTTS_HIP_CHECK(hipGetLastError(), what)

inline bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ---------------------------------------------------------------- f16

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- ordered sums of k-range partials

// The sum of n float4 partials `stride` floats apart, in range order, with up to U of the loads
// requested together: a plain loop issues each load only after the previous add, one memory round
// trip per range. ZERO_START: the sum is 0 + p[0] + p[stride] + ... (as a loop from zero adds);
// otherwise it starts at p[0].
template <int U, bool ZERO_START>
__device__ __forceinline__ float4_t ordered_sum4(const float *p, int n, int64_t stride) {
    float4_t u = float4_t{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < n; k0 += U) {
        float4_t v[U];
#pragma unroll
        for (int k = 0; k < U; ++k)
            if (k0 + k < n) v[k] = *reinterpret_cast<const float4_t *>(p + (k0 + k) * stride);
#pragma unroll
        for (int k = 0; k < U; ++k)
            if (k0 + k < n) u = (!ZERO_START && k0 + k == 0) ? v[k] : u + v[k];
    }
    return u;
}

// ---------------------------------------------------------------- division by a constant

// n / d for 32-bit n and a divisor fixed at launch: q = (umulhi(n, m) + n) >> l with
// l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1 (Granlund and Montgomery, 1994).
struct FastDiv {
    uint32_t d, m, l;
    FastDiv() = default;
    __host__ explicit FastDiv(uint32_t div) : d(div) {
        l = 0;
        while ((1ull << l) < div) ++l;
        m = static_cast<uint32_t>(((1ull << 32) * ((1ull << l) - div)) / div + 1);
    }
    __host__ __device__ inline uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
        const uint32_t hi = __umulhi(n, m);
#else
        const uint32_t hi = static_cast<uint32_t>((static_cast<uint64_t>(n) * m) >> 32);
#endif
        return static_cast<uint32_t>((static_cast<uint64_t>(hi) + n) >> l);
    }
};

// ---------------------------------------------------------------- launch geometry

constexpr int kNumCUs = 256;  // MI355X: 8 XCDs x 32 CUs

inline unsigned grid_for(int64_t work_items, int block, int max_blocks_per_cu = 8) {
    int64_t g = (work_items + block - 1) / block;
    const int64_t cap = int64_t(kNumCUs) * max_blocks_per_cu;
    if (g > cap) g = cap;
    if (g < 1) g = 1;
    return static_cast<unsigned>(g);
}

}  // namespace dtts
