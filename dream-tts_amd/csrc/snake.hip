// Standalone SnakeBeta passes, NCL and NLC, f32 and f16, and the two folded f32 snakes
// (x + sin^2(x), and alpha[c] x + sin^2(alpha[c] x) channel-major).
//
// Bandwidth-bound: one read and one write of the activation. Each thread moves 16 bytes per
// access (8 f16 or 4 f32) when the channel (NLC) or length (NCL) axis allows; the per-channel
// alpha and 1/beta sit in LDS for NLC, where a 16-byte vector spans several channels, and are
// scalar loads for NCL, where a whole vector shares one channel.
#include "snake.hpp"

namespace dtts {
namespace {

template <typename T>
struct Vec;
template <>
struct Vec<float> {
    static constexpr int N = 4;
    typedef float4_t type;
};
template <>
struct Vec<half_t> {
    static constexpr int N = 8;
    typedef half8_t type;
};

template <typename T>
__device__ __forceinline__ float apply(float x, float a, float r);
template <>
__device__ __forceinline__ float apply<float>(float x, float a, float r) { return snake_f32(x, a, r); }
template <>
__device__ __forceinline__ float apply<half_t>(float x, float a, float r) { return snake_f16out(x, a, r); }

constexpr int kBlock = 256;
constexpr int kLdsChannels = 4096;

// Channels-last: element e is channel e % chan. VEC elements per thread step, VEC | chan.
template <typename T, int VEC, bool LDS>
__global__ __launch_bounds__(kBlock) void snake_nlc_kernel(const T *x,
                                                           const float *__restrict__ alpha,
                                                           const float *__restrict__ brecip,
                                                           T *y, uint32_t nvec,
                                                           uint32_t chan, FastDiv per_row) {
    __shared__ float s_a[LDS ? kLdsChannels : 1];
    __shared__ float s_r[LDS ? kLdsChannels : 1];
    const float *pa = alpha;
    const float *pr = brecip;
    if constexpr (LDS) {
        for (uint32_t c = threadIdx.x; c < chan; c += kBlock) {
            s_a[c] = alpha[c];
            s_r[c] = brecip[c];
        }
        __syncthreads();
        pa = s_a;
        pr = s_r;
    }
    const uint32_t vpr = chan / VEC;
    for (uint32_t v = blockIdx.x * kBlock + threadIdx.x; v < nvec; v += gridDim.x * kBlock) {
        const uint32_t c0 = (v - per_row.div(v) * vpr) * VEC;
        if constexpr (VEC == 1) {
            y[v] = static_cast<T>(apply<T>(static_cast<float>(x[v]), pa[c0], pr[c0]));
        } else {
            typedef typename Vec<T>::type V;
            const V in = reinterpret_cast<const V *>(x)[v];
            V out;
#pragma unroll
            for (int j = 0; j < VEC; ++j)
                out[j] = static_cast<T>(apply<T>(static_cast<float>(in[j]), pa[c0 + j], pr[c0 + j]));
            reinterpret_cast<V *>(y)[v] = out;
        }
    }
}

// What a channel-major pass computes per element: SnakeBeta x + r sin^2(a x), or the
// half-folded snake u + sin^2(u), u = a x, whose 1/alpha lives in the next conv's weights.
enum class Form { kBeta, kAlpha };

template <typename T, Form F>
__device__ __forceinline__ float ncl_value(float x, float a, float r) {
    if constexpr (F == Form::kBeta) {
        return apply<T>(x, a, r);
    } else {
        const float u = a * x;
        const float s = sinf(u);
        return u + s * s;
    }
}

// Channel-major: a row of `len` elements shares channel row % chan. VEC | len.
template <typename T, int VEC, Form F = Form::kBeta>
__global__ __launch_bounds__(kBlock) void snake_ncl_kernel(const T *x,
                                                           const float *__restrict__ alpha,
                                                           const float *__restrict__ brecip,
                                                           T *y, uint32_t nvec,
                                                           FastDiv vec_per_row, FastDiv chan) {
    for (uint32_t v = blockIdx.x * kBlock + threadIdx.x; v < nvec; v += gridDim.x * kBlock) {
        const uint32_t row = vec_per_row.div(v);
        const uint32_t c = row - chan.div(row) * chan.d;
        const float a = alpha[c];
        const float r = F == Form::kBeta ? brecip[c] : 0.0f;
        if constexpr (VEC == 1) {
            y[v] = static_cast<T>(ncl_value<T, F>(static_cast<float>(x[v]), a, r));
        } else {
            typedef typename Vec<T>::type V;
            const V in = reinterpret_cast<const V *>(x)[v];
            V out;
#pragma unroll
            for (int j = 0; j < VEC; ++j) out[j] = static_cast<T>(ncl_value<T, F>(static_cast<float>(in[j]), a, r));
            reinterpret_cast<V *>(y)[v] = out;
        }
    }
}

// y = x + sin^2(x) over a flat array (any layout: no per-channel operand). Four floats per
// thread step when x and y are 16-byte aligned; the scalar tail runs in the same launch.
__global__ __launch_bounds__(kBlock) void snake_folded_kernel(const float *x, float *y, int64_t n) {
    const int64_t stride = int64_t(gridDim.x) * kBlock;
    const int64_t t0 = int64_t(blockIdx.x) * kBlock + threadIdx.x;
    const int64_t nv = n / 4;
    for (int64_t v = t0; v < nv; v += stride) {
        const float4_t in = reinterpret_cast<const float4_t *>(x)[v];
        float4_t out;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float s = sinf(in[j]);
            out[j] = in[j] + s * s;
        }
        reinterpret_cast<float4_t *>(y)[v] = out;
    }
    for (int64_t i = nv * 4 + t0; i < n; i += stride) {
        const float s = sinf(x[i]);
        y[i] = x[i] + s * s;
    }
}

__global__ __launch_bounds__(kBlock) void snake_folded_scalar_kernel(const float *x, float *y, int64_t n) {
    const int64_t stride = int64_t(gridDim.x) * kBlock;
    for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const float s = sinf(x[i]);
        y[i] = x[i] + s * s;
    }
}

// Rows per launch so a launch's vector index fits 31 bits.
inline int64_t rows_per_launch(int64_t row_elems, int vec) {
    const int64_t max_vec = int64_t(1) << 31;
    int64_t r = max_vec * vec / (row_elems > 0 ? row_elems : 1);
    return r < 1 ? 1 : r;
}

template <typename T>
int snake_nlc(const char *name, const T *x, const float *alpha, const float *brecip, T *y,
              int64_t rows, int64_t chan, hipStream_t stream) {
    DTTS_REQUIRE(rows >= 0 && chan >= 0, "%s: negative shape (%lld, %lld)", name, (long long)rows,
                 (long long)chan);
    if (rows == 0 || chan == 0) return DTTS_OK;
    DTTS_REQUIRE(x && y && alpha && brecip, "%s: null pointer", name);
    DTTS_REQUIRE(chan < (int64_t(1) << 31), "%s: %lld channels", name, (long long)chan);
    constexpr int V = Vec<T>::N;
    const bool vec = (chan % V == 0) && aligned(x, 16) && aligned(y, 16);
    const int vw = vec ? V : 1;
    const int64_t step = rows_per_launch(chan, vw);
    for (int64_t r0 = 0; r0 < rows; r0 += step) {
        const int64_t nr = (rows - r0 < step) ? rows - r0 : step;
        const uint32_t nvec = static_cast<uint32_t>(nr * chan / vw);
        const T *xs = x + r0 * chan;
        T *ys = y + r0 * chan;
        const FastDiv per_row(static_cast<uint32_t>(chan / vw));
        const unsigned grid = grid_for(nvec, kBlock);
        const bool lds = chan <= kLdsChannels;
        if (vec && lds)
            snake_nlc_kernel<T, V, true><<<grid, kBlock, 0, stream>>>(xs, alpha, brecip, ys, nvec, chan, per_row);
        else if (vec)
            snake_nlc_kernel<T, V, false><<<grid, kBlock, 0, stream>>>(xs, alpha, brecip, ys, nvec, chan, per_row);
        else if (lds)
            snake_nlc_kernel<T, 1, true><<<grid, kBlock, 0, stream>>>(xs, alpha, brecip, ys, nvec, chan, per_row);
        else
            snake_nlc_kernel<T, 1, false><<<grid, kBlock, 0, stream>>>(xs, alpha, brecip, ys, nvec, chan, per_row);
        DTTS_LAUNCH_CHECK(name);
    }
    return DTTS_OK;
}

template <typename T, Form F = Form::kBeta>
int snake_ncl(const char *name, const T *x, const float *alpha, const float *brecip, T *y,
              int64_t lanes, int64_t chan, int64_t len, hipStream_t stream) {
    DTTS_REQUIRE(lanes >= 0 && chan >= 0 && len >= 0, "%s: negative shape", name);
    if (lanes == 0 || chan == 0 || len == 0) return DTTS_OK;
    DTTS_REQUIRE(x && y && alpha && (brecip || F == Form::kAlpha), "%s: null pointer", name);
    DTTS_REQUIRE(chan < (int64_t(1) << 31) && len < (int64_t(1) << 31), "%s: shape too large", name);
    constexpr int V = Vec<T>::N;
    const bool vec = (len % V == 0) && aligned(x, 16) && aligned(y, 16);
    const int vw = vec ? V : 1;
    // Launch whole lanes at a time so the channel of row r is simply r % chan.
    const int64_t rows_step = rows_per_launch(len, vw);
    int64_t lanes_step = rows_step / chan;
    if (lanes_step < 1) lanes_step = 1;
    DTTS_REQUIRE(chan * len / vw < (int64_t(1) << 31), "%s: one lane exceeds 2^31 vectors", name);
    for (int64_t l0 = 0; l0 < lanes; l0 += lanes_step) {
        const int64_t nl = (lanes - l0 < lanes_step) ? lanes - l0 : lanes_step;
        const uint32_t nvec = static_cast<uint32_t>(nl * chan * len / vw);
        const T *xs = x + l0 * chan * len;
        T *ys = y + l0 * chan * len;
        const FastDiv vpr(static_cast<uint32_t>(len / vw));
        const FastDiv cd(static_cast<uint32_t>(chan));
        const unsigned grid = grid_for(nvec, kBlock);
        if (vec)
            snake_ncl_kernel<T, V, F><<<grid, kBlock, 0, stream>>>(xs, alpha, brecip, ys, nvec, vpr, cd);
        else
            snake_ncl_kernel<T, 1, F><<<grid, kBlock, 0, stream>>>(xs, alpha, brecip, ys, nvec, vpr, cd);
        DTTS_LAUNCH_CHECK(name);
    }
    return DTTS_OK;
}

int snake_folded(const float *x, float *y, int64_t n, hipStream_t stream) {
    const char *name = "dtts_snake_folded_f32";
    DTTS_REQUIRE(n >= 0, "%s: negative length %lld", name, (long long)n);
    if (n == 0) return DTTS_OK;
    DTTS_REQUIRE(x && y, "%s: null pointer", name);
    // Enough workgroups to cover the chip several times over; the loops stride the rest.
    const int64_t vecs = (n + 3) / 4;
    const int64_t want = (vecs + kBlock - 1) / kBlock;
    const unsigned grid = static_cast<unsigned>(want < 65536 ? want : 65536);
    if (aligned(x, 16) && aligned(y, 16))
        snake_folded_kernel<<<grid, kBlock, 0, stream>>>(x, y, n);
    else
        snake_folded_scalar_kernel<<<grid, kBlock, 0, stream>>>(x, y, n);
    DTTS_LAUNCH_CHECK(name);
    return DTTS_OK;
}

}  // namespace
}  // namespace dtts

using dtts::half_t;

extern "C" int dtts_snake_ncl_f32(const float *x, const float *alpha, const float *brecip, float *y,
                                  int64_t lanes, int64_t chan, int64_t len, hipStream_t stream) {
    return dtts::snake_ncl<float>("dtts_snake_ncl_f32", x, alpha, brecip, y, lanes, chan, len, stream);
}

extern "C" int dtts_snake_ncl_f16(const dtts_f16 *x, const float *alpha, const float *brecip,
                                  dtts_f16 *y, int64_t lanes, int64_t chan, int64_t len,
                                  hipStream_t stream) {
    return dtts::snake_ncl<half_t>("dtts_snake_ncl_f16", reinterpret_cast<const half_t *>(x), alpha,
                                   brecip, reinterpret_cast<half_t *>(y), lanes, chan, len, stream);
}

extern "C" int dtts_snake_nlc_f32(const float *x, const float *alpha, const float *brecip, float *y,
                                  int64_t rows, int64_t chan, hipStream_t stream) {
    return dtts::snake_nlc<float>("dtts_snake_nlc_f32", x, alpha, brecip, y, rows, chan, stream);
}

extern "C" int dtts_snake_nlc_f16(const dtts_f16 *x, const float *alpha, const float *brecip,
                                  dtts_f16 *y, int64_t rows, int64_t chan, hipStream_t stream) {
    return dtts::snake_nlc<half_t>("dtts_snake_nlc_f16", reinterpret_cast<const half_t *>(x), alpha,
                                   brecip, reinterpret_cast<half_t *>(y), rows, chan, stream);
}

extern "C" int dtts_snake_folded_f32(const float *x, float *y, int64_t n, hipStream_t stream) {
    return dtts::snake_folded(x, y, n, stream);
}

extern "C" int dtts_snake_alpha_f32(const float *x, const float *alpha, float *y, int64_t lanes, int64_t chan,
                                    int64_t len, hipStream_t stream) {
    return dtts::snake_ncl<float, dtts::Form::kAlpha>("dtts_snake_alpha_f32", x, alpha, nullptr, y, lanes, chan,
                                                      len, stream);
}
