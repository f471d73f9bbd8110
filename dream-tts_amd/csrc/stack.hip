// One decode step of a Qwen3 decoder stack (Stack::forward at t = 1, crates/qwen3tts/src/
// qwen3.rs:294-467) over all layers, every lane at its own position:
//
//   h = x
//   per layer:  a = f16(rms_norm(h, attn_norm))                      rms kernel
//               qkv = a . Wqkv^T                    (f32)             NT GEMM
//               q, cache[pos] <- QK-norm, RoPE, append (or RoPE, q*s)  qk-rope kernel
//               o = f16(attention(q, cache[window .. pos]))           decode attention
//               h += (o . Wo^T) * attn_scale                          NT GEMM, residual epilogue
//               a = f16(rms_norm(h, ffn_norm))                        rms kernel
//               t = f16(silu(a . Wg^T) * (a . Wu^T))                  NT GEMM, gate|up epilogue
//               h += (t . Wdown^T) * mlp_scale                        NT GEMM, residual epilogue
//   out = rms_norm(h, norm)
//
// The f16 roundings are the reference's own: Proj::forward casts its input to f16
// (crates/tts-nn/src/lib.rs:517), so the kernel producing a projection's input stores it in f16
// directly. Everything else is f32, as the reference's f32 activations are.
//
// Decode is launch-bound (8 to 12 small launches per layer), so the step can be captured once
// into a HIP graph and replayed: every kernel reads the lanes' positions from a device array
// that a one-block kernel fills from the kernel arguments before each replay, and the attention
// grid is sized for the longest window the cache allows (workgroups past a lane's window
// return at once). The graph is kept until a call brings other pointers or sizes.
#include <cstring>
#include <new>
#include <vector>

#include "attn.hpp"
#include "gemm_nt.hpp"
#include "norm_rope.hpp"
#include "proj.hpp"

struct dtts_stack {
    dtts_stack_geometry geo;
    int32_t how = DTTS_WEIGHT_F16;  // the layers' weight kind (Stack::load's `how`)
    std::vector<dtts_stack_layer> layers;
    const float *final_norm = nullptr;
    float *cos_t = nullptr, *sin_t = nullptr;  // [capacity, head_dim / 2]
    int32_t *pos = nullptr;                    // [256] device positions of the step being run
    // the captured step
    hipStream_t capture_stream = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<const void *> key;
};

namespace dtts {
namespace {

constexpr int kStackMaxLanes = 64;  // the NT GEMM's row limit

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

__global__ __launch_bounds__(256) void set_positions(Positions p, int32_t *dst, int n) {
    if (static_cast<int>(threadIdx.x) < n) dst[threadIdx.x] = p.p[threadIdx.x];
}

// A projection's output as its consumer reads it: the value itself (ys == 1), or ys partial
// arrays `stride` floats apart, summed in order (the projection's k ranges).
struct Partials {
    const float *p;
    int ys;
    int64_t stride;
};

// The ordered sum of ys partial float4s `stride` floats apart, U of the loads requested together.
template <int U>
__device__ __forceinline__ float4_t sum_parts(const float *p, int ys, int64_t stride) {
    return ordered_sum4<U, false>(p, ys, stride);
}

// Each component rounded to f16 and widened back.
__device__ __forceinline__ float4_t round_f16x4(float4_t u) {
    return float4_t{static_cast<float>(static_cast<half_t>(u[0])), static_cast<float>(static_cast<half_t>(u[1])),
                    static_cast<float>(static_cast<half_t>(u[2])), static_cast<float>(static_cast<half_t>(u[3]))};
}

// Row-wise RMSNorm of the stack, f32 in, the f16 input of the next projection out (or the final
// f32 output). When `add` is set, the row first takes the residual update of the projection that
// precedes it: x + (sum of add's partials) * scale (LayerScale, or 1), rounded as the reference
// rounds h + attn; the updated row is written to h. Layer 0 copies x into h the same way (add
// unset, h set). One workgroup per row; each thread holds NV float4 of the row (every load of the
// row in flight at once); the sum of squares is reduced over the wave, then over the TH/64 waves
// through LDS in wave order.
// round16: the added projection output is the f16 matmul's (rounded once, after the sum)
template <typename TO, int NV, int TH>
__global__ __launch_bounds__(TH) void stack_norm(const float *x, Partials add, const half_t *add16, bool round16,
                                                 const float *scale, float *h, const float *gamma, TO *y, int dim,
                                                 float eps) {
#pragma clang fp contract(off)
    constexpr int NWAVE = TH / 64;
    __shared__ float part[NWAVE];
    const int row = blockIdx.x;
    const int t = threadIdx.x;
    const int64_t ro = static_cast<int64_t>(row) * dim;
    float4_t v[NV], gm[NV];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int e = (i * TH + t) * 4;
        const float4_t z = float4_t{0.f, 0.f, 0.f, 0.f};
        v[i] = e < dim ? *reinterpret_cast<const float4_t *>(x + ro + e) : z;
        gm[i] = e < dim ? *reinterpret_cast<const float4_t *>(gamma + e) : z;
        if ((add.p || add16) && e < dim) {
            float4_t u;
            if (add16) {  // a projection whose output the reference rounds to f16 (candle's f16 matmul)
                const half4_t a4 = *reinterpret_cast<const half4_t *>(add16 + ro + e);
                u = float4_t{static_cast<float>(a4[0]), static_cast<float>(a4[1]), static_cast<float>(a4[2]),
                             static_cast<float>(a4[3])};
            } else {
                u = sum_parts<12>(add.p + ro + e, add.ys, add.stride);
                if (round16) u = round_f16x4(u);
            }
            if (scale) {
                const float4_t sc = *reinterpret_cast<const float4_t *>(scale + e);
                u = u * sc;
            }
            v[i] = v[i] + u;
        }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
    ss = wave_sum(ss);
    if ((t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NWAVE; ++k) ss += part[k];
    const float m = sqrtf(ss / static_cast<float>(dim) + eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int e = (i * TH + t) * 4;
        if (e >= dim) continue;
        TO *yo = y + ro + e;
#pragma unroll
        for (int j = 0; j < 4; ++j) yo[j] = static_cast<TO>((v[i][j] / m) * gm[i][j]);
        if (h) *reinterpret_cast<float4_t *>(h + ro + e) = v[i];
    }
}

// dim % 4 == 0 and dim <= 8192 (checked at create)
template <typename TO>
hipError_t launch_norm(const float *x, Partials add, const float *scale, float *h, const float *gamma, TO *y, int rows,
                       int dim, float eps, hipStream_t stream, const half_t *add16 = nullptr, bool round16 = false) {
    // one float4 per thread up to 4096 columns (more threads per row keep more of its loads in
    // flight: the step's rows are few, so each runs alone on a CU), two up to 8192
    if (dim <= 1024)
        stack_norm<TO, 1, 256><<<rows, 256, 0, stream>>>(x, add, add16, round16, scale, h, gamma, y, dim, eps);
    else if (dim <= 2048)
        stack_norm<TO, 1, 512><<<rows, 512, 0, stream>>>(x, add, add16, round16, scale, h, gamma, y, dim, eps);
    else if (dim <= 4096)
        stack_norm<TO, 1, 1024><<<rows, 1024, 0, stream>>>(x, add, add16, round16, scale, h, gamma, y, dim, eps);
    else
        stack_norm<TO, 2, 1024><<<rows, 1024, 0, stream>>>(x, add, add16, round16, scale, h, gamma, y, dim, eps);
    return hipGetLastError();
}

// t = f16(silu(g) * u) from the gate|up projection's partials (gate columns, then up columns, ys
// arrays of [rows, 2 * ffn]); four columns per thread. TO = float: the f32 swiglu_mul the
// reference feeds an f32 or quantized down projection.
template <typename TO = half_t>
__global__ __launch_bounds__(256) void stack_gateup_merge(Partials gu, TO *t, int rows, int ffn,
                                                          bool round16 = false) {
    typedef TO TO4 __attribute__((ext_vector_type(4)));
    const int c4n = ffn / 4;
    const int64_t total = static_cast<int64_t>(rows) * c4n;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t row = e / c4n;
        const int col = static_cast<int>(e - row * c4n) * 4;
        const float *pr = gu.p + row * 2 * ffn + col;
        float4_t g = sum_parts<8>(pr, gu.ys, gu.stride), u = sum_parts<8>(pr + ffn, gu.ys, gu.stride);
        if (round16) {  // gate and up as the f16 matmul gives them
            g = round_f16x4(g);
            u = round_f16x4(u);
        }
        TO4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = static_cast<TO>(silu_mul(g[j], u[j]));
        *reinterpret_cast<TO4 *>(t + row * ffn + col) = o;
    }
}

struct Plan {  // workspace carve-up for one (lanes, cap)
    size_t h, a16, t16, qkv, q, f32out, gemm_part, attn_part, total;
    size_t gemm_bytes, attn_bytes;
    int max_window;
};

Plan plan_of(const dtts_stack_geometry &g, int64_t lanes, int64_t cap) {
    Plan p{};
    const int64_t qw = g.heads * g.head_dim, kvw = g.n_kv * g.head_dim;
    const int64_t aw = g.dim > qw ? g.dim : qw;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += align256(bytes);
        return at;
    };
    p.h = take(sizeof(float) * lanes * g.dim);
    p.a16 = take(2 * lanes * aw);
    p.t16 = take(2 * lanes * g.ffn);
    p.qkv = take(sizeof(float) * lanes * (qw + 2 * kvw));
    p.q = take(sizeof(float) * lanes * qw);
    // the plain f32 output of a projection whose consumer rounds it to f16 (wo, gate|up, down)
    p.f32out = take(sizeof(float) * lanes * (g.dim > 2 * g.ffn ? g.dim : 2 * g.ffn));
    // one partial region serves every projection: each one's partials are summed by its consumer
    // before the next projection runs
    size_t gb = 0;
    const int64_t shapes[5][3] = {
        {g.dim, qw + 2 * kvw, 0}, {qw, g.dim, 2}, {g.dim, 2 * g.ffn, 1}, {g.ffn, g.dim, 2}, {g.dim, 2 * g.ffn, 0}};
    for (const auto &sh : shapes) {
        const size_t v = lds_partial_bytes(pick_lds(lanes, sh[0], sh[1], static_cast<int>(sh[2])), lanes, sh[1]);
        gb = v > gb ? v : gb;
    }
    p.gemm_bytes = gb;
    p.gemm_part = take(gb);
    const int64_t win = g.window > 0 && g.window < cap ? g.window : cap;
    p.max_window = static_cast<int>(win);
    p.attn_bytes = attn_workspace_bytes(lanes, g.n_kv, g.heads / g.n_kv, g.head_dim, win);
    p.attn_part = take(p.attn_bytes);
    p.total = off;
    return p;
}

// One projection of the step on the A-sharing kernel. With several k ranges it leaves the
// partials in `part` and returns them for the consumer to sum; with one it applies its own
// epilogue (c, c16, scale) and returns the plain output (`plain`, or {} for the residual form,
// whose result is already in h).
template <int MODE>
hipError_t stack_gemm(const half_t *a, const half_t *w, float *c, half_t *c16, const float *scale, int m, int k, int n,
                      float *part, const float *plain, Partials &out, hipStream_t stream, int max_m = 64) {
    GemmParams p{};
    p.a = a;
    p.w = w;
    p.c = c;
    p.c16 = c16;
    p.scale = scale;
    p.m = m;
    p.k = k;
    p.n = n;
    const LdsPlan pl = pick_lds(m, k, n, MODE, max_m);
    out = pl.ys > 1 ? Partials{part, pl.ys, static_cast<int64_t>(m) * n} : Partials{plain, 1, 0};
    return launch_lds_nt<MODE>(p, pl, part, stream, false);
}

// skinny::eligible (crates/tts-nn/src/skinny.rs:123-131, MAX_M = 48): the projections Proj::Half
// sends to the skinny GEMM, whose output is f32; every other one goes through candle's f16 matmul,
// whose output is f16 (lib.rs:516-529).
bool skinny_eligible(int64_t m, int64_t k, int64_t n) { return m <= 48 && m % 8 == 0 && k % 32 == 0 && n % 64 == 0; }

#define STACK_STEP(expr)                          \
    do {                                          \
        const hipError_t e_ = (expr);             \
        if (e_ != hipSuccess) return e_;          \
    } while (0)

// Enqueues the step (after the positions are on the device).
hipError_t enqueue_step(const dtts_stack &s, const float *x, float *out, const dtts_stack_cache *caches, int lanes,
                        int cap, char *ws, const Plan &pl, hipStream_t stream) {
    const dtts_stack_geometry &g = s.geo;
    const int dim = static_cast<int>(g.dim), hd = static_cast<int>(g.head_dim);
    const int heads = static_cast<int>(g.heads), n_kv = static_cast<int>(g.n_kv), ffn = static_cast<int>(g.ffn);
    const int qw = heads * hd, qkvw = (heads + 2 * n_kv) * hd;
    const int gqa = heads / n_kv;
    float *h = reinterpret_cast<float *>(ws + pl.h);
    half_t *a16 = reinterpret_cast<half_t *>(ws + pl.a16);
    half_t *t16 = reinterpret_cast<half_t *>(ws + pl.t16);
    float *qkv = reinterpret_cast<float *>(ws + pl.qkv);
    float *q = reinterpret_cast<float *>(ws + pl.q);
    float *gpart = pl.gemm_bytes ? reinterpret_cast<float *>(ws + pl.gemm_part) : nullptr;
    float *apart = pl.attn_bytes ? reinterpret_cast<float *>(ws + pl.attn_part) : nullptr;
    const int max_chunks = apart ? (pl.max_window + kChunk - 1) / kChunk : 0;
    const float qscale = g.qk_norm ? 1.0f : static_cast<float>(1.0 / std::sqrt(static_cast<double>(g.head_dim)));
    const DevSpans spans{s.pos, static_cast<int>(g.window)};
    // Projections the reference runs through candle's f16 matmul (lanes not a multiple of 8, or
    // more than 48: a single lane's decode among them) take the plain-output form here, and each
    // consumer rounds the summed output to f16 as that matmul's output is.
    const bool r_qkv = !skinny_eligible(lanes, dim, qkvw), r_o = !skinny_eligible(lanes, qw, dim);
    const bool r_gu = !skinny_eligible(lanes, dim, ffn), r_d = !skinny_eligible(lanes, ffn, dim);
    float *fbuf = reinterpret_cast<float *>(ws + pl.f32out);
    Partials pending{};             // the previous layer's down projection, not yet in h
    const float *pending_scale = nullptr;
    bool pending_round = false;
    for (int64_t li = 0; li < g.layers; ++li) {
        const dtts_stack_layer &L = s.layers[li];
        // h = x (layer 0) or h + the previous layer's MLP output; a = f16(rms_norm(h))
        STACK_STEP(launch_norm(li == 0 ? x : h, pending, pending_scale, h, L.attn_norm, a16, lanes, dim, g.eps, stream,
                               nullptr, pending_round));
        Partials r{};
        STACK_STEP(stack_gemm<0>(a16, reinterpret_cast<const half_t *>(L.wqkv), qkv, nullptr, nullptr, lanes, dim, qkvw,
                                 gpart, qkv, r, stream));
        const int waves = lanes * (heads + n_kv);
        qk_rope_kernel<float, DevPositions><<<static_cast<unsigned>((waves + 3) / 4), 256, 0, stream>>>(
            r.p, g.qk_norm ? L.qk_norms : nullptr, s.cos_t, s.sin_t, DevPositions{s.pos}, q, nullptr,
            reinterpret_cast<half_t *>(caches[li].k), reinterpret_cast<half_t *>(caches[li].v), lanes, heads, n_kv,
            hd, cap, g.eps, qscale, r.ys, r.stride, r_qkv);
        STACK_STEP(hipGetLastError());
        STACK_STEP(launch_attention(q, reinterpret_cast<const half_t *>(caches[li].k),
                                    reinterpret_cast<const half_t *>(caches[li].v), a16, apart, max_chunks, lanes,
                                    n_kv, gqa, hd, cap, spans, stream));
        const float *attn_scale = g.layer_scale ? L.attn_scale : nullptr;
        if (r_o)
            STACK_STEP(stack_gemm<0>(a16, reinterpret_cast<const half_t *>(L.wo), fbuf, nullptr, nullptr, lanes, qw, dim,
                                     gpart, fbuf, r, stream));
        else
            STACK_STEP(stack_gemm<2>(a16, reinterpret_cast<const half_t *>(L.wo), h, nullptr, attn_scale, lanes, qw, dim,
                                     gpart, nullptr, r, stream));
        // h += attn * attn_scale (when the projection left partials); a = f16(rms_norm(h))
        STACK_STEP(launch_norm(h, r, attn_scale, h, L.ffn_norm, a16, lanes, dim, g.eps, stream, nullptr, r_o));
        if (r_gu) {
            STACK_STEP(stack_gemm<0>(a16, reinterpret_cast<const half_t *>(L.w_gateup), fbuf, nullptr, nullptr, lanes,
                                     dim, 2 * ffn, gpart, fbuf, r, stream));
            stack_gateup_merge<<<grid_for(int64_t(lanes) * ffn / 4, 256, 4), 256, 0, stream>>>(r, t16, lanes, ffn, true);
            STACK_STEP(hipGetLastError());
        } else {
            STACK_STEP(stack_gemm<1>(a16, reinterpret_cast<const half_t *>(L.w_gateup), nullptr, t16, nullptr, lanes,
                                     dim, 2 * ffn, gpart, nullptr, r, stream));
            if (r.p) {
                stack_gateup_merge<<<grid_for(int64_t(lanes) * ffn / 4, 256, 4), 256, 0, stream>>>(r, t16, lanes, ffn);
                STACK_STEP(hipGetLastError());
            }
        }
        const float *mlp_scale = g.layer_scale ? L.mlp_scale : nullptr;
        if (r_d)
            STACK_STEP(stack_gemm<0>(t16, reinterpret_cast<const half_t *>(L.wdown), fbuf, nullptr, nullptr, lanes, ffn,
                                     dim, gpart, fbuf, pending, stream));
        else
            STACK_STEP(stack_gemm<2>(t16, reinterpret_cast<const half_t *>(L.wdown), h, nullptr, mlp_scale, lanes, ffn,
                                     dim, gpart, nullptr, pending, stream));
        pending_scale = mlp_scale;
        pending_round = r_d;
    }
    // h + the last MLP output, then the final norm
    return launch_norm(h, pending, pending_scale, static_cast<float *>(nullptr), s.final_norm, out, lanes, dim, g.eps,
                       stream, nullptr, pending_round);
}

// ---------------------------------------------------------------- f32 and Q8_0 layers
//
// Stack::load with Weight::F32 or Weight::Quant keeps f32 caches (crates/qwen3tts/src/qwen3.rs:
// 242-246), and Proj::forward hands those projections the f32 hidden state and takes f32 back
// (crates/tts-nn/src/lib.rs:509-531): no f16 rounding anywhere in the step. Per layer:
//   a = rms_norm(h)                          rms kernel (f32 out; adds the previous projection)
//   qkv = proj(a)                            f32 (Proj::Dense) or Q8_0 (QMatMul) A-sharing kernel
//   q, cache[pos] <- QK-norm, RoPE, append   qk-rope kernel on f32 caches (the composed route:
//                                            rms_norm over each head, rope, slice_set in f32)
//   o = attention(q, cache)                  decode attention over the f32 caches, f32 out
//   h += proj(o) * attn_scale                (summed by the next norm)
//   t = swiglu_mul(proj_gate(a), proj_up(a)) gate|up rows in one projection, f32 merge
//   h += proj(t) * mlp_scale
// The projections' k ranges are left as partials and summed in order by the consumer.

bool weight_kind_dense_f32(int32_t how) { return how == DTTS_WEIGHT_F32; }
int32_t q8_mode_of(int32_t how) { return how == DTTS_WEIGHT_Q8_0_A32 ? DTTS_Q8_W8A32 : DTTS_Q8_W8A8; }

int proj_ranges(int32_t how, int64_t m, int64_t k, int64_t n) {
    return weight_kind_dense_f32(how) ? f32_proj_ranges(m, k, n) : q8_stack_ranges(m, k, n, q8_mode_of(how));
}

// Whether the kind's projection kernel takes [m, k] x [n, k]: m <= 64, n % 64 == 0, and k a
// multiple of 32 (f32) or 256 (Q8_0, the packed layout).
bool proj_shape_ok(int32_t how, int64_t k, int64_t n) {
    return n % 64 == 0 && (weight_kind_dense_f32(how) ? k % 32 == 0 : k % 256 == 0) && proj_ranges(how, 64, k, n) > 0;
}

struct PlanW {  // workspace carve-up of the f32 / Q8_0 step
    size_t h, a, qkv, q, o, fbuf, t, part, attn_part, total;
    size_t part_bytes, attn_bytes;
    int max_window;
};

PlanW plan_w(const dtts_stack_geometry &g, int32_t how, int64_t lanes, int64_t cap) {
    PlanW p{};
    const int64_t qw = g.heads * g.head_dim, kvw = g.n_kv * g.head_dim, qkvw = qw + 2 * kvw;
    const int64_t aw = g.dim > g.ffn ? g.dim : g.ffn;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += align256(bytes);
        return at;
    };
    const size_t f = sizeof(float) * lanes;
    p.h = take(f * g.dim);
    p.a = take(f * aw);
    p.qkv = take(f * qkvw);
    p.q = take(f * qw);
    p.o = take(f * qw);
    p.fbuf = take(f * (g.dim > 2 * g.ffn ? g.dim : 2 * g.ffn));
    p.t = take(f * g.ffn);
    const int64_t shapes[4][2] = {{g.dim, qkvw}, {qw, g.dim}, {g.dim, 2 * g.ffn}, {g.ffn, g.dim}};
    size_t pb = 0;
    for (const auto &sh : shapes) {
        const int r = proj_ranges(how, lanes, sh[0], sh[1]);
        const size_t v = r > 1 ? f * sh[1] * r : 0;
        pb = v > pb ? v : pb;
    }
    p.part_bytes = pb;
    p.part = take(pb);
    const int64_t win = g.window > 0 && g.window < cap ? g.window : cap;
    p.max_window = static_cast<int>(win);
    p.attn_bytes = attn_workspace_bytes(lanes, g.n_kv, g.heads / g.n_kv, g.head_dim, win);
    p.attn_part = take(p.attn_bytes);
    p.total = off;
    return p;
}

// One f32 or Q8_0 projection: the partials (several k ranges) or the plain output, as its
// consumer reads them.
hipError_t proj_w(int32_t how, const float *x, const void *w, float *plain, float *part, int m, int k, int n,
                  Partials &out, hipStream_t stream) {
    const int r = proj_ranges(how, m, k, n);
    out = r > 1 ? Partials{part, r, static_cast<int64_t>(m) * n} : Partials{plain, 1, 0};
    if (weight_kind_dense_f32(how)) return f32_proj_launch(x, static_cast<const float *>(w), plain, part, m, k, n, false, stream);
    return q8_stack_gemm(x, w, plain, part, m, k, n, q8_mode_of(how), stream) == DTTS_OK ? hipSuccess
                                                                                          : hipErrorInvalidValue;
}

hipError_t enqueue_step_w(const dtts_stack &s, const float *x, float *out, const dtts_stack_cache *caches, int lanes,
                          int cap, char *ws, const PlanW &pl, hipStream_t stream) {
    const dtts_stack_geometry &g = s.geo;
    const int dim = static_cast<int>(g.dim), hd = static_cast<int>(g.head_dim);
    const int heads = static_cast<int>(g.heads), n_kv = static_cast<int>(g.n_kv), ffn = static_cast<int>(g.ffn);
    const int qw = heads * hd, qkvw = (heads + 2 * n_kv) * hd;
    const int gqa = heads / n_kv;
    float *h = reinterpret_cast<float *>(ws + pl.h);
    float *a = reinterpret_cast<float *>(ws + pl.a);
    float *qkv = reinterpret_cast<float *>(ws + pl.qkv);
    float *q = reinterpret_cast<float *>(ws + pl.q);
    float *o = reinterpret_cast<float *>(ws + pl.o);
    float *fbuf = reinterpret_cast<float *>(ws + pl.fbuf);
    float *t = reinterpret_cast<float *>(ws + pl.t);
    float *part = pl.part_bytes ? reinterpret_cast<float *>(ws + pl.part) : nullptr;
    float *apart = pl.attn_bytes ? reinterpret_cast<float *>(ws + pl.attn_part) : nullptr;
    const int max_chunks = apart ? (pl.max_window + kChunk - 1) / kChunk : 0;
    const float qscale = g.qk_norm ? 1.0f : static_cast<float>(1.0 / std::sqrt(static_cast<double>(g.head_dim)));
    const DevSpans spans{s.pos, static_cast<int>(g.window)};
    const int32_t how = s.how;
    Partials pending{};  // the previous layer's down projection, not yet in h
    const float *pending_scale = nullptr;
    for (int64_t li = 0; li < g.layers; ++li) {
        const dtts_stack_layer &L = s.layers[li];
        float *kc = static_cast<float *>(caches[li].k);
        float *vc = static_cast<float *>(caches[li].v);
        STACK_STEP(launch_norm(li == 0 ? x : h, pending, pending_scale, h, L.attn_norm, a, lanes, dim, g.eps, stream));
        Partials r{};
        STACK_STEP(proj_w(how, a, L.wqkv, qkv, part, lanes, dim, qkvw, r, stream));
        const int waves = lanes * (heads + n_kv);
        qk_rope_kernel<float, DevPositions, float><<<static_cast<unsigned>((waves + 3) / 4), 256, 0, stream>>>(
            r.p, g.qk_norm ? L.qk_norms : nullptr, s.cos_t, s.sin_t, DevPositions{s.pos}, q, nullptr, kc, vc, lanes,
            heads, n_kv, hd, cap, g.eps, qscale, r.ys, r.stride, false);
        STACK_STEP(hipGetLastError());
        STACK_STEP(launch_attention(q, static_cast<const float *>(kc), static_cast<const float *>(vc), o, apart,
                                    max_chunks, lanes, n_kv, gqa, hd, cap, spans, stream));
        const float *attn_scale = g.layer_scale ? L.attn_scale : nullptr;
        STACK_STEP(proj_w(how, o, L.wo, fbuf, part, lanes, qw, dim, r, stream));
        STACK_STEP(launch_norm(h, r, attn_scale, h, L.ffn_norm, a, lanes, dim, g.eps, stream));
        STACK_STEP(proj_w(how, a, L.w_gateup, fbuf, part, lanes, dim, 2 * ffn, r, stream));
        stack_gateup_merge<float><<<grid_for(int64_t(lanes) * ffn / 4, 256, 4), 256, 0, stream>>>(r, t, lanes, ffn);
        STACK_STEP(hipGetLastError());
        STACK_STEP(proj_w(how, t, L.wdown, fbuf, part, lanes, ffn, dim, pending, stream));
        pending_scale = g.layer_scale ? L.mlp_scale : nullptr;
    }
    return launch_norm(h, pending, pending_scale, static_cast<float *>(nullptr), s.final_norm, out, lanes, dim, g.eps,
                       stream);
}

size_t step_bytes(const dtts_stack &s, int64_t lanes, int64_t cap) {
    return s.how == DTTS_WEIGHT_F16 ? plan_of(s.geo, lanes, cap).total : plan_w(s.geo, s.how, lanes, cap).total;
}

hipError_t enqueue_any(const dtts_stack &s, const float *x, float *out, const dtts_stack_cache *caches, int lanes,
                       int cap, char *ws, hipStream_t stream) {
    if (s.how == DTTS_WEIGHT_F16) return enqueue_step(s, x, out, caches, lanes, cap, ws, plan_of(s.geo, lanes, cap), stream);
    return enqueue_step_w(s, x, out, caches, lanes, cap, ws, plan_w(s.geo, s.how, lanes, cap), stream);
}

// ---------------------------------------------------------------- prefill (t >= 2)
//
// Stack::forward's prefill branch (qwen3.rs:329-336, 415-444) for lanes sharing `start`: rows are
// (lane, t) pairs, lane-major. Proj::Half sends a projection of at most 48 rows (a multiple of 8)
// to the skinny GEMM (f32 output, skinny.rs:123-131) and every other one to candle's f16 matmul,
// whose output is f16 (lib.rs:516-529); the prefill keeps that routing: the A-sharing kernel for
// the former, the channels-last tile kernel (k = 1, f32 accumulation, one f16 rounding) for the
// latter. The new positions attend over their own f32 k and v and the cache's f16 prefix.

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}


// t = f16(silu(g) * u) from f16 gate|up outputs [rows, 2 * ffn] (swiglu_mul over the widened
// values, fused.rs:289-385); four columns per thread.
__global__ __launch_bounds__(256) void prefill_gateup_merge16(const half_t *gu, half_t *t, int rows, int ffn) {
    const int c4n = ffn / 4;
    const int64_t total = static_cast<int64_t>(rows) * c4n;
    for (int64_t e = blockIdx.x * int64_t(256) + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t row = e / c4n;
        const int col = static_cast<int>(e - row * c4n) * 4;
        const half4_t g = *reinterpret_cast<const half4_t *>(gu + row * 2 * ffn + col);
        const half4_t u = *reinterpret_cast<const half4_t *>(gu + row * 2 * ffn + ffn + col);
        half4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = static_cast<half_t>(silu_mul(static_cast<float>(g[j]), static_cast<float>(u[j])));
        *reinterpret_cast<half4_t *>(t + row * ffn + col) = o;
    }
}

constexpr int kPrefillMaxKeys = 16000;  // a wave's scores and query in LDS: at most 64 KB per workgroup

// The prefill branch's attention, QP consecutive queries of one (lane, head) per wave (rows
// bi*t + ti0 .. ti0+QP-1): query ti attends over keys lo .. start + ti, lo = start + ti + 1 - window
// (or 0), from the f16 cache below start and the f32 kf / vf from start on. scores = q . k (times
// `scale` when the layer has no QK-norm), then softmax_last_dim as candle computes it (max,
// exp(s - max), sum, probs = e / sum), then probs . v; the result is stored f16, as wo's
// Proj::Half casts it. Each key and value row is read once for the wave's queries: a key outside
// a query's range gets probability exactly 0, so its term adds nothing and the sums keep key
// order. WPB waves per workgroup, each with QP * (keys + D) floats of LDS.
template <int D, int QP>
__global__ __launch_bounds__(256) void prefill_attention(const float *q, const half_t *kc, const half_t *vc,
                                                         const float *kf, const float *vf, half_t *out, int lanes, int t,
                                                         int start, int heads, int n_kv, int cap, int window, float scale,
                                                         int keys, int wpb) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float sc_all[];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int groups = (t + QP - 1) / QP;
    const int wid = blockIdx.x * wpb + w;
    if (w >= wpb || wid >= lanes * groups * heads) return;
    float *sc = sc_all + static_cast<int64_t>(w) * QP * (keys + D);  // [QP][keys]
    float *qs = sc + QP * keys;                                       // [QP][D]
    const int h = wid % heads, grp = (wid / heads) % groups, bi = wid / (heads * groups);
    const int ti0 = grp * QP;
    const int nq = t - ti0 < QP ? t - ti0 : QP;  // valid queries of the wave
    const int kh = h / (heads / n_kv);
    auto lo_of = [&](int ti) { return window > 0 && start + ti + 1 > window ? start + ti + 1 - window : 0; };
    const int lo = lo_of(ti0), hi = start + ti0 + nq - 1;  // the union of the queries' key ranges
    const int n = hi - lo + 1;
    const half_t *kcr = kc + (static_cast<int64_t>(bi) * n_kv + kh) * cap * D;
    const half_t *vcr = vc + (static_cast<int64_t>(bi) * n_kv + kh) * cap * D;
    const float *kfr = kf + (static_cast<int64_t>(bi) * n_kv + kh) * t * D;
    const float *vfr = vf + (static_cast<int64_t>(bi) * n_kv + kh) * t * D;
#pragma unroll
    for (int a = 0; a < QP; ++a) {
        const float *qr = q + ((static_cast<int64_t>(bi) * heads + h) * t + (a < nq ? ti0 + a : ti0)) * D;
#pragma unroll
        for (int r = 0; r < D / 64; ++r) qs[a * D + lane + 64 * r] = qr[lane + 64 * r];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the queries, read by every lane below
    // scores: a key per lane, each dot product in dimension order
    float mx[QP];
#pragma unroll
    for (int a = 0; a < QP; ++a) mx[a] = -INFINITY;
    for (int i = lane; i < n; i += 64) {
        const int j = lo + i;
        float acc[QP];
#pragma unroll
        for (int a = 0; a < QP; ++a) acc[a] = 0.0f;
        if (j < start) {
            const half_t *kr = kcr + static_cast<int64_t>(j) * D;
#pragma unroll 4
            for (int d = 0; d < D; d += 8) {
                const half8_t k8 = *reinterpret_cast<const half8_t *>(kr + d);
#pragma unroll
                for (int a = 0; a < QP; ++a) {
                    const float4_t q0 = *reinterpret_cast<const float4_t *>(qs + a * D + d);
                    const float4_t q1 = *reinterpret_cast<const float4_t *>(qs + a * D + d + 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[a] += q0[e] * static_cast<float>(k8[e]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[a] += q1[e] * static_cast<float>(k8[e + 4]);
                }
            }
        } else {
            const float *kr = kfr + static_cast<int64_t>(j - start) * D;
#pragma unroll 4
            for (int d = 0; d < D; d += 4) {
                const float4_t k4 = *reinterpret_cast<const float4_t *>(kr + d);
#pragma unroll
                for (int a = 0; a < QP; ++a) {
                    const float4_t q4 = *reinterpret_cast<const float4_t *>(qs + a * D + d);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[a] += q4[e] * k4[e];
                }
            }
        }
#pragma unroll
        for (int a = 0; a < QP; ++a) {
            const bool in = a < nq && j >= lo_of(ti0 + a) && j <= start + ti0 + a;
            float v = acc[a];
            if (scale != 1.0f) v = v * scale;
            sc[a * keys + i] = in ? v : -INFINITY;
            if (in) mx[a] = fmaxf(mx[a], v);
        }
    }
    float sum[QP];
#pragma unroll
    for (int a = 0; a < QP; ++a) {
        mx[a] = wave_max(mx[a]);
        sum[a] = 0.0f;
    }
    for (int i = lane; i < n; i += 64) {
#pragma unroll
        for (int a = 0; a < QP; ++a) {
            const float e = a < nq ? expf(sc[a * keys + i] - mx[a]) : 0.0f;  // exactly 0 outside the range
            sc[a * keys + i] = e;
            sum[a] += e;
        }
    }
#pragma unroll
    for (int a = 0; a < QP; ++a) sum[a] = wave_sum(sum[a]);
    for (int i = lane; i < n; i += 64) {
#pragma unroll
        for (int a = 0; a < QP; ++a) sc[a * keys + i] = a < nq ? sc[a * keys + i] / sum[a] : 0.0f;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's probabilities, read by every lane below
    // probs . v: the lane owns D / 64 dimensions; U keys' loads in flight, summed in key order
    constexpr int PER = D / 64;
    constexpr int U = 8;
    float o[QP][PER];
#pragma unroll
    for (int a = 0; a < QP; ++a)
#pragma unroll
        for (int r = 0; r < PER; ++r) o[a][r] = 0.0f;
    auto add = [&](int i0, const float (&vv)[PER]) {
#pragma unroll
        for (int a = 0; a < QP; ++a) {
            const float pj = sc[a * keys + i0];
#pragma unroll
            for (int r = 0; r < PER; ++r) o[a][r] += pj * vv[r];
        }
    };
    int i = 0;
    const int n_prior = start > lo ? (start - lo < n ? start - lo : n) : 0;
    for (; i + U <= n_prior; i += U) {
        float vv[U][PER];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const half_t *vr = vcr + static_cast<int64_t>(lo + i + u) * D;
#pragma unroll
            for (int r = 0; r < PER; ++r) vv[u][r] = static_cast<float>(vr[lane + 64 * r]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) add(i + u, vv[u]);
    }
    for (; i < n_prior; ++i) {
        float vv[PER];
        const half_t *vr = vcr + static_cast<int64_t>(lo + i) * D;
#pragma unroll
        for (int r = 0; r < PER; ++r) vv[r] = static_cast<float>(vr[lane + 64 * r]);
        add(i, vv);
    }
    for (; i + U <= n; i += U) {
        float vv[U][PER];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float *vr = vfr + static_cast<int64_t>(lo + i + u - start) * D;
#pragma unroll
            for (int r = 0; r < PER; ++r) vv[u][r] = vr[lane + 64 * r];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) add(i + u, vv[u]);
    }
    for (; i < n; ++i) {
        float vv[PER];
        const float *vr = vfr + static_cast<int64_t>(lo + i - start) * D;
#pragma unroll
        for (int r = 0; r < PER; ++r) vv[r] = vr[lane + 64 * r];
        add(i, vv);
    }
#pragma unroll
    for (int a = 0; a < QP; ++a) {
        if (a >= nq) break;
        half_t *dst = out + (static_cast<int64_t>(bi) * t + ti0 + a) * heads * D + h * D;
#pragma unroll
        for (int r = 0; r < PER; ++r) dst[lane + 64 * r] = static_cast<half_t>(o[a][r]);
    }
}

// The same attention on the f32 matrix cores (v_mfma_f32_32x32x2_f32), one workgroup of NW
// waves per (lane bi, head h, 32 consecutive queries ti0 ..), the waves taking alternate blocks
// of 32 keys. A score block is K . Q^T, so a lane holds 16 keys of one query (its lane index mod
// 32); MFMA step s pairs dimension s (lanes 0-31) with dimension D/2 + s (lanes 32-63), so a
// lane's operands are D/2 contiguous floats of its key row and of its query row (16-byte loads).
// The scores go to LDS ([key][query], rows 34 floats apart), masked to -inf outside each query's
// range; then softmax_last_dim as candle computes it (max, exp(s - max), sum, probs = e / sum),
// the waves' maxima and sums combined through LDS (the sums in wave order); then each wave's
// out^T = V^T . P^T over its key blocks in 32-dimension blocks, two keys per step (key s and
// s + 16 of a block), and wave 0 adds the others' partials in wave order. The dot products are summed in the matrix
// cores' order rather than dimension order; the prefill's f32 tolerance holds either way. A
// block's keys (or values) load under the previous block's MFMAs, within two waves per SIMD's
// registers. LDS: the keys x 34 floats, at least (NW - 1) partial outputs of D x 32 floats.
constexpr int kPrefillMfmaPitch = 34;          // 16 rows x 34 floats = 32 banks apart (mod 64)
constexpr int kPrefillMfmaMaxLds = 64 * 1024;  // dynamic + static LDS; longer key ranges take prefill_attention
constexpr int kPrefillMfmaMinT = 16;           // fewer queries leave most of a 32-query block idle
constexpr int kPrefillMfmaWaves = 2;           // waves per 32-query block, on alternate key blocks (4: slower)

// The kernel's static LDS (its `red` array of maxima and sums), counted against kPrefillMfmaMaxLds
// with the dynamic rows.
template <int NW>
constexpr size_t prefill_mfma_static_lds() { return 2 * NW * 32 * sizeof(float); }

template <int D, int NW>
__global__ __launch_bounds__(64 * NW, 2) void prefill_attention_mfma(const float *q, const half_t *kc, const half_t *vc,
                                                                 const float *kf, const float *vf, half_t *out, int t,
                                                                 int start, int heads, int n_kv, int cap, int window,
                                                                 float scale) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float sc[];  // [keys][kPrefillMfmaPitch], then wave 1's output
    __shared__ float red[2][NW][32];                             // [max | sum][wave][query]
    static_assert(sizeof(red) == prefill_mfma_static_lds<NW>(), "static LDS counted on the host");
    constexpr int H = D / 2, NDB = D / 32, P = kPrefillMfmaPitch;
    static_assert(D == 64 || D == 128, "head dim");
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, l32 = lane & 31, hf = lane >> 5;
    const int qblocks = (t + 31) / 32;
    // the query blocks of lane bi in an order rotated by bi: consecutive workgroups, which land on
    // different CUs, mix long and short key ranges
    const int h = blockIdx.x % heads, bi = blockIdx.x / (heads * qblocks);
    const int qb = ((blockIdx.x / heads) % qblocks + bi) % qblocks;
    const int ti0 = qb * 32;
    const int nq = t - ti0 < 32 ? t - ti0 : 32;
    const int kh = h / (heads / n_kv);
    auto lo_of = [&](int ti) { return window > 0 && start + ti + 1 > window ? start + ti + 1 - window : 0; };
    const int lo = lo_of(ti0), hi = start + ti0 + nq - 1;  // the union of the block's key ranges
    const int nb = (hi - lo + 32) / 32;
    const half_t *kcr = kc + (static_cast<int64_t>(bi) * n_kv + kh) * cap * D;
    const half_t *vcr = vc + (static_cast<int64_t>(bi) * n_kv + kh) * cap * D;
    const float *kfr = kf + (static_cast<int64_t>(bi) * n_kv + kh) * t * D;
    const float *vfr = vf + (static_cast<int64_t>(bi) * n_kv + kh) * t * D;
    const bool qok = l32 < nq;
    const int tq = ti0 + l32;  // this lane's query
    float qv[H];
    {
        const float *qr = q + ((static_cast<int64_t>(bi) * heads + h) * t + (qok ? tq : ti0)) * D + hf * H;
#pragma unroll
        for (int e = 0; e < H; e += 4) {
            const float4_t v = *reinterpret_cast<const float4_t *>(qr + e);
#pragma unroll
            for (int c = 0; c < 4; ++c) qv[e + c] = qok ? v[c] : 0.0f;
        }
    }
    // key row j's dims hf*H .. hf*H + H - 1 as f32 (zeros past the range)
    auto load_k = [&](int j, float (&kv)[H]) {
        if (j > hi) {
#pragma unroll
            for (int e = 0; e < H; ++e) kv[e] = 0.0f;
        } else if (j < start) {
            const half_t *kr = kcr + static_cast<int64_t>(j) * D + hf * H;
#pragma unroll
            for (int e = 0; e < H; e += 8) {
                const half8_t v = *reinterpret_cast<const half8_t *>(kr + e);
#pragma unroll
                for (int c = 0; c < 8; ++c) kv[e + c] = static_cast<float>(v[c]);
            }
        } else {
            const float *kr = kfr + static_cast<int64_t>(j - start) * D + hf * H;
#pragma unroll
            for (int e = 0; e < H; e += 4) {
                const float4_t v = *reinterpret_cast<const float4_t *>(kr + e);
#pragma unroll
                for (int c = 0; c < 4; ++c) kv[e + c] = v[c];
            }
        }
    };
    float mx = -INFINITY;  // over this lane's rows of its query's scores
    auto score_block = [&](int b, const float (&kv)[H]) {
        float16_t acc = {};
#pragma unroll
        for (int s = 0; s < H; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[s], qv[s], acc, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int i = 32 * b + 8 * (v >> 2) + 4 * hf + (v & 3);  // key lo + i
            const int jj = lo + i;
            const bool in = qok && jj <= start + tq && jj >= lo_of(tq);
            float x = acc[v];
            if (scale != 1.0f) x = x * scale;
            sc[i * P + l32] = in ? x : -INFINITY;
            if (in) mx = fmaxf(mx, x);
        }
    };
    {
        // the wave's blocks w, w + 2, ...: the next one's keys load under the current one's MFMAs
        float k0[H], k1[H];
        if (w < nb) load_k(lo + 32 * w + l32, k0);
        for (int b = w; b < nb; b += 2 * NW) {
            if (b + NW < nb) load_k(lo + 32 * (b + NW) + l32, k1);
            score_block(b, k0);
            if (b + NW < nb) {
                if (b + 2 * NW < nb) load_k(lo + 32 * (b + 2 * NW) + l32, k0);
                score_block(b + NW, k1);
            }
        }
    }
    // softmax over the query's keys: each wave over its own blocks' rows, lane (query l32, half
    // hf) taking every second row; the waves' maxima and sums meet in LDS
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (hf == 0) red[0][w][l32] = mx;
    __syncthreads();
    mx = red[0][0][l32];
#pragma unroll
    for (int u = 1; u < NW; ++u) mx = fmaxf(mx, red[0][u][l32]);
    float sum = 0.0f;
    for (int b = w; b < nb; b += NW)
        for (int r = hf; r < 32; r += 2) {
            const int i = 32 * b + r;
            const float e = qok ? expf(sc[i * P + l32] - mx) : 0.0f;  // exactly 0 outside the range
            sc[i * P + l32] = e;
            sum += e;
        }
    sum += __shfl_xor(sum, 32, 64);
    if (hf == 0) red[1][w][l32] = sum;
    __syncthreads();
    sum = red[1][0][l32];
#pragma unroll
    for (int u = 1; u < NW; ++u) sum += red[1][u][l32];  // in wave order
    for (int b = w; b < nb; b += NW)
        for (int r = hf; r < 32; r += 2) {
            const int i = 32 * b + r;
            sc[i * P + l32] = qok ? sc[i * P + l32] / sum : 0.0f;
        }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // the wave's probabilities, read by its lanes below
    __builtin_amdgcn_wave_barrier();
    // out^T[d][query] = sum over the wave's keys of v[key][d] p[query][key]; lane: dimension l32
    // of each 32-dimension block
    float16_t o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = float16_t{};
    auto load_v = [&](int b, float (&vv)[NDB][16]) {
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int j = lo + 32 * b + s + 16 * hf;
            if (j > hi) {
#pragma unroll
                for (int db = 0; db < NDB; ++db) vv[db][s] = 0.0f;
            } else if (j < start) {
                const half_t *vr = vcr + static_cast<int64_t>(j) * D + l32;
#pragma unroll
                for (int db = 0; db < NDB; ++db) vv[db][s] = static_cast<float>(vr[32 * db]);
            } else {
                const float *vr = vfr + static_cast<int64_t>(j - start) * D + l32;
#pragma unroll
                for (int db = 0; db < NDB; ++db) vv[db][s] = vr[32 * db];
            }
        }
    };
    auto pv_block = [&](int b, const float (&vv)[NDB][16]) {
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const float p = sc[(32 * b + s + 16 * hf) * P + l32];
#pragma unroll
            for (int db = 0; db < NDB; ++db) o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[db][s], p, o[db], 0, 0, 0);
        }
    };
    {
        float v0[NDB][16], v1[NDB][16];
        if (w < nb) load_v(w, v0);
        for (int b = w; b < nb; b += 2 * NW) {
            if (b + NW < nb) load_v(b + NW, v1);
            pv_block(b, v0);
            if (b + NW < nb) {
                if (b + 2 * NW < nb) load_v(b + 2 * NW, v0);
                pv_block(b + NW, v1);
            }
        }
    }
    // the other waves' partials to LDS once every wave is done with the probabilities; wave 0 adds
    // them in wave order
    __syncthreads();
    if (w > 0) {
        float *mine = sc + (w - 1) * D * 32;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int v = 0; v < 16; ++v) mine[(db * 16 + v) * 64 + lane] = o[db][v];
    }
    __syncthreads();
    if (w > 0 || !qok) return;
#pragma unroll
    for (int u = 1; u < NW; ++u) {
        const float *part = sc + (u - 1) * D * 32;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[db][v] = o[db][v] + part[(db * 16 + v) * 64 + lane];
    }
    half_t *dst = out + (static_cast<int64_t>(bi) * t + tq) * heads * D + h * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            half4_t r;
#pragma unroll
            for (int c = 0; c < 4; ++c) r[c] = static_cast<half_t>(o[db][4 * g + c]);
            *reinterpret_cast<half4_t *>(dst + 32 * db + 8 * g + 4 * hf) = r;
        }
}

// The largest key range of any 32-query block of a prefill (prefill_attention_mfma's LDS rows).
int prefill_block_keys(int t, int start, int window) {
    int most = 0;
    for (int ti0 = 0; ti0 < t; ti0 += 32) {
        const int nq = t - ti0 < 32 ? t - ti0 : 32;
        const int lo = window > 0 && start + ti0 + 1 > window ? start + ti0 + 1 - window : 0;
        const int n = start + ti0 + nq - lo;
        most = n > most ? n : most;
    }
    return most;
}

// Up to this many rows the prefill's projections run on the A-sharing kernel (its k ranges keep
// the weights streaming at decode's rate); past it, on the tile kernel.
constexpr int kPrefillMaxLdsRows = 128;

struct PrefillPlan {
    size_t h, a16, t16, qkv, q, kf, vf, p16, part, total;
    size_t part_bytes;
    int rows;
};

PrefillPlan prefill_plan_of(const dtts_stack_geometry &g, int64_t lanes, int64_t t) {
    PrefillPlan p{};
    const int64_t rows = lanes * t;
    const int64_t qw = g.heads * g.head_dim, kvw = g.n_kv * g.head_dim, qkvw = qw + 2 * kvw;
    const int64_t aw = g.dim > qw ? g.dim : qw;
    const int64_t pw = g.dim > 2 * g.ffn ? g.dim : 2 * g.ffn;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += align256(bytes);
        return at;
    };
    p.rows = static_cast<int>(rows);
    p.h = take(sizeof(float) * rows * g.dim);
    p.a16 = take(2 * rows * aw);
    p.t16 = take(2 * rows * g.ffn);
    // the QKV output, and at 49 .. 128 rows every projection's f32 output (one at a time)
    const int64_t fw = qkvw > pw ? qkvw : pw;
    p.qkv = take(sizeof(float) * rows * fw);
    p.q = take(sizeof(float) * rows * qw);
    p.kf = take(sizeof(float) * rows * kvw);
    p.vf = take(sizeof(float) * rows * kvw);
    p.p16 = take(2 * rows * pw);
    size_t gb = 0;
    if (rows <= kPrefillMaxLdsRows) {
        const int64_t shapes[5][3] = {
            {g.dim, qkvw, 0}, {qw, g.dim, 2}, {g.dim, 2 * g.ffn, 1}, {g.ffn, g.dim, 2}, {g.dim, 2 * g.ffn, 0}};
        for (const auto &sh : shapes) {
            const size_t v = lds_partial_bytes(
                pick_lds(static_cast<int>(rows), sh[0], sh[1], static_cast<int>(sh[2]), kPrefillMaxLdsRows), rows, sh[1]);
            gb = v > gb ? v : gb;
        }
    }
    p.part_bytes = gb;
    p.part = take(gb);
    p.total = off;
    return p;
}

// One projection of the prefill on the tile kernel: y16 [rows, n] = f16(a16 [rows, k] . w^T).
int prefill_gemm16(const half_t *a16, const half_t *w, half_t *y16, int rows, int k, int n, hipStream_t stream) {
    dtts_conv_desc d{};
    d.lanes = 1;
    d.len = rows;
    d.cin = k;
    d.cout = n;
    d.k = 1;
    d.dilation = 1;
    d.pad_left = 0;
    d.x = a16;
    d.w = w;
    d.y = y16;
    return dtts_conv1d_nlc_f16_ex(&d, stream);
}

#define PREFILL_STEP(expr)                                         \
    do {                                                           \
        const hipError_t e_ = (expr);                              \
        if (e_ != hipSuccess) {                                    \
            set_error("dtts_stack_prefill: %s", hipGetErrorString(e_)); \
            return DTTS_ERR_HIP;                                   \
        }                                                          \
    } while (0)
#define PREFILL_CALL(expr)               \
    do {                                 \
        const int rc_ = (expr);          \
        if (rc_ != DTTS_OK) return rc_;  \
    } while (0)

int enqueue_prefill(const dtts_stack &s, const float *x, float *out, const dtts_stack_cache *caches, int lanes, int t,
                    int start, int cap, char *ws, const PrefillPlan &pl, hipStream_t stream) {
    const dtts_stack_geometry &g = s.geo;
    const int dim = static_cast<int>(g.dim), hd = static_cast<int>(g.head_dim);
    const int heads = static_cast<int>(g.heads), n_kv = static_cast<int>(g.n_kv), ffn = static_cast<int>(g.ffn);
    const int qw = heads * hd, kvw = n_kv * hd, qkvw = qw + 2 * kvw;
    const int rows = lanes * t;
    float *h = reinterpret_cast<float *>(ws + pl.h);
    half_t *a16 = reinterpret_cast<half_t *>(ws + pl.a16);
    half_t *t16 = reinterpret_cast<half_t *>(ws + pl.t16);
    float *qkv = reinterpret_cast<float *>(ws + pl.qkv);
    float *q = reinterpret_cast<float *>(ws + pl.q);
    float *kf = reinterpret_cast<float *>(ws + pl.kf);
    float *vf = reinterpret_cast<float *>(ws + pl.vf);
    half_t *p16 = reinterpret_cast<half_t *>(ws + pl.p16);
    float *gpart = pl.part_bytes ? reinterpret_cast<float *>(ws + pl.part) : nullptr;
    // the layers without QK-norm scale the scores (qwen3.rs:311-316, 433-436)
    const float scale = g.qk_norm ? 1.0f : static_cast<float>(1.0 / std::sqrt(static_cast<double>(g.head_dim)));
    const bool sk_qkv = skinny_eligible(rows, dim, qkvw), sk_o = skinny_eligible(rows, qw, dim);
    const bool sk_gu = skinny_eligible(rows, dim, ffn), sk_d = skinny_eligible(rows, ffn, dim);
    // not skinny-eligible but few rows: the A-sharing kernel in f32, each consumer rounding the
    // summed output to f16 as the f16 matmul would
    const bool mid = rows <= kPrefillMaxLdsRows;
    constexpr int MM = kPrefillMaxLdsRows;
    const int keys = start + t;
    // queries per wave: 4 (2 at t = 2 or 3) while their scores fit, else 1
    const int qp = t >= 4 && (keys + hd) * 4 * 4 <= 65536 ? 4 : (t >= 2 && (keys + hd) * 4 * 2 <= 65536 ? 2 : 1);
    const int per_wave = (keys + hd) * 4 * qp;  // LDS bytes: the scores and the queries
    const int wpb = per_wave * 4 <= 65536 ? 4 : (per_wave * 2 <= 65536 ? 2 : 1);
    const int att_waves = lanes * ((t + qp - 1) / qp) * heads;
    // 32-query blocks on the matrix cores when there are enough queries and every block's keys
    // fit its LDS
    const size_t mfma_lds = static_cast<size_t>((prefill_block_keys(t, start, static_cast<int>(g.window)) + 31) / 32) *
                            32 * kPrefillMfmaPitch * sizeof(float);
    const size_t mfma_parts = static_cast<size_t>(kPrefillMfmaWaves - 1) * hd * 32 * sizeof(float);  // waves 1.. partials
    const size_t mfma_lds_launch = mfma_lds > mfma_parts ? mfma_lds : mfma_parts;
    // the whole workgroup's LDS within 64 KB: 14 key blocks (448 keys) at most
    const bool attn_mfma = t >= kPrefillMfmaMinT && (hd == 64 || hd == 128) &&
                           mfma_lds_launch + prefill_mfma_static_lds<kPrefillMfmaWaves>() <= kPrefillMfmaMaxLds;
    const unsigned mfma_blocks = static_cast<unsigned>(lanes * ((t + 31) / 32) * heads);
    Partials pending{};
    const half_t *pending16 = nullptr;
    bool pending_round = false;
    const float *pending_scale = nullptr;
    for (int64_t li = 0; li < g.layers; ++li) {
        const dtts_stack_layer &L = s.layers[li];
        half_t *kc = reinterpret_cast<half_t *>(caches[li].k);
        half_t *vc = reinterpret_cast<half_t *>(caches[li].v);
        PREFILL_STEP(launch_norm(li == 0 ? x : h, pending, pending_scale, h, L.attn_norm, a16, rows, dim, g.eps, stream,
                                 pending16, pending_round));
        const unsigned qk_blocks = static_cast<unsigned>((rows * (heads + n_kv) + 3) / 4);
        const float *norms = g.qk_norm ? L.qk_norms : nullptr;
        if (sk_qkv || mid) {
            Partials r{};
            PREFILL_STEP(stack_gemm<0>(a16, reinterpret_cast<const half_t *>(L.wqkv), qkv, nullptr, nullptr, rows, dim,
                                       qkvw, gpart, qkv, r, stream, MM));
            qk_rope_span_kernel<float><<<qk_blocks, 256, 0, stream>>>(r.p, norms, s.cos_t, s.sin_t, q, kf, vf, kc, vc, rows,
                                                                  t, start, heads, n_kv, hd, cap, g.eps, r.ys, r.stride,
                                                                  !sk_qkv);
        } else {
            half_t *qkv16 = reinterpret_cast<half_t *>(qkv);
            PREFILL_CALL(prefill_gemm16(a16, reinterpret_cast<const half_t *>(L.wqkv), qkv16, rows, dim, qkvw, stream));
            qk_rope_span_kernel<half_t><<<qk_blocks, 256, 0, stream>>>(qkv16, norms, s.cos_t, s.sin_t, q, kf, vf, kc, vc,
                                                                   rows, t, start, heads, n_kv, hd, cap, g.eps, 1, 0,
                                                                   false);
        }
        PREFILL_STEP(hipGetLastError());
        const unsigned at_blocks = static_cast<unsigned>((att_waves + wpb - 1) / wpb);
        const size_t lds = static_cast<size_t>(per_wave) * wpb;
#define DTTS_PREFILL_ATTN(D_, QP_)                                                                                   \
    prefill_attention<D_, QP_><<<at_blocks, 256, lds, stream>>>(q, kc, vc, kf, vf, a16, lanes, t, start, heads, n_kv, \
                                                                 cap, static_cast<int>(g.window), scale, keys, wpb)
        if (attn_mfma && hd == 128) {
            prefill_attention_mfma<128, kPrefillMfmaWaves><<<mfma_blocks, 64 * kPrefillMfmaWaves, mfma_lds_launch, stream>>>(
                q, kc, vc, kf, vf, a16, t, start, heads, n_kv, cap, static_cast<int>(g.window), scale);
        } else if (attn_mfma) {
            prefill_attention_mfma<64, kPrefillMfmaWaves><<<mfma_blocks, 64 * kPrefillMfmaWaves, mfma_lds_launch, stream>>>(
                q, kc, vc, kf, vf, a16, t, start, heads, n_kv, cap, static_cast<int>(g.window), scale);
        } else if (hd == 128) {
            if (qp == 4)
                DTTS_PREFILL_ATTN(128, 4);
            else if (qp == 2)
                DTTS_PREFILL_ATTN(128, 2);
            else
                DTTS_PREFILL_ATTN(128, 1);
        } else {
            if (qp == 4)
                DTTS_PREFILL_ATTN(64, 4);
            else if (qp == 2)
                DTTS_PREFILL_ATTN(64, 2);
            else
                DTTS_PREFILL_ATTN(64, 1);
        }
#undef DTTS_PREFILL_ATTN
        PREFILL_STEP(hipGetLastError());
        const float *attn_scale = g.layer_scale ? L.attn_scale : nullptr;
        Partials r{};
        const half_t *r16 = nullptr;
        if (sk_o) {
            PREFILL_STEP(stack_gemm<2>(a16, reinterpret_cast<const half_t *>(L.wo), h, nullptr, attn_scale, rows, qw, dim,
                                       gpart, nullptr, r, stream));
        } else if (mid) {
            PREFILL_STEP(stack_gemm<0>(a16, reinterpret_cast<const half_t *>(L.wo), qkv, nullptr, nullptr, rows, qw, dim,
                                       gpart, qkv, r, stream, MM));
        } else {
            PREFILL_CALL(prefill_gemm16(a16, reinterpret_cast<const half_t *>(L.wo), p16, rows, qw, dim, stream));
            r16 = p16;
        }
        PREFILL_STEP(launch_norm(h, r, attn_scale, h, L.ffn_norm, a16, rows, dim, g.eps, stream, r16, !sk_o && mid));
        if (sk_gu) {
            PREFILL_STEP(stack_gemm<1>(a16, reinterpret_cast<const half_t *>(L.w_gateup), nullptr, t16, nullptr, rows,
                                       dim, 2 * ffn, gpart, nullptr, r, stream));
            if (r.p) stack_gateup_merge<<<grid_for(int64_t(rows) * ffn / 4, 256, 4), 256, 0, stream>>>(r, t16, rows, ffn);
        } else if (mid) {
            PREFILL_STEP(stack_gemm<0>(a16, reinterpret_cast<const half_t *>(L.w_gateup), qkv, nullptr, nullptr, rows,
                                       dim, 2 * ffn, gpart, qkv, r, stream, MM));
            stack_gateup_merge<<<grid_for(int64_t(rows) * ffn / 4, 256, 4), 256, 0, stream>>>(r, t16, rows, ffn, true);
        } else {
            PREFILL_CALL(prefill_gemm16(a16, reinterpret_cast<const half_t *>(L.w_gateup), p16, rows, dim, 2 * ffn, stream));
            prefill_gateup_merge16<<<grid_for(int64_t(rows) * ffn / 4, 256, 4), 256, 0, stream>>>(p16, t16, rows, ffn);
        }
        PREFILL_STEP(hipGetLastError());
        const float *mlp_scale = g.layer_scale ? L.mlp_scale : nullptr;
        pending = Partials{};
        pending16 = nullptr;
        pending_round = false;
        if (sk_d) {
            PREFILL_STEP(stack_gemm<2>(t16, reinterpret_cast<const half_t *>(L.wdown), h, nullptr, mlp_scale, rows, ffn,
                                       dim, gpart, nullptr, pending, stream));
        } else if (mid) {
            PREFILL_STEP(stack_gemm<0>(t16, reinterpret_cast<const half_t *>(L.wdown), qkv, nullptr, nullptr, rows, ffn,
                                       dim, gpart, qkv, pending, stream, MM));
            pending_round = true;
        } else {
            PREFILL_CALL(prefill_gemm16(t16, reinterpret_cast<const half_t *>(L.wdown), p16, rows, ffn, dim, stream));
            pending16 = p16;
        }
        pending_scale = mlp_scale;
    }
    PREFILL_STEP(launch_norm(h, pending, pending_scale, static_cast<float *>(nullptr), s.final_norm, out, rows, dim,
                             g.eps, stream, pending16, pending_round));
    return DTTS_OK;
}

bool tiles_ok(int64_t k, int64_t n, int mode) { return pick_lds(kStackMaxLanes, k, n, mode).nc > 0; }

}  // namespace
}  // namespace dtts

using dtts::half_t;

extern "C" int dtts_stack_create(const dtts_stack_geometry *geo, const dtts_stack_layer *layers,
                                 const float *final_norm, dtts_stack **out) {
    return dtts_stack_create_as(geo, layers, final_norm, DTTS_WEIGHT_F16, out);
}

extern "C" int dtts_stack_create_as(const dtts_stack_geometry *geo, const dtts_stack_layer *layers,
                                    const float *final_norm, int32_t how, dtts_stack **out) {
    DTTS_REQUIRE(geo && layers && final_norm && out, "dtts_stack_create: null argument");
    *out = nullptr;
    DTTS_REQUIRE(how == DTTS_WEIGHT_F16 || how == DTTS_WEIGHT_F32 || how == DTTS_WEIGHT_Q8_0 ||
                     how == DTTS_WEIGHT_Q8_0_A32,
                 "dtts_stack_create: weight kind %d unknown", how);
    const dtts_stack_geometry &g = *geo;
    DTTS_REQUIRE(g.layers > 0 && g.dim > 0 && g.heads > 0 && g.n_kv > 0 && g.ffn > 0 && g.capacity > 0,
                 "dtts_stack_create: bad geometry (layers %lld, dim %lld, heads %lld, n_kv %lld, ffn %lld, "
                 "capacity %lld)",
                 (long long)g.layers, (long long)g.dim, (long long)g.heads, (long long)g.n_kv, (long long)g.ffn,
                 (long long)g.capacity);
    DTTS_REQUIRE(g.head_dim == 64 || g.head_dim == 128, "dtts_stack_create: head_dim %lld (64 or 128 supported)",
                 (long long)g.head_dim);
    DTTS_REQUIRE(g.heads % g.n_kv == 0, "dtts_stack_create: %lld heads over %lld kv heads", (long long)g.heads,
                 (long long)g.n_kv);
    const int64_t gqa = g.heads / g.n_kv;
    DTTS_REQUIRE(gqa == 1 || gqa == 2 || gqa == 4 || gqa == 8, "dtts_stack_create: gqa %lld (1, 2, 4 or 8)",
                 (long long)gqa);
    DTTS_REQUIRE(g.window >= 0 && g.eps >= 0.0f && g.rope_base > 0.0, "dtts_stack_create: bad window, eps or base");
    const int64_t qw = g.heads * g.head_dim, qkvw = (g.heads + 2 * g.n_kv) * g.head_dim;
    if (how == DTTS_WEIGHT_F16)
        DTTS_REQUIRE(dtts::tiles_ok(g.dim, qkvw, 0) && dtts::tiles_ok(qw, g.dim, 2) &&
                         dtts::tiles_ok(g.dim, 2 * g.ffn, 1) && dtts::tiles_ok(g.ffn, g.dim, 2),
                     "dtts_stack_create: projection shapes need dim, heads*head_dim and ffn multiples of 128");
    else
        DTTS_REQUIRE(dtts::proj_shape_ok(how, g.dim, qkvw) && dtts::proj_shape_ok(how, qw, g.dim) &&
                         dtts::proj_shape_ok(how, g.dim, 2 * g.ffn) && dtts::proj_shape_ok(how, g.ffn, g.dim),
                     "dtts_stack_create: projection shapes need dim, heads*head_dim and ffn multiples of %d",
                     how == DTTS_WEIGHT_F32 ? 64 : 256);
    DTTS_REQUIRE(g.dim % 4 == 0 && g.dim <= 8192, "dtts_stack_create: dim %lld (a multiple of 4, at most 8192)",
                 (long long)g.dim);
    DTTS_REQUIRE(g.capacity < (int64_t(1) << 24) && g.dim * g.ffn < (int64_t(1) << 31) && qkvw * g.dim < (int64_t(1) << 31),
                 "dtts_stack_create: geometry too large");
    for (int64_t i = 0; i < g.layers; ++i) {
        const dtts_stack_layer &L = layers[i];
        DTTS_REQUIRE(L.attn_norm && L.ffn_norm && L.wqkv && L.wo && L.w_gateup && L.wdown,
                     "dtts_stack_create: layer %lld incomplete", (long long)i);
        DTTS_REQUIRE(!g.qk_norm || L.qk_norms, "dtts_stack_create: layer %lld has no qk_norms", (long long)i);
        DTTS_REQUIRE(!g.layer_scale || (L.attn_scale && L.mlp_scale), "dtts_stack_create: layer %lld has no scales",
                     (long long)i);
        DTTS_REQUIRE(dtts::aligned(L.attn_norm, 16) && dtts::aligned(L.ffn_norm, 16),
                     "dtts_stack_create: layer %lld norm weights not 16-byte aligned", (long long)i);
        DTTS_REQUIRE(dtts::aligned(L.wqkv, 16) && dtts::aligned(L.wo, 16) && dtts::aligned(L.w_gateup, 16) &&
                         dtts::aligned(L.wdown, 16),
                     "dtts_stack_create: layer %lld projection weights not 16-byte aligned", (long long)i);
    }
    DTTS_REQUIRE(dtts::aligned(final_norm, 16), "dtts_stack_create: final norm weight not 16-byte aligned");
    dtts_stack *s = new (std::nothrow) dtts_stack();
    DTTS_REQUIRE(s, "dtts_stack_create: out of host memory");
    s->geo = g;
    s->how = how;
    s->layers.assign(layers, layers + g.layers);
    s->final_norm = final_norm;
    const int64_t half = g.head_dim / 2;
    std::vector<float> c(static_cast<size_t>(g.capacity * half)), sn(c.size());
    int rc = dtts_rope_table_f32(g.capacity, g.head_dim, g.rope_base, c.data(), sn.data());
    hipError_t e = hipSuccess;
    if (rc == DTTS_OK) {
        e = hipMalloc(&s->cos_t, sizeof(float) * c.size());
        if (e == hipSuccess) e = hipMalloc(&s->sin_t, sizeof(float) * c.size());
        if (e == hipSuccess) e = hipMalloc(&s->pos, sizeof(int32_t) * 256);
        if (e == hipSuccess) e = hipMemcpy(s->cos_t, c.data(), sizeof(float) * c.size(), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(s->sin_t, sn.data(), sizeof(float) * c.size(), hipMemcpyHostToDevice);
    }
    if (rc != DTTS_OK || e != hipSuccess) {
        dtts_stack_destroy(s);
        if (e != hipSuccess) dtts::set_error("dtts_stack_create: %s", hipGetErrorString(e));
        return rc != DTTS_OK ? rc : DTTS_ERR_HIP;
    }
    *out = s;
    return DTTS_OK;
}

extern "C" void dtts_stack_destroy(dtts_stack *s) {
    if (!s) return;
    if (s->exec) (void)hipGraphExecDestroy(s->exec);
    if (s->capture_stream) (void)hipStreamDestroy(s->capture_stream);
    if (s->cos_t) (void)hipFree(s->cos_t);
    if (s->sin_t) (void)hipFree(s->sin_t);
    if (s->pos) (void)hipFree(s->pos);
    delete s;
}

extern "C" size_t dtts_stack_workspace_bytes(const dtts_stack *s, int64_t lanes, int64_t cap) {
    if (!s || lanes <= 0 || lanes > dtts::kStackMaxLanes || cap <= 0) return 0;
    return dtts::step_bytes(*s, lanes, cap);
}

extern "C" int dtts_stack_decode(dtts_stack *s, const float *x, float *out, const dtts_stack_cache *caches,
                                 int64_t lanes, int64_t cap, const int32_t *pos, void *workspace, size_t ws_bytes,
                                 int32_t flags, hipStream_t stream) {
    const char *name = "dtts_stack_decode";
    DTTS_REQUIRE(s, "%s: null stack", name);
    DTTS_REQUIRE(lanes >= 0 && lanes <= dtts::kStackMaxLanes, "%s: %lld lanes (1 to %d)", name, (long long)lanes,
                 dtts::kStackMaxLanes);
    DTTS_REQUIRE((flags & ~DTTS_STACK_GRAPH) == 0, "%s: unknown flags 0x%x", name, static_cast<unsigned>(flags));
    if (lanes == 0) return DTTS_OK;
    const dtts_stack_geometry &g = s->geo;
    DTTS_REQUIRE(cap > 0 && cap <= g.capacity, "%s: cache capacity %lld outside (0, %lld] (the RoPE table)", name,
                 (long long)cap, (long long)g.capacity);
    DTTS_REQUIRE(lanes * g.n_kv * cap * g.head_dim < (int64_t(1) << 40), "%s: caches too large", name);
    DTTS_REQUIRE(x && out && caches && pos && workspace, "%s: null pointer", name);
    DTTS_REQUIRE(dtts::aligned(x, 16) && dtts::aligned(out, 16) && dtts::aligned(workspace, 256),
                 "%s: x and out must be 16-byte aligned, the workspace 256-byte aligned", name);
    for (int64_t i = 0; i < g.layers; ++i)
        DTTS_REQUIRE(caches[i].k && caches[i].v && dtts::aligned(caches[i].k, 16) && dtts::aligned(caches[i].v, 16),
                     "%s: layer %lld cache missing or misaligned", name, (long long)i);
    const size_t need = dtts::step_bytes(*s, lanes, cap);
    DTTS_REQUIRE(ws_bytes >= need, "%s: workspace %zu bytes < %zu needed", name, ws_bytes, need);
    dtts::Positions p{};
    for (int64_t i = 0; i < lanes; ++i) {
        // Stack::forward refuses start + t > capacity (crates/qwen3tts/src/qwen3.rs:303-309)
        DTTS_REQUIRE(pos[i] >= 0 && pos[i] < cap, "%s: lane %lld position %d exceeds cache capacity %lld", name,
                     (long long)i, pos[i], (long long)cap);
        p.p[i] = pos[i];
    }
    dtts::set_positions<<<1, 256, 0, stream>>>(p, s->pos, static_cast<int>(lanes));
    DTTS_LAUNCH_CHECK(name);
    char *ws = static_cast<char *>(workspace);
    if (!(flags & DTTS_STACK_GRAPH)) {
        DTTS_HIP_CHECK(dtts::enqueue_any(*s, x, out, caches, static_cast<int>(lanes), static_cast<int>(cap), ws, stream),
                       name);
        return DTTS_OK;
    }
    std::vector<const void *> key = {x, out, workspace, reinterpret_cast<const void *>(lanes),
                                     reinterpret_cast<const void *>(cap), reinterpret_cast<const void *>(ws_bytes)};
    for (int64_t i = 0; i < g.layers; ++i) {
        key.push_back(caches[i].k);
        key.push_back(caches[i].v);
    }
    if (!s->exec || key != s->key) {
        if (s->exec) {
            DTTS_HIP_CHECK(hipGraphExecDestroy(s->exec), name);
            s->exec = nullptr;
        }
        if (!s->capture_stream) DTTS_HIP_CHECK(hipStreamCreateWithFlags(&s->capture_stream, hipStreamNonBlocking), name);
        DTTS_HIP_CHECK(hipStreamBeginCapture(s->capture_stream, hipStreamCaptureModeThreadLocal), name);
        const hipError_t le =
            dtts::enqueue_any(*s, x, out, caches, static_cast<int>(lanes), static_cast<int>(cap), ws, s->capture_stream);
        hipGraph_t graph = nullptr;
        const hipError_t ee = hipStreamEndCapture(s->capture_stream, &graph);
        hipError_t ie = hipSuccess;
        if (le == hipSuccess && ee == hipSuccess) ie = hipGraphInstantiate(&s->exec, graph, nullptr, nullptr, 0);
        if (graph) (void)hipGraphDestroy(graph);
        DTTS_HIP_CHECK(le, name);
        DTTS_HIP_CHECK(ee, name);
        DTTS_HIP_CHECK(ie, name);
        s->key = key;
    }
    DTTS_HIP_CHECK(hipGraphLaunch(s->exec, stream), name);
    return DTTS_OK;
}

extern "C" size_t dtts_stack_prefill_workspace_bytes(const dtts_stack *s, int64_t lanes, int64_t t) {
    if (!s || s->how != DTTS_WEIGHT_F16 || lanes <= 0 || t < 2 || lanes * t > (int64_t(1) << 20)) return 0;
    return dtts::prefill_plan_of(s->geo, lanes, t).total;
}

extern "C" int dtts_stack_prefill(dtts_stack *s, const float *x, float *out, const dtts_stack_cache *caches,
                                  int64_t lanes, int64_t t, int64_t start, int64_t cap, void *workspace,
                                  size_t ws_bytes, hipStream_t stream) {
    const char *name = "dtts_stack_prefill";
    DTTS_REQUIRE(s, "%s: null stack", name);
    if (s->how != DTTS_WEIGHT_F16) {
        dtts::set_error("%s: the prefill branch runs f16 layers (this stack was made with weight kind %d)", name, s->how);
        return DTTS_ERR_UNSUPPORTED;
    }
    DTTS_REQUIRE(lanes >= 0 && t >= 2, "%s: %lld lanes, t = %lld (t >= 2; one position is dtts_stack_decode)", name,
                 (long long)lanes, (long long)t);
    if (lanes == 0) return DTTS_OK;
    const dtts_stack_geometry &g = s->geo;
    DTTS_REQUIRE(lanes * t <= (int64_t(1) << 20), "%s: %lld rows (at most 2^20)", name, (long long)(lanes * t));
    DTTS_REQUIRE(cap > 0 && cap <= g.capacity, "%s: cache capacity %lld outside (0, %lld] (the RoPE table)", name,
                 (long long)cap, (long long)g.capacity);
    // Stack::forward refuses start + t > capacity (crates/qwen3tts/src/qwen3.rs:303-309)
    DTTS_REQUIRE(start >= 0 && start + t <= cap, "%s: %lld positions exceeds cache capacity %lld", name,
                 (long long)(start + t), (long long)cap);
    DTTS_REQUIRE(start + t <= dtts::kPrefillMaxKeys, "%s: %lld positions (at most %d attended at once)", name,
                 (long long)(start + t), dtts::kPrefillMaxKeys);
    DTTS_REQUIRE(lanes * g.n_kv * cap * g.head_dim < (int64_t(1) << 40), "%s: caches too large", name);
    DTTS_REQUIRE(x && out && caches && workspace, "%s: null pointer", name);
    DTTS_REQUIRE(dtts::aligned(x, 16) && dtts::aligned(out, 16) && dtts::aligned(workspace, 256),
                 "%s: x and out must be 16-byte aligned, the workspace 256-byte aligned", name);
    for (int64_t i = 0; i < g.layers; ++i)
        DTTS_REQUIRE(caches[i].k && caches[i].v && dtts::aligned(caches[i].k, 16) && dtts::aligned(caches[i].v, 16),
                     "%s: layer %lld cache missing or misaligned", name, (long long)i);
    const dtts::PrefillPlan pl = dtts::prefill_plan_of(g, lanes, t);
    DTTS_REQUIRE(ws_bytes >= pl.total, "%s: workspace %zu bytes < %zu needed", name, ws_bytes, pl.total);
    return dtts::enqueue_prefill(*s, x, out, caches, static_cast<int>(lanes), static_cast<int>(t),
                                 static_cast<int>(start), static_cast<int>(cap), static_cast<char *>(workspace), pl,
                                 stream);
}
