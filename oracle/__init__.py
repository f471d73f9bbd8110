"""CPU oracle for the tts-nn fused-op hot path -- TEST INFRASTRUCTURE ONLY.

ctypes bindings over ``liboracle.so`` (built from ``oracle.c`` by ``make -C oracle``). Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
module, and only as the checker or the timed CPU baseline; the product library never does.

Every function here restates the reference's CPU arithmetic (drmhse/dream-tts ``crates/tts-nn``
on candle's CPU device); the C source names the reference file:line each one follows.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_I64 = ctypes.c_int64
_P = ctypes.c_void_p


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle not built: {_LIB_PATH} (run `make -C oracle`)")
        _lib = ctypes.CDLL(_LIB_PATH)
    return _lib


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _f64(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float64)


def _u16(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.uint16)


# ---------------------------------------------------------------- f16

def f32_to_f16(x):
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16_array(_ptr(x), _ptr(out), _I64(x.size))
    return out


def f16_to_f32(h):
    h = _u16(h)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_array(_ptr(h), _ptr(out), _I64(h.size))
    return out


# ---------------------------------------------------------------- snake

def snake_ncl_f32(x, alpha, brecip):
    x, a, r = _f32(x), _f32(alpha), _f32(brecip)
    lanes, c, l = x.shape
    y = np.empty_like(x)
    lib().or_snake_ncl_f32(_ptr(x), _ptr(a), _ptr(r), _ptr(y), _I64(lanes), _I64(c), _I64(l))
    return y


def snake_ncl_f16(x_bits, alpha, brecip):
    x, a, r = _u16(x_bits), _f32(alpha), _f32(brecip)
    lanes, c, l = x.shape
    y = np.empty_like(x)
    lib().or_snake_ncl_f16(_ptr(x), _ptr(a), _ptr(r), _ptr(y), _I64(lanes), _I64(c), _I64(l))
    return y


def snake_nlc_f32(x, alpha, brecip):
    x, a, r = _f32(x), _f32(alpha), _f32(brecip)
    c = x.shape[-1]
    y = np.empty_like(x)
    lib().or_snake_nlc_f32(_ptr(x), _ptr(a), _ptr(r), _ptr(y), _I64(x.size // c), _I64(c))
    return y


def snake_nlc_f16(x_bits, alpha, brecip):
    x, a, r = _u16(x_bits), _f32(alpha), _f32(brecip)
    c = x.shape[-1]
    y = np.empty_like(x)
    lib().or_snake_nlc_f16(_ptr(x), _ptr(a), _ptr(r), _ptr(y), _I64(x.size // c), _I64(c))
    return y


def snake_folded_f32(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().or_snake_folded_f32(_ptr(x), _ptr(y), _I64(x.size))
    return y


def snake_alpha_f32(x, alpha):
    x, a = _f32(x), _f32(alpha)
    lanes, c, l = x.shape
    y = np.empty_like(x)
    lib().or_snake_alpha_f32(_ptr(x), _ptr(a), _ptr(y), _I64(lanes), _I64(c), _I64(l))
    return y


def snake_nlc_f64(x, alpha, brecip):
    x, a, r = _f64(x), _f64(alpha), _f64(brecip)
    c = x.shape[-1]
    y = np.empty_like(x)
    lib().or_snake_nlc_f64(_ptr(x), _ptr(a), _ptr(r), _ptr(y), _I64(x.size // c), _I64(c))
    return y


# ---------------------------------------------------------------- im2col / weights

def im2col_tap_major_f32(x, k, dil, pad_left):
    x = _f32(x)
    cin, length = x.shape
    cols = np.empty((k * cin, length), np.float32)
    lib().or_im2col_tap_major_f32(_ptr(x), _ptr(cols), _I64(cin), _I64(length), _I64(k),
                                  _I64(dil), _I64(pad_left))
    return cols


def tap_weight_f32(w_oik):
    w = _f32(w_oik)
    cout, cin, k = w.shape
    out = np.empty((k, cin, cout), np.float32)
    lib().or_tap_weight_f32(_ptr(w), _ptr(out), _I64(cout), _I64(cin), _I64(k))
    return out


def tap_major_weight_f32(w_oik):
    w = _f32(w_oik)
    cout, cin, k = w.shape
    out = np.empty((cout, k * cin), np.float32)
    lib().or_tap_major_weight_f32(_ptr(w), _ptr(out), _I64(cout), _I64(cin), _I64(k))
    return out


def transpose_tap_weight_f32(w_iok, stride):
    w = _f32(w_iok)
    cin, cout, k = w.shape
    assert k % stride == 0
    out = np.empty((k // stride, cin, stride * cout), np.float32)
    lib().or_transpose_tap_weight_f32(_ptr(w), _ptr(out), _I64(cin), _I64(cout), _I64(k),
                                      _I64(stride))
    return out


def transpose_bias_f32(b, stride):
    b = _f32(b)
    out = np.empty((stride * b.size,), np.float32)
    lib().or_transpose_bias_f32(_ptr(b), _ptr(out), _I64(b.size), _I64(stride))
    return out


# ---------------------------------------------------------------- convs

def conv1d_nlc_f32(x, w_tap, bias, dil, pad_left=None, snake=None, res=None):
    """x [lanes, L, cin]; w_tap [k, cin, cout] (or [k*cin, cout]); causal when pad_left is None."""
    x, w = _f32(x), _f32(w_tap)
    lanes, length, cin = x.shape
    cout = w.shape[-1]
    k = w.size // (cin * cout)
    if pad_left is None:
        pad_left = (k - 1) * dil
    a, r = (None, None) if snake is None else (_f32(snake[0]), _f32(snake[1]))
    b, rs = _f32(bias), _f32(res)
    y = np.empty((lanes, length, cout), np.float32)
    lib().or_conv1d_nlc_f32(_ptr(x), _ptr(w), _ptr(b), _ptr(a), _ptr(r), _ptr(rs), _ptr(y),
                            _I64(lanes), _I64(length), _I64(cin), _I64(cout), _I64(k), _I64(dil),
                            _I64(pad_left))
    return y


def conv1d_nlc_f64(x, w_tap, bias, dil, pad_left=None, snake=None, res=None):
    x, w = _f64(x), _f64(w_tap)
    lanes, length, cin = x.shape
    cout = w.shape[-1]
    k = w.size // (cin * cout)
    if pad_left is None:
        pad_left = (k - 1) * dil
    a, r = (None, None) if snake is None else (_f64(snake[0]), _f64(snake[1]))
    b, rs = _f64(bias), _f64(res)
    y = np.empty((lanes, length, cout), np.float64)
    lib().or_conv1d_nlc_f64(_ptr(x), _ptr(w), _ptr(b), _ptr(a), _ptr(r), _ptr(rs), _ptr(y),
                            _I64(lanes), _I64(length), _I64(cin), _I64(cout), _I64(k), _I64(dil),
                            _I64(pad_left))
    return y


def conv1d_nlc_f16(x_bits, w_tap_bits, bias_bits, dil, pad_left=None, snake=None, res_bits=None,
                   act_tanh=False, act=None, scale=None):
    """f16 storage, f32 accumulation. act: None, "tanh" or "gelu" (act_tanh=True is "tanh");
    scale: f32 [cout] applied to (sum + bias) before the residual."""
    x, w = _u16(x_bits), _u16(w_tap_bits)
    lanes, length, cin = x.shape
    cout = w.shape[-1]
    k = w.size // (cin * cout)
    if pad_left is None:
        pad_left = (k - 1) * dil
    a, r = (None, None) if snake is None else (_f32(snake[0]), _f32(snake[1]))
    b, rs, sc = _u16(bias_bits), _u16(res_bits), _f32(scale)
    code = {None: 0, "tanh": 1, "gelu": 2, "clamp": 3}["tanh" if act_tanh else act]
    y = np.empty((lanes, length, cout), np.uint16)
    lib().or_conv1d_nlc_f16_ex(_ptr(x), _ptr(w), _ptr(b), _ptr(a), _ptr(r), _ptr(rs), _ptr(y),
                               _I64(lanes), _I64(length), _I64(cin), _I64(cout), _I64(k), _I64(dil),
                               _I64(pad_left), ctypes.c_int32(code), _ptr(sc))
    return y


def gelu_erf(x):
    """gelu_exact's formula in f32 with the C library's erf, elementwise over x (f32)."""
    x = _f32(x)
    f = lib().or_gelu_erf
    f.restype = ctypes.c_float
    f.argtypes = [ctypes.c_float]
    return np.array([f(float(v)) for v in x.ravel()], np.float32).reshape(x.shape)


def conv_transpose1d_causal_f64(x, w_iok, bias, stride):
    x, w = _f64(x), _f64(w_iok)
    length, cin = x.shape
    _, cout, k = w.shape
    b = _f64(bias)
    y = np.empty((length * stride, cout), np.float64)
    lib().or_conv_transpose1d_causal_f64(_ptr(x), _ptr(w), _ptr(b), _ptr(y), _I64(length),
                                         _I64(cin), _I64(cout), _I64(k), _I64(stride))
    return y


def sgemm(a, b):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    lib().or_sgemm(_ptr(a), _ptr(b), _ptr(c), _I64(m), _I64(n), _I64(k), ctypes.c_int32(0))
    return c


def conv1d_ncl_gemm_f32(x, w_tm, bias, k, dil, pad_left):
    x, w = _f32(x), _f32(w_tm)
    lanes, cin, length = x.shape
    cout = w.shape[0]
    b = _f32(bias)
    y = np.empty((lanes, cout, length), np.float32)
    lib().or_conv1d_ncl_gemm_f32(_ptr(x), _ptr(w), _ptr(b), _ptr(y), _I64(lanes), _I64(cin),
                                 _I64(cout), _I64(length), _I64(k), _I64(dil), _I64(pad_left))
    return y


def conv1d_nlc_cat_gemm_f32(x, w_tap, bias, dil):
    """One lane: x [L, cin], w_tap [k, cin, cout] -> [L, cout] (the reference's cat route)."""
    x, w = _f32(x), _f32(w_tap)
    length, cin = x.shape
    cout = w.shape[-1]
    k = w.size // (cin * cout)
    b = _f32(bias)
    y = np.empty((length, cout), np.float32)
    lib().or_conv1d_nlc_cat_gemm_f32(_ptr(x), _ptr(w), _ptr(b), _ptr(y), _I64(length), _I64(cin),
                                     _I64(cout), _I64(k), _I64(dil))
    return y


# ---------------------------------------------------------------- norm / rope / cache

def rms_norm_f32(x, gamma, eps):
    x, g = _f32(x), _f32(gamma)
    dim = x.shape[-1]
    y = np.empty_like(x)
    lib().or_rms_norm_f32(_ptr(x), _ptr(g), _ptr(y), _I64(x.size // dim), _I64(dim),
                          ctypes.c_float(eps))
    return y


def rms_norm_f16(x_bits, gamma_bits, eps):
    x, g = _u16(x_bits), _u16(gamma_bits)
    dim = x.shape[-1]
    y = np.empty_like(x)
    lib().or_rms_norm_f16(_ptr(x), _ptr(g), _ptr(y), _I64(x.size // dim), _I64(dim),
                          ctypes.c_float(eps))
    return y


def rms_norm_f64(x, gamma, eps):
    x, g = _f64(x), _f64(gamma)
    dim = x.shape[-1]
    y = np.empty_like(x)
    lib().or_rms_norm_f64(_ptr(x), _ptr(g), _ptr(y), _I64(x.size // dim), _I64(dim),
                          ctypes.c_double(eps))
    return y


def rope_table_f32(length, head_dim, base):
    c = np.empty((length, head_dim // 2), np.float32)
    s = np.empty((length, head_dim // 2), np.float32)
    lib().or_rope_table_f32(_I64(length), _I64(head_dim), ctypes.c_double(base), _ptr(c), _ptr(s))
    return c, s


def rope_halfsplit_f32(x, cos_t, sin_t, pos):
    x = _f32(x)
    rows, heads, hd = x.shape
    p = np.ascontiguousarray(pos, dtype=np.int32)
    y = np.empty_like(x)
    lib().or_rope_halfsplit_f32(_ptr(x), _ptr(_f32(cos_t)), _ptr(_f32(sin_t)), _ptr(p), _ptr(y),
                                _I64(rows), _I64(heads), _I64(hd))
    return y


def rope_halfsplit_f16(x_bits, cos_t, sin_t, pos):
    x = _u16(x_bits)
    rows, heads, hd = x.shape
    p = np.ascontiguousarray(pos, dtype=np.int32)
    y = np.empty_like(x)
    lib().or_rope_halfsplit_f16(_ptr(x), _ptr(_f32(cos_t)), _ptr(_f32(sin_t)), _ptr(p), _ptr(y),
                                _I64(rows), _I64(heads), _I64(hd))
    return y


def qk_norm_rope_append_f32(qkv, norms, cos_t, sin_t, pos, kcache, vcache, heads, n_kv, eps):
    """kcache/vcache (uint16 [b, n_kv, cap, D]) are updated in place; returns (q, k_f32)."""
    qkv = _f32(qkv)
    b = qkv.shape[0]
    hd = norms.shape[-1]
    cap = kcache.shape[2]
    p = np.ascontiguousarray(pos, dtype=np.int32)
    q = np.empty((b, heads, hd), np.float32)
    k = np.empty((b, n_kv, hd), np.float32)
    assert kcache.dtype == np.uint16 and kcache.flags["C_CONTIGUOUS"]
    lib().or_qk_norm_rope_append_f32(_ptr(qkv), _ptr(_f32(norms)), _ptr(_f32(cos_t)),
                                     _ptr(_f32(sin_t)), _ptr(p), _ptr(q), _ptr(k), _ptr(kcache),
                                     _ptr(vcache), _I64(b), _I64(heads), _I64(n_kv), _I64(hd),
                                     _I64(cap), ctypes.c_float(eps))
    return q, k


def qkrope_apply_f32(qkv, norms, cos_t, sin_t, kcache, vcache, heads, start, eps, f32_kv=True):
    """qkrope::apply's result as the composed CPU path computes it (crates/qwen3tts/src/qwen3.rs:
    358-394; the op's contract, crates/tts-nn/src/qkrope.rs:19-69): split q|k|v, rms_norm each
    head over D (candle: f32 sum of squares, (x / m) * w), heads first [b, h, t, D], half-split
    rope at positions start .. start + t - 1, then slice_set of f16(k) and f16(v) into the caches
    (uint16 [b, n_kv, cap, D], updated in place). Returns (q, (k, v) or None), all f32."""
    qkv = _f32(qkv)
    b, t, width = qkv.shape
    hd = norms.shape[-1]
    n_kv = (width // hd - heads) // 2
    cap = kcache.shape[2]
    assert start + t <= cap, f"{start + t} positions exceed {cap}"
    assert kcache.dtype == np.uint16 and kcache.flags["C_CONTIGUOUS"]
    x = qkv.reshape(b, t, heads + 2 * n_kv, hd)
    norms = _f32(norms)
    q = rms_norm_f32(x[:, :, :heads].reshape(-1, hd), norms[0], eps).reshape(b, t, heads, hd)
    k = rms_norm_f32(x[:, :, heads:heads + n_kv].reshape(-1, hd), norms[1], eps).reshape(b, t, n_kv, hd)
    v = np.ascontiguousarray(x[:, :, heads + n_kv:])
    pos = np.tile(start + np.arange(t, dtype=np.int32), b)  # row bi * t + ti sits at start + ti
    q = rope_halfsplit_f32(q.reshape(b * t, heads, hd), cos_t, sin_t, pos).reshape(b, t, heads, hd)
    k = rope_halfsplit_f32(k.reshape(b * t, n_kv, hd), cos_t, sin_t, pos).reshape(b, t, n_kv, hd)
    q, k, v = (np.ascontiguousarray(a.transpose(0, 2, 1, 3)) for a in (q, k, v))
    kcache[:, :, start:start + t] = f32_to_f16(k)
    vcache[:, :, start:start + t] = f32_to_f16(v)
    return q, ((k, v) if f32_kv else None)


def kv_append_f32(k, v, pos, kcache, vcache):
    k, v = _f32(k), _f32(v)
    b, n_kv, hd = k.shape
    p = np.ascontiguousarray(pos, dtype=np.int32)
    lib().or_kv_append_f32(_ptr(k), _ptr(v), _ptr(p), _ptr(kcache), _ptr(vcache), _I64(b),
                           _I64(n_kv), _I64(hd), _I64(kcache.shape[2]))


def kv_append_f16(k_bits, v_bits, pos, kcache, vcache):
    k, v = _u16(k_bits), _u16(v_bits)
    b, n_kv, hd = k.shape
    p = np.ascontiguousarray(pos, dtype=np.int32)
    lib().or_kv_append_f16(_ptr(k), _ptr(v), _ptr(p), _ptr(kcache), _ptr(vcache), _I64(b),
                           _I64(n_kv), _I64(hd), _I64(kcache.shape[2]))


# ---------------------------------------------------------------- GEMMs

def _stack_decode_dense(geo, layers, final_norm, x, kcaches, vcaches, pos, weight):
    """stack_decode_f32 for the f32 and Q8_0 weight kinds (f32 caches, f32 projections in and out,
    no f16 rounding anywhere), citing qwen3.rs line by line."""
    b = x.shape[0]
    hd, heads, n_kv = geo.head_dim, geo.heads, geo.n_kv
    qw, kvw = heads * hd, n_kv * hd
    pos = np.ascontiguousarray(np.broadcast_to(np.asarray(pos, np.int32), (b,)))
    cos_t, sin_t = rope_table_f32(geo.capacity, hd, geo.rope_base)  # Stack::load (qwen3.rs:240)
    span = pos + 1
    wstart = np.where(span > geo.window, span - geo.window, 0).astype(np.int32) if geo.window else np.zeros(b, np.int32)
    for c in list(kcaches) + list(vcaches):
        assert c.dtype == np.float32 and c.flags["C_CONTIGUOUS"], "f32 caches for this weight kind"
    h = _f32(x).copy()
    for li, L in enumerate(layers):
        normed = rms_norm_f32(h, L["attn_norm"], geo.eps)                             # :339
        qkv = _proj_as(normed, np.concatenate([L["wq"], L["wk"], L["wv"]], axis=0), weight)  # :340, :69-77
        q = qkv[:, :qw].reshape(b, heads, hd)                                         # :358-364
        k = qkv[:, qw:qw + kvw].reshape(b, n_kv, hd)
        v = qkv[:, qw + kvw:].reshape(b, n_kv, hd)
        if geo.qk_norm:                                                               # :369-376
            s = np.float32(1.0 / np.sqrt(np.float64(hd)))
            q = rms_norm_f32(q, _f32(L["q_norm"]) * s, geo.eps)                       # :78-91 (folded)
            k = rms_norm_f32(k, _f32(L["k_norm"]), geo.eps)
        q = rope_halfsplit_f32(q, cos_t, sin_t, pos)                                  # :381-387
        k = rope_halfsplit_f32(k, cos_t, sin_t, pos)
        for i in range(b):                                                            # :391-392 (slice_set, f32)
            kcaches[li][i, :, pos[i]] = k[i]
            vcaches[li][i, :, pos[i]] = v[i]
        if not geo.qk_norm:
            q = q * np.float32(1.0 / np.sqrt(np.float64(hd)))                         # :404-408
        attn = decode_attention_f32(q.reshape(b, n_kv, heads // n_kv, hd), kcaches[li], vcaches[li],
                                    span, wstart).reshape(b, qw)                      # :413-414
        o = _proj_as(attn, L["wo"], weight)                                           # :446
        if geo.layer_scale:
            o = o * _f32(L["attn_scale"])                                             # :447-450
        h = h + o                                                                     # :451
        normed = rms_norm_f32(h, L["ffn_norm"], geo.eps)                              # :453
        tail = swiglu_mul_f32(_proj_as(normed, L["gate"], weight), _proj_as(normed, L["up"], weight))  # :454-457
        mlp = _proj_as(tail, L["down"], weight)                                       # :458
        if geo.layer_scale:
            mlp = mlp * _f32(L["mlp_scale"])                                          # :459-462
        h = h + mlp                                                                   # :463
    return rms_norm_f32(h, final_norm, geo.eps)                                       # :466


def decode_attention_f32(q, k, v, span, window_start=0):
    """attn::decode_attention's CPU path (crates/tts-nn/src/attn.rs:18-73, 85-126, 189-226).
    q [b, n_kv, gqa, D] f32; caches [b, n_kv, cap, D] as f16 bit patterns (uint16) or f32; span
    and window_start one int or one per lane. Returns [b, n_kv, gqa, D] f32."""
    q = _f32(q)
    b, n_kv, gqa, hd = q.shape
    kv_f16 = 1 if np.asarray(k).dtype == np.uint16 else 0
    k = _u16(k) if kv_f16 else _f32(k)
    v = _u16(v) if kv_f16 else _f32(v)
    sp = np.ascontiguousarray(np.broadcast_to(np.asarray(span, np.int32), (b,)))
    ws = np.ascontiguousarray(np.broadcast_to(np.asarray(window_start, np.int32), (b,)))
    out = np.empty_like(q)
    lib().or_decode_attention_f32(_ptr(q), _ptr(k), _ptr(v), ctypes.c_int(kv_f16), _ptr(out), _I64(b), _I64(n_kv),
                                  _I64(gqa), _I64(hd), _I64(k.shape[2]), _ptr(sp), _ptr(ws))
    return out


def gemm_f16_f32acc(a_bits, b_kn_bits):
    a, b = _u16(a_bits), _u16(b_kn_bits)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float32)
    lib().or_gemm_f16_f32acc(_ptr(a), _ptr(b), _ptr(c), _I64(m), _I64(k), _I64(n))
    return c


def gemm_f16_f64(a_bits, b_kn_bits):
    a, b = _u16(a_bits), _u16(b_kn_bits)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), np.float64)
    lib().or_gemm_f16_f64(_ptr(a), _ptr(b), _ptr(c), _I64(m), _I64(k), _I64(n))
    return c


def swiglu_mul_f32(g, u):
    g, u = _f32(g), _f32(u)
    y = np.empty_like(g)
    lib().or_swiglu_mul_f32(_ptr(g), _ptr(u), _ptr(y), _I64(g.size))
    return y


# ---------------------------------------------------------------- codec front half

def rvq_lookup_sum_f16(codes, books, n_first):
    """codes [rows, n_books] int32, books [n_books, size, dim] f32 -> [rows, 2*dim] f16 bits."""
    codes = np.ascontiguousarray(codes, np.int32)
    books = _f32(books)
    rows, n_books = codes.shape
    _, size, dim = books.shape
    out = np.empty((rows, 2 * dim), np.uint16)
    lib().or_rvq_lookup_sum_f16(_ptr(codes), _ptr(books), _I64(n_books), _I64(n_first), _I64(size), _I64(dim),
                                _ptr(out), _I64(rows))
    return out


def depthwise_layernorm_f16(x_bits, taps, bias, ln_w, ln_b, eps):
    """x [lanes, L, C] f16 bits; taps [C, K] f32 -> [lanes, L, C] f16 bits."""
    x = _u16(x_bits)
    lanes, length, c = x.shape
    taps = _f32(taps)
    y = np.empty_like(x)
    lib().or_depthwise_layernorm_f16(_ptr(x), _ptr(taps), _ptr(_f32(bias)), _ptr(_f32(ln_w)), _ptr(_f32(ln_b)),
                                     ctypes.c_float(eps), _ptr(y), _I64(lanes), _I64(length), _I64(c),
                                     _I64(taps.shape[1]))
    return y


def window_attention_prefill_f16(qkv_bits, cos_t, sin_t, heads, n_kv, head_dim, window, scale):
    """qkv [lanes, T, (heads + 2 n_kv) D] f16 bits -> [lanes, T, heads D] f16 bits."""
    qkv = _u16(qkv_bits)
    lanes, length, _ = qkv.shape
    out = np.empty((lanes, length, heads * head_dim), np.uint16)
    lib().or_window_attention_prefill_f16(_ptr(qkv), _ptr(_f32(cos_t)), _ptr(_f32(sin_t)), _ptr(out), _I64(lanes),
                                          _I64(length), _I64(heads), _I64(n_kv), _I64(head_dim), _I64(window),
                                          ctypes.c_float(scale))
    return out


def rms_norm_rows_f16(x_bits, gamma, eps):
    x = _u16(x_bits)
    dim = x.shape[-1]
    y = np.empty_like(x)
    lib().or_rms_norm_rows_f16(_ptr(x), _ptr(_f32(gamma)), _ptr(y), _I64(x.size // dim), _I64(dim), ctypes.c_float(eps))
    return y


def swiglu_rows_f16(gu_bits):
    gu = _u16(gu_bits)
    ffn = gu.shape[-1] // 2
    y = np.empty(gu.shape[:-1] + (ffn,), np.uint16)
    lib().or_swiglu_rows_f16(_ptr(gu), _ptr(y), _I64(gu.size // (2 * ffn)), _I64(ffn))
    return y


# ---------------------------------------------------------------- decoder stack step

def _proj_f16(x, w_out_in):
    """Proj::Half's forward on the decode path (crates/tts-nn/src/lib.rs:514-524): x cast to f16,
    times the f16 weight, f32 accumulation and output. w is [out, in] f32 (rounded to f16 here)."""
    return gemm_f16_f32acc(f32_to_f16(x), np.ascontiguousarray(f32_to_f16(w_out_in).T))


def _skinny_eligible(m, k, n):
    """skinny::eligible (crates/tts-nn/src/skinny.rs:123-131, MAX_M = 48 at :152): the shapes
    Proj::Half sends to the skinny GEMM (f32 output); every other shape goes through candle's f16
    matmul, whose output is f16 (lib.rs:516-529)."""
    return m <= 48 and m % 8 == 0 and k % 32 == 0 and n % 64 == 0


def _proj_half(x, w_out_in):
    """Proj::Half's forward at any row count (crates/tts-nn/src/lib.rs:514-529): the skinny GEMM's
    f32 result for eligible shapes, else the f16 matmul's output (f32 accumulation, rounded once
    to f16) widened back to f32."""
    y = _proj_f16(x, w_out_in)
    m, k = x.shape
    return y if _skinny_eligible(m, k, w_out_in.shape[0]) else f16_to_f32(f32_to_f16(y))


STACK_WEIGHTS = ("f16", "f32", "q8_0", "q8_0_a32")


def _proj_as(x, w_out_in, weight):
    """Proj::forward for each weight kind (crates/tts-nn/src/lib.rs:509-531), f32 in and out:
    f16 -> Proj::Half's routing; f32 -> Proj::Dense's f32 GEMM (matmul_2d, lib.rs:438-459),
    evaluated in float64 and rounded once; q8_0 -> QMatMul on the Q8_0 blocks of the weight
    (QTensor::quantize_onto, lib.rs:480-486) with the f32 activations quantized per block
    (candle CPU's vec_dot, q8_0_matmul_w8a8); q8_0_a32 -> the same blocks times the unquantized
    f32 activations (float64, rounded once)."""
    if weight == "f16":
        return _proj_half(x, w_out_in)
    x = _f32(x)
    if weight == "f32":
        return (x.astype(np.float64) @ _f32(w_out_in).astype(np.float64).T).astype(np.float32)
    blocks = q8_0_quantize(_f32(w_out_in))
    if weight == "q8_0":
        return q8_0_matmul_w8a8(x, blocks)
    if weight == "q8_0_a32":
        return q8_0_matmul_f64(x, blocks).astype(np.float32)
    raise ValueError(f"weight kind {weight!r}")


def stack_decode_f32(geo, layers, final_norm, x, kcaches, vcaches, pos, weight="f16"):
    """Stack::forward at t = 1 (crates/qwen3tts/src/qwen3.rs:294-467) with f16 weights and f16
    caches, each lane at its own position; the projections follow Proj::Half's routing by lane
    count (f32 outputs for 8, 16, .. 48 lanes, f16 outputs otherwise, one lane included). geo: an object with the Geometry fields (dim, layers,
    heads, n_kv, head_dim, ffn, eps, rope_base, qk_norm, layer_scale, window, capacity); layers:
    dicts of checkpoint-layout f32 weights (wq, wk, wv, wo, gate, up, down [out, in]; attn_norm,
    ffn_norm; q_norm, k_norm; attn_scale, mlp_scale); x [b, dim] f32; kcaches / vcaches: per
    layer uint16 [b, n_kv, cap, head_dim], updated in place; pos int32[b]. Returns the final
    rms_norm of the residual stream, [b, dim] f32.

    weight: Stack::load's `how` (qwen3.rs:228-250), one of STACK_WEIGHTS. Every kind but f16 keeps
    f32 caches (kcaches / vcaches float32 arrays, qwen3.rs:242-246), which qkrope::eligible refuses
    (qkrope.rs:11-18), so its step takes the composed route (qwen3.rs:358-400): rms_norm over each
    head with the folded norms, rope, and the f32 k and v set into the caches as they are."""
    if weight != "f16":
        return _stack_decode_dense(geo, layers, final_norm, x, kcaches, vcaches, pos, weight)
    b = x.shape[0]
    hd, heads, n_kv = geo.head_dim, geo.heads, geo.n_kv
    qw, kvw = heads * hd, n_kv * hd
    pos = np.ascontiguousarray(np.broadcast_to(np.asarray(pos, np.int32), (b,)))
    cos_t, sin_t = rope_table_f32(geo.capacity, hd, geo.rope_base)  # Stack::load (qwen3.rs:240)
    span = pos + 1
    # the window start of the decode branch (qwen3.rs:409-412)
    wstart = np.where(span > geo.window, span - geo.window, 0).astype(np.int32) if geo.window else np.zeros(b, np.int32)
    h = _f32(x).copy()
    for li, L in enumerate(layers):
        normed = rms_norm_f32(h, L["attn_norm"], geo.eps)                             # :339
        qkv = _proj_half(normed, np.concatenate([L["wq"], L["wk"], L["wv"]], axis=0))  # :340, :69-77
        if geo.qk_norm:                                                               # :343-357
            s = np.float32(1.0 / np.sqrt(np.float64(hd)))
            norms = np.stack([_f32(L["q_norm"]) * s, _f32(L["k_norm"])])              # :78-91
            q, _ = qk_norm_rope_append_f32(qkv, norms, cos_t, sin_t, pos, kcaches[li], vcaches[li],
                                           heads, n_kv, geo.eps)
        else:                                                                         # :358-400
            q = rope_halfsplit_f32(qkv[:, :qw].reshape(b, heads, hd), cos_t, sin_t, pos)
            k = rope_halfsplit_f32(qkv[:, qw:qw + kvw].reshape(b, n_kv, hd), cos_t, sin_t, pos)
            kv_append_f32(k, qkv[:, qw + kvw:].reshape(b, n_kv, hd), pos, kcaches[li], vcaches[li])
            q = q * np.float32(1.0 / np.sqrt(np.float64(hd)))                         # :404-408
        attn = decode_attention_f32(q.reshape(b, n_kv, heads // n_kv, hd), kcaches[li], vcaches[li],
                                    span, wstart).reshape(b, qw)                      # :413-414
        o = _proj_half(attn, L["wo"])                                                 # :446
        if geo.layer_scale:
            o = o * _f32(L["attn_scale"])                                             # :447-450
        h = h + o                                                                     # :451
        normed = rms_norm_f32(h, L["ffn_norm"], geo.eps)                              # :453
        tail = swiglu_mul_f32(_proj_half(normed, L["gate"]), _proj_half(normed, L["up"]))  # :454-457
        mlp = _proj_half(tail, L["down"])                                             # :458
        if geo.layer_scale:
            mlp = mlp * _f32(L["mlp_scale"])                                          # :459-462
        h = h + mlp                                                                   # :463
    return rms_norm_f32(h, final_norm, geo.eps)                                       # :466


def prefill_attention_f32(q, k_all, v_all, start, window, scale):
    """The prefill branch's attention (crates/qwen3tts/src/qwen3.rs:415-444): q [b, heads, t, D]
    f32, k_all / v_all [b, n_kv, start + t, D] f32 (the cache's prefix widened, then the new
    positions' own f32 k and v); query heads sharing a kv head stacked along rows; scores scaled
    by `scale` (None when folded into q_norm), plus causal_window_mask(start + t, window) rows
    start .. start + t - 1 (lib.rs:1210-1224); softmax_last_dim; probs . v. Returns
    [b, t, heads * D] f32."""
    q, k_all, v_all = _f32(q), _f32(k_all), _f32(v_all)
    b, heads, t, hd = q.shape
    n_kv, n = k_all.shape[1], k_all.shape[2]
    assert n == start + t
    gqa = heads // n_kv
    rows = np.arange(start, start + t)[:, None]
    cols = np.arange(n)[None, :]
    lo = np.maximum(rows + 1 - window, 0) if window else np.zeros_like(rows)
    mask = np.where((cols > rows) | (cols < lo), np.float32(-np.inf), np.float32(0.0)).astype(np.float32)
    mask = np.concatenate([mask] * gqa, axis=0)                                      # [gqa * t, n]
    qg = q.reshape(b, n_kv, gqa * t, hd)
    scores = np.matmul(qg, np.swapaxes(k_all, -1, -2)).astype(np.float32)
    if scale is not None:
        scores = (scores * np.float32(scale)).astype(np.float32)
    scores = scores + mask
    e = np.exp(scores - scores.max(-1, keepdims=True)).astype(np.float32)
    probs = (e / e.sum(-1, keepdims=True)).astype(np.float32)
    out = np.matmul(probs, v_all).astype(np.float32)                                 # [b, n_kv, gqa*t, D]
    return out.reshape(b, heads, t, hd).transpose(0, 2, 1, 3).reshape(b, t, heads * hd)


def stack_prefill_f32(geo, layers, final_norm, x, kcaches, vcaches, start):
    """Stack::forward at t >= 2 (crates/qwen3tts/src/qwen3.rs:294-467, the prefill branch) for a
    batch that shares `start`: x [b, t, dim] f32; kcaches / vcaches per layer uint16
    [b, n_kv, cap, D], written at start .. start + t - 1 in place and read below start. The
    projections follow Proj::Half's routing by row count (b * t rows); the new positions attend
    over their own f32 k and v and the cache's f16 prefix. Returns [b, t, dim] f32."""
    b, t, dim = x.shape
    rows = b * t
    hd, heads, n_kv = geo.head_dim, geo.heads, geo.n_kv
    qw, kvw = heads * hd, n_kv * hd
    cos_t, sin_t = rope_table_f32(geo.capacity, hd, geo.rope_base)
    scale = None if geo.qk_norm else float(1.0 / np.sqrt(np.float64(hd)))          # :311-316
    h = _f32(x).reshape(rows, dim).copy()
    for li, L in enumerate(layers):
        normed = rms_norm_f32(h, L["attn_norm"], geo.eps)                             # :339
        qkv = _proj_half(normed, np.concatenate([L["wq"], L["wk"], L["wv"]], axis=0)).reshape(b, t, -1)
        q = np.empty((b, heads, t, hd), np.float32)
        kf = np.empty((b, n_kv, t, hd), np.float32)
        vf = np.ascontiguousarray(qkv[:, :, qw + kvw:].reshape(b, t, n_kv, hd).transpose(0, 2, 1, 3))
        for ti in range(t):                          # qkrope::apply with f32_kv (qkrope.rs:26-69)
            pos = np.full(b, start + ti, np.int32)
            row = np.ascontiguousarray(qkv[:, ti])
            if geo.qk_norm:
                s = np.float32(1.0 / np.sqrt(np.float64(hd)))
                norms = np.stack([_f32(L["q_norm"]) * s, _f32(L["k_norm"])])
                q[:, :, ti], kf[:, :, ti] = qk_norm_rope_append_f32(row, norms, cos_t, sin_t, pos, kcaches[li],
                                                                    vcaches[li], heads, n_kv, geo.eps)
            else:                                                                     # :358-394
                q[:, :, ti] = rope_halfsplit_f32(row[:, :qw].reshape(b, heads, hd), cos_t, sin_t, pos)
                kf[:, :, ti] = rope_halfsplit_f32(row[:, qw:qw + kvw].reshape(b, n_kv, hd), cos_t, sin_t, pos)
                kv_append_f32(kf[:, :, ti], vf[:, :, ti], pos, kcaches[li], vcaches[li])
        prior = lambda c: f16_to_f32(c[:, :, :start])                                 # :425-431
        k_all = np.concatenate([prior(kcaches[li]), kf], axis=2)
        v_all = np.concatenate([prior(vcaches[li]), vf], axis=2)
        attn = prefill_attention_f32(q, k_all, v_all, start, geo.window, scale).reshape(rows, qw)
        o = _proj_half(attn, L["wo"])                                                 # :446
        if geo.layer_scale:
            o = o * _f32(L["attn_scale"])
        h = h + o
        normed = rms_norm_f32(h, L["ffn_norm"], geo.eps)                              # :453
        tail = swiglu_mul_f32(_proj_half(normed, L["gate"]), _proj_half(normed, L["up"]))
        mlp = _proj_half(tail, L["down"])                                             # :458
        if geo.layer_scale:
            mlp = mlp * _f32(L["mlp_scale"])
        h = h + mlp
    return rms_norm_f32(h, final_norm, geo.eps).reshape(b, t, dim)                    # :466


def q8_0_quantize(w):
    w = _f32(w)
    rows, k = w.shape
    out = np.empty((rows, k // 32, 34), np.uint8)
    lib().or_q8_0_quantize(_ptr(w), _ptr(out), _I64(rows), _I64(k))
    return out


def q8_0_dequantize(blocks, k):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    rows = blocks.shape[0]
    w = np.empty((rows, k), np.float32)
    lib().or_q8_0_dequantize(_ptr(blocks), _ptr(w), _I64(rows), _I64(k))
    return w


def q8_0_matmul_w8a8(x, blocks):
    x = _f32(x)
    m, k = x.shape
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.shape[0]
    y = np.empty((m, n), np.float32)
    lib().or_q8_0_matmul_w8a8(_ptr(x), _ptr(blocks), _ptr(y), _I64(m), _I64(k), _I64(n))
    return y


def q8_0_matmul_f64(x, blocks):
    x = _f32(x)
    m, k = x.shape
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.shape[0]
    y = np.empty((m, n), np.float64)
    lib().or_q8_0_matmul_f64(_ptr(x), _ptr(blocks), _ptr(y), _I64(m), _I64(k), _I64(n))
    return y


# ---------------------------------------------------------------- metric

def abs_and_rel(a, b):
    a, b = _f32(a), _f32(b)
    assert a.size == b.size
    ab, rl = ctypes.c_float(), ctypes.c_float()
    lib().or_abs_and_rel(_ptr(a), _ptr(b), _I64(a.size), ctypes.byref(ab), ctypes.byref(rl))
    return float(ab.value), float(rl.value)
