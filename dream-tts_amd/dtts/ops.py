"""tts-nn's op surface over libdtts, on torch device tensors.

Each function keeps the reference function's name and argument meaning (drmhse/dream-tts,
crates/tts-nn) and, like the reference's CustomOps, allocates its output. The C ABI underneath
is what a Rust shim binds; this layer is the tests' and the bench's way in. Nothing here
computes: every op is one or more libdtts kernel launches on the current stream.
"""
from __future__ import annotations

import torch

from ._lib import DttsError, call, ptr, stream_handle

_F16 = torch.float16
_F32 = torch.float32


def _check(t, name, dtypes, what):
    if not isinstance(t, torch.Tensor):
        raise DttsError(f"{name}: {what} must be a tensor")
    if not t.is_cuda:
        raise DttsError(f"{name}: {what} must be on the device")
    if t.dtype not in dtypes:
        raise DttsError(f"{name}: {what} dtype {t.dtype} not in {dtypes}")
    if not t.is_contiguous():
        raise DttsError(f"{name}: {what} must be contiguous")


def _params(name, alpha, beta_recip, chan):
    for t, w in ((alpha, "alpha"), (beta_recip, "beta_recip")):
        _check(t, name, (_F32,), w)
        if t.numel() != chan:
            raise DttsError(f"{name}: {w} has {t.numel()} elements for {chan} channels")


# ---------------------------------------------------------------- a1/a2 snake

def snake_beta(x, alpha, beta_recip, out=None):
    """`x + beta_recip[c] * sin^2(alpha[c] * x)` over NCL `[lanes, C, L]`.

    crates/tts-nn/src/fused.rs:665-681 (SnakeBeta, batch 1 there; any lane count here)."""
    _check(x, "snake_beta", (_F32, _F16), "x")
    if x.dim() != 3:
        raise DttsError(f"snake_beta: x must be [lanes, C, L], got {tuple(x.shape)}")
    lanes, c, length = x.shape
    _params("snake_beta", alpha, beta_recip, c)
    y = torch.empty_like(x) if out is None else out
    fn = "dtts_snake_ncl_f32" if x.dtype == _F32 else "dtts_snake_ncl_f16"
    call(fn, ptr(x), ptr(alpha), ptr(beta_recip), ptr(y), lanes, c, length, stream_handle())
    return y


def snake_beta_nlc(x, alpha, beta_recip, out=None):
    """The same over channels-last `[..., C]`. crates/tts-nn/src/fused.rs:526-551."""
    _check(x, "snake_beta_nlc", (_F32, _F16), "x")
    c = x.shape[-1]
    _params("snake_beta_nlc", alpha, beta_recip, c)
    y = torch.empty_like(x) if out is None else out
    fn = "dtts_snake_nlc_f32" if x.dtype == _F32 else "dtts_snake_nlc_f16"
    call(fn, ptr(x), ptr(alpha), ptr(beta_recip), ptr(y), x.numel() // max(c, 1), c, stream_handle())
    return y


# ---------------------------------------------------------------- a8-a11 norm, RoPE, KV cache

def _pos_array(pos, n, name):
    import ctypes

    import numpy as np

    p = np.ascontiguousarray(np.asarray(pos, dtype=np.int32).reshape(-1))
    if p.size != n:
        raise DttsError(f"{name}: {p.size} positions for {n} lanes")
    return p, ctypes.c_void_p(p.ctypes.data)


def rms_norm(x, gamma, eps, out=None):
    """crates/tts-nn/src/lib.rs:1000-1003 (candle_nn::ops::rms_norm), over the last dim."""
    _check(x, "rms_norm", (_F32, _F16), "x")
    _check(gamma, "rms_norm", (x.dtype,), "gamma")
    dim = x.shape[-1]
    if gamma.numel() != dim:
        raise DttsError(f"rms_norm: gamma has {gamma.numel()} elements for dim {dim}")
    y = torch.empty_like(x) if out is None else out
    fn = "dtts_rms_norm_f32" if x.dtype == _F32 else "dtts_rms_norm_f16"
    call(fn, ptr(x), ptr(gamma), ptr(y), x.numel() // dim, dim, float(eps), stream_handle())
    return y


def rope_table_f32(length, head_dim, base):
    """crates/tts-nn/src/lib.rs:1192-1205 on the host: (cos, sin) numpy f32 [length, D/2]."""
    import ctypes

    import numpy as np

    c = np.empty((length, head_dim // 2), np.float32)
    s = np.empty((length, head_dim // 2), np.float32)
    call("dtts_rope_table_f32", length, head_dim, float(base), ctypes.c_void_p(c.ctypes.data),
         ctypes.c_void_p(s.ctypes.data))
    return c, s


def rope(x, cos, sin, pos, out=None):
    """Half-split RoPE on [rows, heads, D] with a position per row (host ints)."""
    _check(x, "rope", (_F32, _F16), "x")
    for t, w in ((cos, "cos"), (sin, "sin")):
        _check(t, "rope", (_F32,), w)
    rows, heads, hd = x.shape
    p, pp = _pos_array(pos, rows, "rope")
    y = torch.empty_like(x) if out is None else out
    fn = "dtts_rope_halfsplit_f32" if x.dtype == _F32 else "dtts_rope_halfsplit_f16"
    call(fn, ptr(x), ptr(cos), ptr(sin), pp, ptr(y), rows, heads, hd, cos.shape[0], stream_handle())
    return y


def qk_norm_rope_kv_append(qkv, norms, cos, sin, pos, k_cache, v_cache, heads, eps, f32_k=False):
    """qkrope::apply (crates/tts-nn/src/qkrope.rs:26-69) for one position per lane.

    qkv [b, (heads + 2*n_kv) * D]; caches [b, n_kv, cap, D] f16, updated in place. Returns q
    [b, heads, D] (qkv's dtype) and, with f32_k, the roped k [b, n_kv, D] f32."""
    _check(qkv, "qk_norm_rope_kv_append", (_F32, _F16), "qkv")
    _check(norms, "qk_norm_rope_kv_append", (_F32,), "norms")
    for t, w in ((cos, "cos"), (sin, "sin")):
        _check(t, "qk_norm_rope_kv_append", (_F32,), w)
    for t, w in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        _check(t, "qk_norm_rope_kv_append", (_F16,), w)
    b = qkv.shape[0]
    _, n_kv, cap, hd = k_cache.shape
    if qkv.shape[-1] != (heads + 2 * n_kv) * hd:
        raise DttsError(f"qk_norm_rope_kv_append: qkv width {qkv.shape[-1]} != (heads + 2*n_kv)*D")
    p, pp = _pos_array(pos, b, "qk_norm_rope_kv_append")
    q = torch.empty((b, heads, hd), dtype=qkv.dtype, device=qkv.device)
    k = torch.empty((b, n_kv, hd), dtype=_F32, device=qkv.device) if f32_k else None
    fn = ("dtts_qk_norm_rope_kv_append_f32" if qkv.dtype == _F32 else "dtts_qk_norm_rope_kv_append_f16")
    call(fn, ptr(qkv), ptr(norms), ptr(cos), ptr(sin), pp, ptr(q), ptr(k), ptr(k_cache), ptr(v_cache),
         b, heads, n_kv, hd, cap, cos.shape[0], float(eps), stream_handle())
    return (q, k) if f32_k else q


def kv_append(k, v, pos, k_cache, v_cache):
    """cache.slice_set(k.to_dtype(F16), 2, pos) for k and v (crates/qwen3tts/src/qwen3.rs:389-392),
    a position per lane: k, v [b, n_kv, D]; caches [b, n_kv, cap, D] f16, in place."""
    _check(k, "kv_append", (_F32, _F16), "k")
    _check(v, "kv_append", (k.dtype,), "v")
    for t, w in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        _check(t, "kv_append", (_F16,), w)
    b, n_kv, hd = k.shape
    if tuple(k_cache.shape[:2]) != (b, n_kv) or k_cache.shape[3] != hd:
        raise DttsError(f"kv_append: cache {tuple(k_cache.shape)} does not hold k {tuple(k.shape)}")
    p, pp = _pos_array(pos, b, "kv_append")
    fn = "dtts_kv_append_f32" if k.dtype == _F32 else "dtts_kv_append_f16"
    call(fn, ptr(k), ptr(v), pp, ptr(k_cache), ptr(v_cache), b, n_kv, hd, k_cache.shape[2], stream_handle())
