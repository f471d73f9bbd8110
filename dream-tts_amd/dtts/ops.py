"""tts-nn's op surface over libdtts, on torch device tensors.

Each function keeps the reference function's name and argument meaning (drmhse/dream-tts,
crates/tts-nn) and, like the reference's CustomOps, allocates its output. The C ABI underneath
is what a Rust shim binds; this layer is the tests' and the bench's way in. Nothing here
computes: every op is one or more libdtts kernel launches on the current stream.
"""
from __future__ import annotations

import torch

from ._lib import DttsError, call, lib, ptr, stream_handle

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


def snake_folded(x, out=None):
    """`x + sin^2(x)`, f32, any contiguous shape. crates/tts-nn/src/fused.rs:501-508."""
    _check(x, "snake_folded", (_F32,), "x")
    y = torch.empty_like(x) if out is None else out
    _check(y, "snake_folded", (_F32,), "out")
    if y.numel() != x.numel():
        raise DttsError(f"snake_folded: out has {y.numel()} elements for {x.numel()}")
    call("dtts_snake_folded_f32", ptr(x), ptr(y), x.numel(), stream_handle())
    return y


def snake_alpha(x, alpha, out=None):
    """`u + sin^2(u)`, `u = alpha[c] * x`, over NCL `[lanes, C, L]` f32.

    crates/tts-nn/src/fused.rs:510-522 (lanes == 1 there) and tts_nn::snake, lib.rs:1075-1083."""
    _check(x, "snake_alpha", (_F32,), "x")
    if x.dim() != 3:
        raise DttsError(f"snake_alpha: x must be [lanes, C, L], got {tuple(x.shape)}")
    lanes, c, length = x.shape
    _check(alpha, "snake_alpha", (_F32,), "alpha")
    if alpha.numel() != c:
        raise DttsError(f"snake_alpha: alpha has {alpha.numel()} elements for {c} channels")
    y = torch.empty_like(x) if out is None else out
    call("dtts_snake_alpha_f32", ptr(x), ptr(alpha), ptr(y), lanes, c, length, stream_handle())
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


def qkrope_apply(qkv, norms, cos, sin, k_cache, v_cache, heads, start, eps, f32_kv=False):
    """qkrope::apply (crates/tts-nn/src/qkrope.rs:19-69) with the reference's signature.

    qkv [b, t, (heads + 2*n_kv) * D] f32; norms [2, D]; cos/sin [positions, D/2]; caches
    [b, n_kv, cap, D] f16 (a lane window, e.g. ``cache.narrow(0, off, b)``, is fine), written in
    place at start .. start + t - 1. Returns (q [b, heads, t, D], (k, v) [b, n_kv, t, D] f32 when
    f32_kv else None)."""
    name = "qkrope_apply"
    _check(qkv, name, (_F32,), "qkv")
    _check(norms, name, (_F32,), "norms")
    for t_, w in ((cos, "cos"), (sin, "sin")):
        _check(t_, name, (_F32,), w)
    for t_, w in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        _check(t_, name, (_F16,), w)
    if qkv.dim() != 3:
        raise DttsError(f"{name}: qkv must be [b, t, width]")
    b, t, width = qkv.shape
    if k_cache.shape != v_cache.shape or k_cache.shape[0] != b:
        raise DttsError(f"{name}: caches {tuple(k_cache.shape)} / {tuple(v_cache.shape)} do not hold {b} lanes")
    _, n_kv, cap, hd = k_cache.shape
    if width != (heads + 2 * n_kv) * hd:
        raise DttsError(f"{name}: qkv width {width} != (heads + 2*n_kv)*D")
    q = torch.empty((b, heads, t, hd), dtype=_F32, device=qkv.device)
    side = None
    if f32_kv:
        side = tuple(torch.empty((b, n_kv, t, hd), dtype=_F32, device=qkv.device) for _ in range(2))
    call("dtts_qkrope_apply_f32", ptr(qkv), ptr(norms), ptr(cos), ptr(sin), ptr(k_cache), ptr(v_cache),
         heads, start, float(eps), ptr(q), ptr(side[0]) if side else None, ptr(side[1]) if side else None,
         b, t, n_kv, hd, cap, cos.shape[0], stream_handle())
    return q, side


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


# ---------------------------------------------------------------- f-1 decode attention

def decode_attention(q, k, v, span, window_start=0, out=None, workspace=None):
    """attn::decode_attention (crates/tts-nn/src/attn.rs:18-73): q [b, n_kv, gqa, D] f32 (scale
    folded in), caches k, v [b, n_kv, cap, D] (f16 or f32, read in place) -> [b, n_kv, gqa, D] f32
    over positions [window_start, span). span and window_start are one int for the whole batch,
    as in the reference, or one per lane. `workspace` (a device byte tensor of at least
    decode_attention_workspace_bytes) lets long spans split over workgroups; allocated here when
    not given."""
    import numpy as np

    _check(q, "decode_attention", (_F32,), "q")
    _check(k, "decode_attention", (_F16, _F32), "k")
    _check(v, "decode_attention", (k.dtype,), "v")
    if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape:
        raise DttsError(f"decode_attention: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    b, n_kv, gqa, hd = q.shape
    if tuple(k.shape[:2]) != (b, n_kv) or k.shape[3] != hd:
        raise DttsError(f"decode_attention: cache {tuple(k.shape)} does not match q {tuple(q.shape)}")
    sp, spp = _pos_array(np.broadcast_to(np.asarray(span, np.int32), (b,)), b, "decode_attention")
    ws, wsp = _pos_array(np.broadcast_to(np.asarray(window_start, np.int32), (b,)), b, "decode_attention")
    y = torch.empty_like(q) if out is None else out
    if workspace is None:
        need = decode_attention_workspace_bytes(b, n_kv, gqa, hd, int(np.max(sp - ws)) if b else 0)
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    fn = "dtts_decode_attention_f16" if k.dtype == _F16 else "dtts_decode_attention_f32"
    call(fn, ptr(q), ptr(k), ptr(v), ptr(y), b, n_kv, gqa, hd, k.shape[2], spp, wsp, ptr(workspace),
         workspace.numel(), stream_handle())
    return y


def decode_attention_workspace_bytes(b, n_kv, gqa, head_dim, max_window):
    """Workspace bytes decode_attention splits spans of up to max_window positions with."""
    from ._lib import lib as _l

    return int(_l().dtts_decode_attention_workspace_bytes(b, n_kv, gqa, head_dim, max_window))


# ---------------------------------------------------------------- a12-a15 projections

def _mat(t, name, what, dtype):
    _check(t, name, (dtype,), what)
    if t.dim() != 2:
        raise DttsError(f"{name}: {what} must be 2-D, got {tuple(t.shape)}")


def skinny_matmul(a, b):
    """skinny::matmul (crates/tts-nn/src/skinny.rs:155-165): [m, k] f16 x [k, n] f16 -> [m, n] f32."""
    _mat(a, "skinny_matmul", "a", _F16)
    _mat(b, "skinny_matmul", "b", _F16)
    m, k = a.shape
    if b.shape[0] != k:
        raise DttsError(f"gemm_skinny: {k} != {b.shape[0]}")
    c = torch.empty((m, b.shape[1]), dtype=_F32, device=a.device)
    call("dtts_gemm_f16_skinny", ptr(a), ptr(b), ptr(c), m, k, b.shape[1], stream_handle())
    return c


def gemm_workspace_bytes(m, k, n, gateup=False):
    """Workspace bytes matmul_nt (gateup=False, n outputs) or gateup_silu (n = ffn) split k with."""
    from ._lib import lib as _l

    return int(_l().dtts_gemm_f16_workspace_bytes(m, k, n, 1 if gateup else 0))


def _workspace(t, nbytes):
    return t if t is not None else torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")


def matmul_nt(a, w, workspace=None, out=None):
    """[m, k] f16 x [n, k]^T f16 -> [m, n] f32 (Proj::Half on the checkpoint's [out, in] weight).
    `workspace`: a device byte tensor of gemm_workspace_bytes(m, k, n) (allocated when not given)."""
    _mat(a, "matmul_nt", "a", _F16)
    _mat(w, "matmul_nt", "w", _F16)
    m, k = a.shape
    if w.shape[1] != k:
        raise DttsError(f"matmul_nt: {k} != {w.shape[1]}")
    c = torch.empty((m, w.shape[0]), dtype=_F32, device=a.device) if out is None else out
    ws = _workspace(workspace, gemm_workspace_bytes(m, k, w.shape[0]))
    call("dtts_gemm_f16_nt", ptr(a), ptr(w), ptr(c), m, k, w.shape[0], ptr(ws), ws.numel(), stream_handle())
    return c


def gateup_silu(a, w_gu, workspace=None, out=None):
    """silu(a . Wg^T) * (a . Wu^T), w_gu [2*ffn, k] = gate rows then up rows; f32 [m, ffn]."""
    _mat(a, "gateup_silu", "a", _F16)
    _mat(w_gu, "gateup_silu", "w_gu", _F16)
    m, k = a.shape
    ffn = w_gu.shape[0] // 2
    if w_gu.shape[1] != k or w_gu.shape[0] != 2 * ffn:
        raise DttsError("gateup_silu: w_gu must be [2*ffn, k]")
    y = torch.empty((m, ffn), dtype=_F32, device=a.device) if out is None else out
    ws = _workspace(workspace, gemm_workspace_bytes(m, k, ffn, True))
    call("dtts_gemm_f16_gateup_silu", ptr(a), ptr(w_gu), ptr(y), m, k, ffn, ptr(ws), ws.numel(), stream_handle())
    return y


def gemm_f32_nt(x, w_nk, workspace=None):
    """Proj::Dense's forward (crates/tts-nn/src/lib.rs:438-459, 527) on the [out, in] layout:
    x [m, k] f32 . w [n, k]^T f32 -> [m, n] f32 (dtts_gemm_f32_nt)."""
    _mat(x, "gemm_f32_nt", "x", _F32)
    _mat(w_nk, "gemm_f32_nt", "w", _F32)
    m, k = x.shape
    n = w_nk.shape[0]
    if w_nk.shape[1] != k:
        raise DttsError(f"gemm_f32_nt: w [{n}, {w_nk.shape[1]}] for k = {k}")
    y = torch.empty((m, n), dtype=_F32, device=x.device)
    need = int(lib().dtts_gemm_f32_nt_workspace_bytes(m, k, n))
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=x.device)
    call("dtts_gemm_f32_nt", ptr(x), ptr(w_nk), ptr(y), m, k, n, ptr(workspace), workspace.numel(), stream_handle())
    return y


def swiglu_mul(gate, up):
    """fused::swiglu_mul (crates/tts-nn/src/fused.rs:376-385), f32."""
    _check(gate, "swiglu_mul", (_F32,), "gate")
    _check(up, "swiglu_mul", (_F32,), "up")
    if gate.shape != up.shape:
        raise DttsError("swiglu_mul: shapes differ")
    y = torch.empty_like(gate)
    call("dtts_swiglu_mul_f32", ptr(gate), ptr(up), ptr(y), gate.numel(), stream_handle())
    return y


def q8_0_quantize(w):
    """Host: f32 numpy [rows, k] -> uint8 [rows, k/32, 34] GGML Q8_0 blocks."""
    import ctypes

    import numpy as np

    w = np.ascontiguousarray(w, np.float32)
    rows, k = w.shape
    out = np.empty((rows, k // 32, 34), np.uint8)
    call("dtts_q8_0_quantize", ctypes.c_void_p(w.ctypes.data), ctypes.c_void_p(out.ctypes.data), rows, k)
    return out


def q8_0_dequantize(blocks, k):
    """Device uint8 blocks [rows, k/32, 34] -> f32 [rows, k]."""
    rows = blocks.shape[0]
    w = torch.empty((rows, k), dtype=_F32, device=blocks.device)
    call("dtts_q8_0_dequantize_f32", ptr(blocks), ptr(w), rows, k, stream_handle())
    return w


def q8_0_workspace_bytes(m, k, n):
    return int(lib().dtts_gemm_q8_0_workspace_bytes(m, k, n))


def q8_0_repack(blocks, k):
    """GGML blocks (device uint8 [n, k/32, 34]) -> the packed layout (dtts_q8_0_repack)."""
    n = blocks.shape[0]
    out = torch.empty(int(lib().dtts_q8_0_packed_bytes(n, k)), dtype=torch.uint8, device=blocks.device)
    call("dtts_q8_0_repack", ptr(blocks), ptr(out), n, k, stream_handle())
    return out


_Q8_MODES = {"w8a16": 0, "w8a8": 1, "w8a32": 2}


def _q8_x(x, name):
    """x [m, k] f16 or f32 (Proj::forward hands QMatMul f32, crates/tts-nn/src/lib.rs:509-531):
    the entry-point suffix for its dtype."""
    _check(x, name, (_F16, _F32), "x")
    if x.dim() != 2:
        raise DttsError(f"{name}: x must be 2-D, got {tuple(x.shape)}")
    return "_f32" if x.dtype == _F32 else ""


def q8_0_matmul_packed(x, packed, n, mode="w8a16", workspace=None):
    """dtts_gemm_q8_0_packed{,_f32}: x [m, k] f16 or f32 times a repacked Q8_0 weight [n, k] ->
    y [m, n] f32."""
    sfx = _q8_x(x, "q8_0_matmul_packed")
    m, k = x.shape
    y = torch.empty((m, n), dtype=_F32, device=x.device)
    if workspace is None:
        workspace = torch.empty(max(q8_0_workspace_bytes(m, k, n), 16), dtype=torch.uint8, device=x.device)
    call("dtts_gemm_q8_0_packed" + sfx, ptr(x), ptr(packed), ptr(y), m, k, n, _Q8_MODES[mode], ptr(workspace),
         workspace.numel(), stream_handle())
    return y


def q8_0_matmul(x, blocks, mode="w8a16", workspace=None):
    """QMatMul::forward on a Q8_0 weight [n, k]: x [m, k] f16 or f32 -> y [m, n] f32 (f32 x goes
    to the _f32 entry points, whose W8A8 quantizes it directly). With a workspace (a device uint8
    tensor, or "auto" to allocate one) the A-sharing kernel runs (dtts_gemm_q8_0_ws{,_f32})."""
    sfx = _q8_x(x, "q8_0_matmul")
    m, k = x.shape
    n = blocks.shape[0]
    if blocks.dtype != torch.uint8 or not blocks.is_cuda or blocks.numel() != n * (k // 32) * 34:
        raise DttsError("q8_0_matmul: blocks must be device uint8 [n, k/32, 34]")
    y = torch.empty((m, n), dtype=_F32, device=x.device)
    md = _Q8_MODES[mode]
    if workspace is None:
        call("dtts_gemm_q8_0" + sfx, ptr(x), ptr(blocks), ptr(y), m, k, n, md, stream_handle())
        return y
    if isinstance(workspace, str):
        workspace = torch.empty(max(q8_0_workspace_bytes(m, k, n), 16), dtype=torch.uint8, device=x.device)
    call("dtts_gemm_q8_0_ws" + sfx, ptr(x), ptr(blocks), ptr(y), m, k, n, md, ptr(workspace), workspace.numel(),
         stream_handle())
    return y


# ---------------------------------------------------------------- codec front half

def rvq_lookup_sum(codes, codebooks, n_first, out=None):
    """Rvq::decode's lookups for both quantizer stacks (dtts_rvq_lookup_sum_f16): codes [rows,
    n_books] int32, codebooks [n_books, size, dim] f32 (folded) -> [rows, 2*dim] f16."""
    name = "rvq_lookup_sum"
    _check(codes, name, (torch.int32,), "codes")
    _check(codebooks, name, (torch.float32,), "codebooks")
    rows, n_books = codes.shape
    nb, size, dim = codebooks.shape
    if nb != n_books:
        raise DttsError(f"{name}: {n_books} codes per row for {nb} codebooks")
    y = torch.empty((rows, 2 * dim), dtype=torch.float16, device=codes.device) if out is None else out
    call("dtts_rvq_lookup_sum_f16", ptr(codes), ptr(codebooks), n_books, n_first, size, dim, ptr(y), rows,
         stream_handle())
    return y


def depthwise_layernorm(x, taps, bias, ln_weight, ln_bias, eps, out=None):
    """ConvNext's depthwise causal conv + LayerNorm (dtts_depthwise_layernorm_nlc_f16): x [lanes,
    L, C] f16, taps [C, k] f32, the rest [C] f32."""
    name = "depthwise_layernorm"
    _check(x, name, (torch.float16,), "x")
    for t, what in ((taps, "taps"), (bias, "bias"), (ln_weight, "ln_weight"), (ln_bias, "ln_bias")):
        _check(t, name, (torch.float32,), what)
    lanes, length, c = x.shape
    y = torch.empty_like(x) if out is None else out
    call("dtts_depthwise_layernorm_nlc_f16", ptr(x), ptr(taps), ptr(bias), ptr(ln_weight), ptr(ln_bias),
         float(eps), ptr(y), lanes, length, c, taps.shape[1], stream_handle())
    return y
