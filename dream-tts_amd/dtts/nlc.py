"""tts-nn's channels-last conv surface (crates/tts-nn/src/nlc.rs) over libdtts.

Weights go through the host layout functions once (as the reference's loaders do) and then live
on the device in the tap-major [cout, k*cin] form the matrix-core kernel reads.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from ._lib import DttsError, call, lib, ptr, stream_handle


class ConvDesc(ctypes.Structure):
    _fields_ = [
        ("lanes", ctypes.c_int64), ("len", ctypes.c_int64), ("cin", ctypes.c_int64),
        ("cout", ctypes.c_int64), ("k", ctypes.c_int64), ("dilation", ctypes.c_int64),
        ("pad_left", ctypes.c_int64),
        ("x", ctypes.c_void_p), ("w", ctypes.c_void_p), ("bias", ctypes.c_void_p),
        ("in_alpha", ctypes.c_void_p), ("in_brecip", ctypes.c_void_p),
        ("residual", ctypes.c_void_p), ("y_pre", ctypes.c_void_p),
        ("out_alpha", ctypes.c_void_p), ("out_brecip", ctypes.c_void_p),
        ("y", ctypes.c_void_p), ("act", ctypes.c_int32), ("out_scale", ctypes.c_void_p),
    ]


def _p(t):
    return None if t is None else t.data_ptr()


def _need(t, name, what, dtype, shape=None):
    if t is None:
        return
    if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == dtype and t.is_contiguous()):
        raise DttsError(f"{name}: {what} must be a contiguous {dtype} device tensor")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise DttsError(f"{name}: {what} shape {tuple(t.shape)} != {tuple(shape)}")


def conv1d(x, w_tm, bias=None, *, k, dilation=1, pad_left=None, snake_in=None, residual=None,
           snake_out=None, want_pre=False, act=None, scale=None, out=None):
    """The general fused channels-last conv (dtts_conv1d_nlc_f16_ex, or dtts_conv1d_nlc_f32_ex
    when x is f32: NlcConv's own precision).

    x [lanes, L, cin], w_tm [cout, k*cin], bias [cout], residual: all f16, or all f32. snake_in /
    snake_out are (alpha, brecip) f32 pairs applied to the input as loaded / to the (rounded)
    output. act: None, "tanh", "gelu" (f16 only) or "clamp"; scale: f32 [cout] on (sum + bias)
    before the residual. Returns y, or (y_pre, y) when want_pre."""
    name = "nlc.conv1d"
    if x.dim() != 3:
        raise DttsError(f"{name}: x must be [lanes, L, cin]")
    lanes, length, cin = x.shape
    cout = w_tm.shape[0]
    dt = x.dtype
    if dt not in (torch.float16, torch.float32):
        raise DttsError(f"{name}: x must be f16 or f32, not {dt}")
    _need(x, name, "x", dt)
    _need(w_tm, name, "w_tm", dt, (cout, k * cin))
    _need(bias, name, "bias", dt, (cout,))
    _need(residual, name, "residual", dt, (lanes, length, cout))
    _need(scale, name, "scale", torch.float32, (cout,))
    for pair, what, c in ((snake_in, "snake_in", cin), (snake_out, "snake_out", cout)):
        if pair is not None:
            for t in pair:
                _need(t, name, what, torch.float32, (c,))
    y = torch.empty((lanes, length, cout), dtype=dt, device=x.device) if out is None else out
    y_pre = torch.empty_like(y) if want_pre else None
    d = ConvDesc(lanes, length, cin, cout, k, dilation,
                 (k - 1) * dilation if pad_left is None else pad_left,
                 _p(x), _p(w_tm), _p(bias),
                 _p(snake_in[0]) if snake_in else None, _p(snake_in[1]) if snake_in else None,
                 _p(residual), _p(y_pre),
                 _p(snake_out[0]) if snake_out else None, _p(snake_out[1]) if snake_out else None,
                 _p(y), {None: 0, "tanh": 1, "gelu": 2, "clamp": 3}[act], _p(scale))
    call("dtts_conv1d_nlc_f16_ex" if dt == torch.float16 else "dtts_conv1d_nlc_f32_ex", ctypes.byref(d),
         stream_handle())
    return (y_pre, y) if want_pre else y


def split_weight(w_tm, k):
    """dtts_conv_split_weight: a tap-major f32 weight [cout, k*cin] -> (the split weight
    [cout, k*3*cin] f16, w_inv = 2^-s) for conv1d_f32_split. Synchronises the stream once."""
    name = "nlc.split_weight"
    cout, kc = w_tm.shape
    _need(w_tm, name, "w_tm", torch.float32, (cout, kc))
    cin = kc // k
    w3 = torch.empty(int(lib().dtts_conv_split_weight_bytes(cout, k, cin)) // 2, dtype=torch.float16,
                     device=w_tm.device).view(cout, 3 * kc)
    inv = ctypes.c_float(0.0)
    call("dtts_conv_split_weight", _p(w_tm), cout, k, cin, _p(w3), ctypes.byref(inv), stream_handle())
    return w3, inv.value


def conv1d_f32_split(x, w3, w_inv, bias=None, *, k, dilation=1, pad_left=None, residual=None, snake_out=None,
                     want_pre=False, workspace=None):
    """NlcConv on f32 operands through the split route (dtts_conv1d_nlc_f32_split): x, bias,
    residual f32 as conv1d takes them, the weight as split_weight returns it. Returns y, or
    (y_pre, y) when want_pre."""
    name = "nlc.conv1d_f32_split"
    lanes, length, cin = x.shape
    cout = w3.shape[0]
    _need(x, name, "x", torch.float32)
    _need(w3, name, "w3", torch.float16, (cout, 3 * k * cin))
    _need(bias, name, "bias", torch.float32, (cout,))
    _need(residual, name, "residual", torch.float32, (lanes, length, cout))
    y = torch.empty((lanes, length, cout), dtype=torch.float32, device=x.device)
    y_pre = torch.empty_like(y) if want_pre else None
    d = ConvDesc(lanes, length, cin, cout, k, dilation,
                 (k - 1) * dilation if pad_left is None else pad_left,
                 _p(x), _p(w3), _p(bias), None, None, _p(residual), _p(y_pre),
                 _p(snake_out[0]) if snake_out else None, _p(snake_out[1]) if snake_out else None,
                 _p(y), 0, None)
    need = int(lib().dtts_conv1d_nlc_f32_split_workspace_bytes(ctypes.byref(d)))
    ws = workspace if workspace is not None else torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    call("dtts_conv1d_nlc_f32_split", ctypes.byref(d), ctypes.c_float(w_inv), _p(ws), ws.numel(), stream_handle())
    return (y_pre, y) if want_pre else y


class RuDesc(ctypes.Structure):
    _fields_ = [("lanes", ctypes.c_int64), ("len", ctypes.c_int64), ("channels", ctypes.c_int64),
                ("k", ctypes.c_int64), ("dilation", ctypes.c_int64)] + [
        (n, ctypes.c_void_p) for n in ("x", "act1_alpha", "act1_brecip", "w1", "b1", "act2_alpha",
                                       "act2_brecip", "w2", "b2", "y_pre", "out_alpha", "out_brecip", "y")]


def residual_unit(x, act1, w1_tm, b1, act2, w2_tm, b2, *, k, dilation, snake_out=None, want_pre=False):
    """ResidualUnit::forward (crates/qwen3tts/src/codec.rs:215-229) in one launch:
    x + conv_1(act2(conv_k(act1(x)))), optionally followed by the next SnakeBeta. x [lanes, L, C] f16."""
    name = "residual_unit"
    lanes, length, c = x.shape
    _need(x, name, "x", torch.float16)
    _need(w1_tm, name, "w1", torch.float16, (c, k * c))
    _need(w2_tm, name, "w2", torch.float16, (c, c))
    y = torch.empty_like(x)
    y_pre = torch.empty_like(x) if want_pre else None
    d = RuDesc(lanes, length, c, k, dilation, _p(x), _p(act1[0]), _p(act1[1]), _p(w1_tm), _p(b1),
               _p(act2[0]), _p(act2[1]), _p(w2_tm), _p(b2), _p(y_pre),
               _p(snake_out[0]) if snake_out else None, _p(snake_out[1]) if snake_out else None, _p(y))
    call("dtts_residual_unit_nlc_f16", ctypes.byref(d), stream_handle())
    return (y_pre, y) if want_pre else y


def conv1d_ncl_f32(x, w_tm, bias=None, *, k, dilation=1, pad_left=None, snake_in=None, residual=None,
                   snake_out=None, want_pre=False, out=None):
    """The channel-major f32 conv (dtts_conv1d_ncl_f32_ex): x [lanes, cin, L] f32, w_tm
    [cout, k*cin] f32 -> [lanes, cout, L]. centered_conv1d_gemm / causal_conv1d_gemm
    (crates/tts-nn/src/lib.rs:704-767) with the neighbouring SnakeBeta and residual fused."""
    name = "conv1d_ncl_f32"
    lanes, cin, length = x.shape
    cout = w_tm.shape[0]
    _need(x, name, "x", torch.float32)
    _need(w_tm, name, "w_tm", torch.float32, (cout, k * cin))
    _need(bias, name, "bias", torch.float32, (cout,))
    _need(residual, name, "residual", torch.float32, (lanes, cout, length))
    y = torch.empty((lanes, cout, length), dtype=torch.float32, device=x.device) if out is None else out
    y_pre = torch.empty_like(y) if want_pre else None
    d = ConvDesc(lanes, length, cin, cout, k, dilation,
                 (k - 1) * dilation if pad_left is None else pad_left,
                 _p(x), _p(w_tm), _p(bias),
                 _p(snake_in[0]) if snake_in else None, _p(snake_in[1]) if snake_in else None,
                 _p(residual), _p(y_pre),
                 _p(snake_out[0]) if snake_out else None, _p(snake_out[1]) if snake_out else None,
                 _p(y), 0)
    call("dtts_conv1d_ncl_f32_ex", ctypes.byref(d), stream_handle())
    return (y_pre, y) if want_pre else y


def im2col_tap_major(x, k, dilation, pad_left=None):
    """im2col::im2col_tap_major / im2col_centered (crates/tts-nn/src/im2col.rs:150-166): one lane
    [cin, L] f32 -> [k*cin, L]."""
    _need(x, "im2col_tap_major", "x", torch.float32)
    cin, length = x.shape
    cols = torch.empty((k * cin, length), dtype=torch.float32, device=x.device)
    call("dtts_im2col_tap_major_f32", _p(x), _p(cols), cin, length, k, dilation,
         (k - 1) * dilation if pad_left is None else pad_left, stream_handle())
    return cols


def causal_conv1d(x, w_tm, bias, dilation):
    """nlc::causal_conv1d (crates/tts-nn/src/nlc.rs:70-132), w in tap-major [cout, k*cin]."""
    k = w_tm.shape[1] // x.shape[-1]
    return conv1d(x, w_tm, bias, k=k, dilation=dilation)


def snake_conv_residual(x, w_tm, bias, dilation, snake, res):
    """nlc::snake_conv_residual (crates/tts-nn/src/nlc.rs:40-68): res + conv(SnakeBeta(x))."""
    k = w_tm.shape[1] // x.shape[-1]
    return conv1d(x, w_tm, bias, k=k, dilation=dilation, snake_in=snake, residual=res)


def causal_conv_transpose1d(x, w_tm, bias_rep, stride):
    """The polyphase transposed conv (crates/tts-nn/src/codec.rs:153-158 with
    nlc::transpose_tap_weight): one causal conv, then [b, L, s*cout] viewed as [b, L*s, cout]."""
    lanes, length, cin = x.shape
    k = w_tm.shape[1] // cin
    y = conv1d(x, w_tm, bias_rep, k=k, dilation=1)
    return y.view(lanes, length * stride, w_tm.shape[0] // stride)


# ---------------------------------------------------------------- host layouts

def _host_layout(fn, arr, out_shape, *dims):
    a = np.ascontiguousarray(arr)
    es = a.dtype.itemsize
    out = np.empty(out_shape, a.dtype)
    status = getattr(lib(), fn)(ctypes.c_void_p(a.ctypes.data), ctypes.c_void_p(out.ctypes.data),
                                *[ctypes.c_int64(d) for d in dims], ctypes.c_int64(es))
    if status != 0:
        raise DttsError(f"{fn}: {lib().dtts_last_error().decode()}")
    return out


def tap_major_weight(w_oik: np.ndarray) -> np.ndarray:
    """lib.rs:630-635: torch [cout, cin, k] -> [cout, k*cin] (host, numpy in/out)."""
    cout, cin, k = w_oik.shape
    return _host_layout("dtts_tap_major_weight", w_oik, (cout, k * cin), cout, cin, k)


def tap_weight_to_tap_major(w_kio: np.ndarray) -> np.ndarray:
    k, cin, cout = w_kio.shape
    return _host_layout("dtts_tap_weight_to_tap_major", w_kio, (cout, k * cin), k, cin, cout)


def transpose_tap_major_weight(w_iok: np.ndarray, stride: int) -> np.ndarray:
    """nlc.rs:158-174 in tap-major form: [cin, cout, K] -> [stride*cout, (K/stride)*cin]."""
    cin, cout, kernel = w_iok.shape
    return _host_layout("dtts_transpose_tap_major_weight", w_iok,
                        (stride * cout, (kernel // stride) * cin), cin, cout, kernel, stride)


def transpose_bias(b: np.ndarray, stride: int) -> np.ndarray:
    """nlc.rs:177-183: [cout] -> [stride*cout]."""
    return _host_layout("dtts_transpose_bias", b, (stride * b.shape[0],), b.shape[0], stride)
