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
