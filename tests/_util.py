"""Shared helpers for the parity tests: host<->device moves and the reference's metrics."""
from __future__ import annotations

import numpy as np

import oracle


def to_dev(a, dev, dtype=None):
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:  # f16 bit patterns
        t = torch.from_numpy(a.view(np.int16).copy()).view(torch.float16)
    else:
        t = torch.from_numpy(a.copy())
    if dtype is not None:
        t = t.to(dtype)
    return t.to(dev)


def to_host(t):
    import torch

    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def rel(got, want):
    """abs_and_rel's relative figure (crates/tts-nn/src/lib.rs:1239-1248)."""
    return oracle.abs_and_rel(np.asarray(got, np.float32).ravel(), np.asarray(want, np.float32).ravel())


def f16_ulp_diff(a_bits, b_bits):
    """Largest distance in f16 ulps between two arrays of finite f16 bit patterns."""
    def ordered(h):
        h = np.asarray(h, np.uint16).astype(np.int32)
        return np.where(h & 0x8000, 0x8000 - (h & 0x7FFF), 0x8000 + h)
    return int(np.max(np.abs(ordered(a_bits) - ordered(b_bits)))) if np.size(a_bits) else 0
