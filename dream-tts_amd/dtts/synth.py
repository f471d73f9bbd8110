"""Seeded synthetic inputs, identical on every machine.

A counter-based SplitMix64 stream per (seed, tag): element i of stream (seed, tag) is
``mix(base + (i + 1) * GAMMA)`` with ``base = mix(seed * GAMMA + fnv1a(tag))``, so any tensor
can be regenerated alone and in any order. Uniforms take the top 53 bits; normals are
Box-Muller pairs ``(r cos 2 pi u2, r sin 2 pi u2)`` with ``r = sqrt(-2 ln u1)``,
``u1 in (0, 1]``. Values are produced in f64 and rounded to the requested dtype.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_TWO53 = float(2 ** -53)


def _mix(z):
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _fnv1a(tag: str) -> np.uint64:
    h = 0xCBF29CE484222325
    for b in tag.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return np.uint64(h)


def raw(seed: int, tag: str, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        base = _mix(np.array([np.uint64(seed) * GAMMA + _fnv1a(tag)], dtype=np.uint64))[0]
        idx = np.arange(1, n + 1, dtype=np.uint64)
        return _mix(base + idx * GAMMA)


def uniform(seed: int, tag: str, shape, lo: float = 0.0, hi: float = 1.0, dtype=np.float32):
    n = int(np.prod(shape))
    u = (raw(seed, tag, n) >> np.uint64(11)).astype(np.float64) * _TWO53
    return (lo + (hi - lo) * u).reshape(shape).astype(dtype)


def normal(seed: int, tag: str, shape, mean: float = 0.0, std: float = 1.0, dtype=np.float32):
    n = int(np.prod(shape))
    pairs = (n + 1) // 2
    z = raw(seed, tag, 2 * pairs)
    u1 = ((z[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * _TWO53
    u2 = (z[1::2] >> np.uint64(11)).astype(np.float64) * _TWO53
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * pairs, np.float64)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (mean + std * out[:n]).reshape(shape).astype(dtype)


def randint(seed: int, tag: str, shape, lo: int, hi: int):
    """Integers in [lo, hi] inclusive."""
    n = int(np.prod(shape))
    span = np.uint64(hi - lo + 1)
    return (lo + (raw(seed, tag, n) % span).astype(np.int64)).reshape(shape)


def f16_bits(x) -> np.ndarray:
    """IEEE binary16 bit patterns of x (round to nearest-even), as uint16."""
    return np.ascontiguousarray(np.asarray(x, np.float32).astype(np.float16).view(np.uint16))


def from_f16_bits(h) -> np.ndarray:
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def kaiming_normal(seed: int, tag: str, shape, fan_in: int, gain: float = float(np.sqrt(2.0)),
                   dtype=np.float32):
    """torch.nn.init.kaiming_normal_ (fan_in mode): std = gain / sqrt(fan_in); gain sqrt(2) is
    nonlinearity='relu' (the default), 1 is nonlinearity='linear'."""
    return normal(seed, tag, shape, 0.0, float(gain / np.sqrt(fan_in)), dtype)
