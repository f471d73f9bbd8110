"""Snake kernels (a1/a2) against the CPU oracle and double precision, through the C ABI.

Tolerances: f32 outputs max-rel <= 1e-5 against the oracle (the reference's bound,
crates/tts-nn/src/fused.rs:2452-2482) and <= 1e-6 / 2e-6 of max(|x|, r, 1) against f64
(fused.rs:2356-2391, 2227-2337); f16 outputs within 1 f16 ulp of the oracle's f16 result.
"""
import numpy as np
import pytest
import torch

import oracle
from dtts import ops, synth

from _util import f16_ulp_diff, rel, to_dev, to_host

pytestmark = pytest.mark.gpu


def _params(seed, c):
    a = np.exp(synth.normal(seed, "alpha", (c,))).astype(np.float32)
    r = np.exp(synth.normal(seed, "brecip", (c,))).astype(np.float32)
    return a, r


@pytest.mark.parametrize("rows,c", [(33, 7), (601, 1536), (4801, 24), (1000, 96), (5, 1), (3, 8)])
def test_snake_nlc_f32(dev, rows, c):
    x = synth.normal(20, "x", (rows, c), 0, 2)
    a, r = _params(20, c)
    got = to_host(ops.snake_beta_nlc(to_dev(x, dev), to_dev(a, dev), to_dev(r, dev)))
    want = oracle.snake_nlc_f32(x, a, r)
    assert rel(got, want)[1] < 1e-5


def test_snake_f32_generator_range_accuracy(dev):
    # crates/tts-nn/src/fused.rs:2356-2391: x over +-12, alpha 0.03..2.33, brecip 0.5 + j;
    # error against f64 scaled by max(|x|, r, 1) < 1e-6.
    c, length = 8, 2048
    xs = (-12.0 + 24.0 * (np.arange(c * length) % length) / (length - 1)).astype(np.float32)
    x = xs.reshape(1, c, length)
    al = np.array([0.03 + 2.3 * j / (c - 1) for j in range(c)], np.float32)
    br = np.array([0.5 + j for j in range(c)], np.float32)
    got = to_host(ops.snake_beta(to_dev(x, dev), to_dev(al, dev), to_dev(br, dev)))
    want = x + br[None, :, None].astype(np.float64) * np.sin(al[None, :, None].astype(np.float64) * x) ** 2
    scale = np.maximum(np.maximum(np.abs(x), br[None, :, None]), 1.0)
    assert np.max(np.abs(got - want) / scale) < 1e-6


@pytest.mark.parametrize("lanes,c,length", [(1, 7, 33), (1, 1536, 601), (1, 24, 4801),
                                            (1, 512, 4800), (3, 5, 17)])
def test_snake_ncl_f32(dev, lanes, c, length):
    x = synth.normal(21, "x", (lanes, c, length), 0, 2)
    a, r = _params(21, c)
    got = to_host(ops.snake_beta(to_dev(x, dev), to_dev(a, dev), to_dev(r, dev)))
    want = oracle.snake_ncl_f32(x, a, r)
    assert rel(got, want)[1] < 1e-5


def test_snake_f32_wide_sweep_accuracy(dev):
    # crates/tts-nn/src/fused.rs:2227-2337: x over +-30, alpha 0.05..2.55; bound 2e-6.
    c, length = 8, 4096
    xs = (-30.0 + 60.0 * (np.arange(c * length) % length) / (length - 1)).astype(np.float32)
    x = xs.reshape(length, c)
    al = np.array([0.05 + 2.5 * j / (c - 1) for j in range(c)], np.float32)
    br = np.array([0.5 + j for j in range(c)], np.float32)
    got = to_host(ops.snake_beta_nlc(to_dev(x, dev), to_dev(al, dev), to_dev(br, dev)))
    want = oracle.snake_nlc_f64(x, al, br)
    scale = np.maximum(np.maximum(np.abs(x), br[None, :]), 1.0)
    assert np.max(np.abs(got - want) / scale) < 2e-6


def test_snake_f32_exact_product_reduction(dev):
    # The f32 SnakeBeta reduces the exact product a x, not its f32 rounding: with x in [-1, 1],
    # r = 1 and a up to 2^20, y is within 4e-7 of x + sin^2(a x) in f64 (the product's rounding
    # alone would move sin^2 by up to |a x| 2^-24, 0.03 at 2^19). Past |a x| = 2^20 y stays in
    # [x, x + r]; inf and nan give nan.
    c, length = 16, 2048
    x = synth.uniform(23, "x", (length, c), -1.0, 1.0)
    a = (2.0 ** np.linspace(-2.0, 20.0, c)).astype(np.float32)
    r = np.ones(c, np.float32)
    got = to_host(ops.snake_beta_nlc(to_dev(x, dev), to_dev(a, dev), to_dev(r, dev))).astype(np.float64)
    want = oracle.snake_nlc_f64(x, a, r)
    assert np.max(np.abs(got - want)) < 4e-7

    big = np.array([[3.0e6, -7.5e8, 1.0e30, np.inf, -np.inf, np.nan, 2.0e6, -1.0]], np.float32)
    ab = np.array([1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 0.7, 3.0e6], np.float32)
    rb = np.full(8, 2.5, np.float32)
    yb = to_host(ops.snake_beta_nlc(to_dev(big, dev), to_dev(ab, dev), to_dev(rb, dev)))[0]
    assert np.all(np.isnan(yb[3:6]))
    for j in (0, 1, 2, 6, 7):
        lo, hi = sorted((float(big[0, j]), float(big[0, j]) + 2.5))
        tol = np.spacing(np.float32(abs(big[0, j]) + 2.5))
        assert lo - tol <= yb[j] <= hi + tol, (j, yb[j])


@pytest.mark.parametrize("rows,c", [(33, 7), (601, 1536), (4801, 24), (2000, 96), (9, 8)])
def test_snake_nlc_f16(dev, rows, c):
    x = synth.f16_bits(synth.normal(22, "x", (rows, c), 0, 3))
    a = synth.uniform(22, "a", (c,), 0.5, 1.5)
    r = (1.0 / a).astype(np.float32)
    got = to_host(ops.snake_beta_nlc(to_dev(x, dev), to_dev(a, dev), to_dev(r, dev)))
    want = oracle.snake_nlc_f16(x, a, r)
    assert f16_ulp_diff(got, want) <= 1
    assert rel(synth.from_f16_bits(got), synth.from_f16_bits(want))[1] < 1e-3


@pytest.mark.parametrize("lanes,c,length", [(1, 7, 33), (2, 96, 4800), (1, 3, 8)])
def test_snake_ncl_f16(dev, lanes, c, length):
    x = synth.f16_bits(synth.normal(23, "x", (lanes, c, length), 0, 3))
    a = synth.uniform(23, "a", (c,), 0.5, 1.5)
    r = (1.0 / a).astype(np.float32)
    got = to_host(ops.snake_beta(to_dev(x, dev), to_dev(a, dev), to_dev(r, dev)))
    want = oracle.snake_ncl_f16(x, a, r)
    assert f16_ulp_diff(got, want) <= 1


def test_snake_f16_fast_sine_accuracy(dev):
    # The f16 path's hardware sine over the generator's range (|alpha x| up to ~75): error
    # against f64 stays within half an f16 ulp of the result plus 2e-6 of the operand scale.
    c, length = 8, 4096
    xs = (-30.0 + 60.0 * (np.arange(c * length) % length) / (length - 1)).astype(np.float32)
    x = synth.f16_bits(xs.reshape(length, c))
    xf = synth.from_f16_bits(x)
    al = np.array([0.05 + 2.5 * j / (c - 1) for j in range(c)], np.float32)
    br = np.array([0.5 + j for j in range(c)], np.float32)
    got = synth.from_f16_bits(to_host(ops.snake_beta_nlc(to_dev(x, dev), to_dev(al, dev), to_dev(br, dev))))
    want = oracle.snake_nlc_f64(xf, al, br)
    half_ulp = np.abs(want) * 2.0 ** -11 + 2.0 ** -25
    scale = np.maximum(np.maximum(np.abs(xf), br[None, :]), 1.0)
    assert np.all(np.abs(got - want) <= half_ulp + 2e-6 * scale)


def test_snake_in_place_and_zero(dev):
    x = synth.normal(24, "x", (100, 96), 0, 1)
    a, r = _params(24, 96)
    t = to_dev(x, dev)
    ops.snake_beta_nlc(t, to_dev(a, dev), to_dev(r, dev), out=t)
    assert rel(to_host(t), oracle.snake_nlc_f32(x, a, r))[1] < 1e-5
    z = torch.zeros((10, 96), device=dev)
    assert torch.count_nonzero(ops.snake_beta_nlc(z, to_dev(a, dev), to_dev(r, dev))).item() == 0


def test_snake_rejects_bad_arguments(dev):
    from dtts import DttsError

    x = torch.zeros((4, 8), device=dev)
    a = torch.ones(7, device=dev)
    with pytest.raises(DttsError, match="alpha"):
        ops.snake_beta_nlc(x, a, a)


# ---------------------------------------------------------------- the folded snakes

@pytest.mark.parametrize("shape,offset", [((1, 7, 33), 0), ((1, 96, 131072), 0), ((4801,), 0), ((1, 96, 1003), 1),
                                          ((3,), 0), ((0,), 0)])
def test_snake_folded_f32(dev, shape, offset):
    """snake_folded against the oracle (fused.rs:2429-2446's 1e-5 against the composed form) and
    f64; offset 1 runs the unaligned scalar kernel, odd counts the vector kernel's tail."""
    n = int(np.prod(shape))
    x = synth.normal(25, "x", (n + offset,), 0, 2)
    xd = to_dev(x, dev)[offset:]
    got = to_host(ops.snake_folded(xd))
    want = oracle.snake_folded_f32(x[offset:])
    if n:
        assert rel(got, want)[1] < 1e-5
        xf = x[offset:].astype(np.float64)
        assert np.max(np.abs(got - (xf + np.sin(xf) ** 2)) / np.maximum(np.abs(xf), 1.0)) < 2e-6


@pytest.mark.parametrize("lanes,c,length", [(1, 7, 33), (1, 96, 131072), (1, 1536, 601), (3, 5, 17), (2, 24, 4801)])
def test_snake_alpha_f32(dev, lanes, c, length):
    x = synth.normal(26, "x", (lanes, c, length), 0, 2)
    a = synth.normal(26, "alpha", (c,))
    got = to_host(ops.snake_alpha(to_dev(x, dev), to_dev(a, dev)))
    assert rel(got, oracle.snake_alpha_f32(x, a))[1] < 1e-5


def test_folded_snakes_wide_sweep_accuracy(dev):
    # crates/tts-nn/src/fused.rs:2227-2283 ("snake_folded", "snake (alpha)"): x over +-30, alpha
    # 0.05..2.55; error scaled by max(|x|, 1) resp. max(|alpha x|, 1) below 2e-6.
    c, length = 8, 4096
    x = (-30.0 + 60.0 * (np.arange(c * length) % length) / (length - 1)).astype(np.float32).reshape(1, c, length)
    al = np.array([0.05 + 2.5 * j / (c - 1) for j in range(c)], np.float32)
    xd = x.astype(np.float64)
    got = to_host(ops.snake_folded(to_dev(x, dev)))
    assert np.max(np.abs(got - (xd + np.sin(xd) ** 2)) / np.maximum(np.abs(xd), 1.0)) < 2e-6
    u = al.astype(np.float64)[None, :, None] * xd
    got = to_host(ops.snake_alpha(to_dev(x, dev), to_dev(al, dev)))
    assert np.max(np.abs(got - (u + np.sin(u) ** 2)) / np.maximum(np.abs(u), 1.0)) < 2e-6


def test_folded_snakes_in_place_and_identities(dev):
    """In place; alpha = 1 gives snake_folded bit for bit (the same sine of the same argument)."""
    x = synth.normal(27, "x", (2, 96, 1000), 0, 2)
    t = to_dev(x, dev)
    ref = ops.snake_folded(t)
    ones = torch.ones(96, device=dev)
    assert torch.equal(ops.snake_alpha(t, ones), ref)
    ops.snake_folded(t, out=t)
    assert torch.equal(t, ref)


def test_folded_snakes_reject_bad_arguments(dev):
    from dtts import DttsError

    with pytest.raises(DttsError, match="alpha"):
        ops.snake_alpha(torch.zeros((1, 8, 4), device=dev), torch.ones(7, device=dev))
    with pytest.raises(DttsError, match="dtype"):
        ops.snake_folded(torch.zeros(8, dtype=torch.float16, device=dev))
    from dtts._lib import call
    with pytest.raises(DttsError, match="negative"):
        call("dtts_snake_folded_f32", None, None, -1, None)
