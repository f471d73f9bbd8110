"""The codec front half's own kernels through the C ABI against the oracle: the RVQ lookup-sum
(bit-exact: the same f32 additions in codebook order, one rounding), the depthwise conv +
LayerNorm (one f16 ulp plus 1e-5 per element: the channel sums run in another order, which
moves outputs near zero by a few of their tiny ulps), and the conv epilogue's
GELU and per-channel scale at ConvNeXt's pointwise shapes (the conv bar: max-abs 2e-2 and one
ulp plus f32 summation-order error per element)."""
import numpy as np
import pytest
import torch

import oracle
from dtts import DttsError, nlc, ops, synth

from _util import to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,n_books,size,dim,first", [(48 * 75, 16, 2048, 256, 1), (7, 5, 33, 8, 2)])
def test_rvq_lookup_sum_bit_exact(dev, rows, n_books, size, dim, first):
    books = synth.normal(30, "books", (n_books, size, dim))
    codes = synth.randint(30, "codes", (rows, n_books), 0, size - 1).astype(np.int32)
    got = to_host(ops.rvq_lookup_sum(to_dev(codes, dev), to_dev(books, dev), first))
    assert np.array_equal(got, oracle.rvq_lookup_sum_f16(codes, books, first))


@pytest.mark.parametrize("lanes,length,c,k", [(2, 300, 1024, 7), (3, 41, 64, 7), (1, 17, 2048, 3), (2, 5, 8, 7)])
def test_depthwise_layernorm_matches_oracle(dev, lanes, length, c, k):
    x = synth.f16_bits(synth.normal(31, "x", (lanes, length, c)))
    taps = synth.normal(31, "taps", (c, k), 0, 0.3)
    bias = synth.normal(31, "bias", (c,), 0, 0.1)
    w = synth.uniform(31, "w", (c,), 0.5, 1.5)
    b = synth.normal(31, "b", (c,), 0, 0.1)
    got = to_host(ops.depthwise_layernorm(to_dev(x, dev), to_dev(taps, dev), to_dev(bias, dev), to_dev(w, dev),
                                          to_dev(b, dev), 1e-6))
    want = synth.from_f16_bits(oracle.depthwise_layernorm_f16(x, taps, bias, w, b, 1e-6)).astype(np.float64)
    g = synth.from_f16_bits(got).astype(np.float64)
    bad = np.abs(g - want) > np.abs(want) * 2.0 ** -10 + 1e-5
    assert not bad.any(), f"{int(bad.sum())} elements off, worst {np.max(np.abs(g - want)):.3e}"


def _close_elementwise(got, want):
    g = synth.from_f16_bits(got).astype(np.float64)
    w = synth.from_f16_bits(want).astype(np.float64)
    assert np.max(np.abs(g - w)) <= 2e-2
    bad = np.abs(g - w) > np.abs(w) * 2.0 ** -10 + 1e-4
    assert not bad.any(), f"{int(bad.sum())} elements off"


@pytest.mark.parametrize("lanes,length,cin,cout", [(2, 200, 1024, 4096), (1, 70, 256, 512)])
def test_pointwise_gelu(dev, lanes, length, cin, cout):
    x = synth.f16_bits(synth.normal(32, "x", (lanes, length, cin)))
    w = synth.f16_bits(synth.normal(32, "w", (cout, cin), 0, 1 / np.sqrt(cin)))
    b = synth.f16_bits(synth.normal(32, "b", (cout,), 0, 0.1))
    got = to_host(nlc.conv1d(to_dev(x, dev), to_dev(w, dev), to_dev(b, dev), k=1, act="gelu"))
    want = oracle.conv1d_nlc_f16(x, np.ascontiguousarray(w.T), b, 1, act="gelu")
    _close_elementwise(got, want)


@pytest.mark.parametrize("lanes,length,cin,cout", [(2, 200, 4096, 1024), (1, 33, 96, 64)])
def test_pointwise_scale_residual(dev, lanes, length, cin, cout):
    x = synth.f16_bits(synth.normal(33, "x", (lanes, length, cin)))
    w = synth.f16_bits(synth.normal(33, "w", (cout, cin), 0, 1 / np.sqrt(cin)))
    b = synth.f16_bits(synth.normal(33, "b", (cout,), 0, 0.1))
    r = synth.f16_bits(synth.normal(33, "r", (lanes, length, cout)))
    s = synth.uniform(33, "s", (cout,), 0.05, 0.15)
    got = to_host(nlc.conv1d(to_dev(x, dev), to_dev(w, dev), to_dev(b, dev), k=1, residual=to_dev(r, dev),
                             scale=to_dev(s, dev)))
    want = oracle.conv1d_nlc_f16(x, np.ascontiguousarray(w.T), b, 1, res_bits=r, scale=s)
    _close_elementwise(got, want)


def test_front_ops_reject_bad_arguments(dev):
    x = torch.zeros((1, 4, 12), dtype=torch.float16, device=dev)
    f = torch.zeros(12, dtype=torch.float32, device=dev)
    with pytest.raises(DttsError, match="multiple of 8"):
        ops.depthwise_layernorm(x, torch.zeros((12, 7), device=dev), f, f, f, 1e-6)
    codes = torch.zeros((3, 4), dtype=torch.int32, device=dev)
    with pytest.raises(DttsError, match="codes per row"):
        ops.rvq_lookup_sum(codes, torch.zeros((5, 8, 4), device=dev), 1)
