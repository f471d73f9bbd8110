"""Pins the oracle's codec front-half pieces on the CPU: the RVQ lookup-sum (Rvq::decode,
crates/qwen3tts/src/codec.rs:296-313) against numpy fancy indexing summed in float64 (one f16
ulp at most apart), with a one-book stack returning its row exactly; the depthwise conv +
LayerNorm (codec.rs:186-188) against an independent float64 restatement (np.convolve over the
zero-padded sequence, then mean / variance), with its invariants (zero mean and unit variance
per position before the affine part, causality, a per-channel offset absorbed by the
normalisation); and the conv epilogue's GELU (erf form) and per-channel scale against float64."""
import math

import numpy as np

import oracle
from dtts import synth

from _util import f16_ulp_diff, rel


def test_rvq_lookup_sum_against_numpy():
    rows, n_books, size, dim, first = 37, 6, 50, 16, 1
    books = synth.normal(20, "books", (n_books, size, dim))
    codes = synth.randint(20, "codes", (rows, n_books), 0, size - 1).astype(np.int32)
    got = oracle.rvq_lookup_sum_f16(codes, books, first)
    pick = books[np.arange(n_books)[None, :], codes]  # [rows, n_books, dim]
    sem = pick[:, :first].astype(np.float64).sum(1)
    ac = pick[:, first:].astype(np.float64).sum(1)
    want = synth.f16_bits(np.concatenate([sem, ac], 1).astype(np.float32))
    assert f16_ulp_diff(got, want) <= 1
    # the first stack holds one book: its row comes back exactly (rounded once to f16)
    assert np.array_equal(got[:, :dim], synth.f16_bits(pick[:, 0]))


def _dwln_f64(x, taps, bias, w, b, eps):
    lanes, length, c = x.shape
    k = taps.shape[1]
    h = np.zeros((lanes, length, c))
    xp = np.concatenate([np.zeros((lanes, k - 1, c)), x.astype(np.float64)], 1)
    for t in range(k):
        h += xp[:, t:t + length] * taps[:, t].astype(np.float64)
    h += bias
    m = h.mean(-1, keepdims=True)
    v = ((h - m) ** 2).mean(-1, keepdims=True)
    return (h - m) / np.sqrt(v + eps) * w + b


def test_depthwise_layernorm_against_f64_and_invariants():
    lanes, length, c, k = 3, 40, 64, 7
    x = synth.f16_bits(synth.normal(21, "x", (lanes, length, c)))
    taps = synth.normal(21, "taps", (c, k), 0, 0.3)
    bias = synth.normal(21, "bias", (c,), 0, 0.1)
    w = synth.uniform(21, "w", (c,), 0.5, 1.5)
    b = synth.normal(21, "b", (c,), 0, 0.1)
    got = oracle.depthwise_layernorm_f16(x, taps, bias, w, b, 1e-6)
    want = _dwln_f64(synth.from_f16_bits(x), taps, bias, w, b, 1e-6)
    assert rel(synth.from_f16_bits(got), want)[1] < 2e-3  # one f16 rounding of the output
    # without the affine part every position is normalised
    plain = synth.from_f16_bits(oracle.depthwise_layernorm_f16(x, taps, bias, np.ones(c, np.float32),
                                                                np.zeros(c, np.float32), 1e-6)).astype(np.float64)
    assert np.max(np.abs(plain.mean(-1))) < 2e-3 and np.max(np.abs(plain.var(-1) - 1)) < 4e-3
    # causal: later positions never change earlier outputs
    x2 = x.copy()
    x2[:, 25:] = synth.f16_bits(synth.normal(22, "x2", (lanes, length - 25, c)))
    got2 = oracle.depthwise_layernorm_f16(x2, taps, bias, w, b, 1e-6)
    assert np.array_equal(got2[:, :25], got[:, :25]) and not np.array_equal(got2[:, 25:], got[:, 25:])
    # a constant per position is removed by the mean: with taps summing the same, shifting every
    # channel's bias by one constant leaves the output as it was (to rounding)
    shifted = oracle.depthwise_layernorm_f16(x, taps, bias + np.float32(0.25), w, b, 1e-6)
    assert f16_ulp_diff(shifted, got) <= 2


def test_conv_gelu_and_scale_epilogue_against_f64():
    lanes, length, cin, cout = 2, 30, 16, 24
    x = synth.f16_bits(synth.normal(23, "x", (lanes, length, cin)))
    w = synth.f16_bits(synth.normal(23, "w", (1, cin, cout), 0, 0.4))
    bias = synth.f16_bits(synth.normal(23, "b", (cout,), 0, 0.1))
    res = synth.f16_bits(synth.normal(23, "r", (lanes, length, cout)))
    scale = synth.uniform(23, "s", (cout,), 0.05, 0.15)
    xf, wf = synth.from_f16_bits(x).astype(np.float64), synth.from_f16_bits(w)[0].astype(np.float64)
    s = xf @ wf + synth.from_f16_bits(bias)
    g = oracle.conv1d_nlc_f16(x, w, bias, 1, act="gelu")
    erf = np.vectorize(math.erf)
    want_g = 0.5 * s * (1 + erf(s / math.sqrt(2)))
    assert rel(synth.from_f16_bits(g), want_g)[1] < 1e-3
    y = oracle.conv1d_nlc_f16(x, w, bias, 1, res_bits=res, scale=scale)
    want_y = synth.from_f16_bits(res) + s * scale
    assert rel(synth.from_f16_bits(y), want_y)[1] < 1e-3
    # GELU's closed points: 0 -> 0, large positive -> x, large negative -> 0
    v = oracle.gelu_erf(np.array([0.0, 8.0, -8.0, 1.0], np.float32))
    assert v[0] == 0 and v[1] == np.float32(8.0) and abs(v[2]) < 1e-12
    assert abs(v[3] - 0.5 * (1 + math.erf(1 / math.sqrt(2)))) < 1e-7
