"""Pins the oracle's decode-attention restatement (attn::decode_attention's CPU path,
crates/tts-nn/src/attn.rs:18-73, 85-126, 189-226; softmax_last_dim from candle-nn 0.10.2, not
vendored) against an independent float64 evaluation (numpy einsum and exp over the masked
scores) at the reference test's shapes (attn.rs:391-398), and against what the mathematics fixes:
a one-position window returns that position's v exactly, constant v rows come back unchanged,
q = 0 averages v over the window, permuting the window's positions changes nothing, and cache
slots outside [window_start, span) never reach the result."""
import numpy as np
import pytest

import oracle
from dtts import synth

from _util import rel as _abs_rel


def rel(a, b):
    return _abs_rel(a, b)[1]

# (b, n_kv, gqa, cap, span, window_start): attn.rs:393-398
REF_SHAPES = [(48, 8, 2, 400, 250, 0), (40, 8, 2, 17, 3, 0), (8, 8, 2, 300, 211, 90), (4, 8, 1, 64, 33, 0)]


def _inputs(seed, b, n_kv, gqa, cap, hd=128):
    q = synth.normal(seed, "q", (b, n_kv, gqa, hd), 0, 0.1)
    k = synth.f16_bits(synth.normal(seed, "k", (b, n_kv, cap, hd)))
    v = synth.f16_bits(synth.normal(seed, "v", (b, n_kv, cap, hd)))
    return q, k, v


def attention_f64(q, k, v, span, ws):
    """float64: softmax over [ws, span) of q.k, weighting v (k, v given as f32 values)."""
    b = q.shape[0]
    span = np.broadcast_to(np.asarray(span), (b,))
    ws = np.broadcast_to(np.asarray(ws), (b,))
    out = np.empty(q.shape, np.float64)
    for i in range(b):
        kk = k[i, :, ws[i]:span[i]].astype(np.float64)
        vv = v[i, :, ws[i]:span[i]].astype(np.float64)
        s = np.einsum("hgd,hpd->hgp", q[i].astype(np.float64), kk)
        e = np.exp(s - s.max(-1, keepdims=True))
        out[i] = np.einsum("hgp,hpd->hgd", e / e.sum(-1, keepdims=True), vv)
    return out


@pytest.mark.parametrize("b,n_kv,gqa,cap,span,ws", REF_SHAPES)
def test_attention_matches_f64_at_reference_shapes(b, n_kv, gqa, cap, span, ws):
    q, k, v = _inputs(60, b, n_kv, gqa, cap)
    got = oracle.decode_attention_f32(q, k, v, span, ws)
    want = attention_f64(q, synth.from_f16_bits(k), synth.from_f16_bits(v), span, ws)
    assert rel(got, want) < 4e-6  # f32 sums over up to 250 positions


def test_attention_per_lane_windows_and_f32_cache():
    b, n_kv, gqa, cap, hd = 6, 2, 4, 50, 64
    q = synth.normal(61, "q", (b, n_kv, gqa, hd), 0, 0.3)
    k = synth.normal(61, "k", (b, n_kv, cap, hd))
    v = synth.normal(61, "v", (b, n_kv, cap, hd))
    span = np.array([1, 50, 17, 33, 2, 40], np.int32)
    ws = np.array([0, 10, 16, 0, 1, 39], np.int32)
    got = oracle.decode_attention_f32(q, k, v, span, ws)
    assert rel(got, attention_f64(q, k, v, span, ws)) < 1e-6


def test_attention_closed_forms():
    b, n_kv, gqa, cap, hd = 3, 2, 2, 40, 128
    q, k, v = _inputs(62, b, n_kv, gqa, cap)
    vf = synth.from_f16_bits(v)
    # a one-position window: probability exactly 1 on that position
    one = oracle.decode_attention_f32(q, k, v, 8, 7)
    assert np.array_equal(one, np.broadcast_to(vf[:, :, 7:8, :], one.shape))
    # every row of v the same vector: the weights sum to 1
    row = synth.f16_bits(synth.normal(62, "row", (hd,)))
    vc = np.ascontiguousarray(np.broadcast_to(row, v.shape))
    same = oracle.decode_attention_f32(q, k, vc, 30, 5)
    assert np.max(np.abs(same - synth.from_f16_bits(row))) < 2e-6 * np.max(np.abs(synth.from_f16_bits(row)))
    # q = 0: equal weights, the mean of v over the window
    zero = oracle.decode_attention_f32(np.zeros_like(q), k, v, 25, 4)
    mean = vf[:, :, 4:25, :].astype(np.float64).mean(2)[:, :, None, :]
    assert np.max(np.abs(zero - mean)) < 1e-6


def test_attention_is_order_free_and_ignores_slots_outside_the_window():
    b, n_kv, gqa, cap, hd = 2, 3, 2, 64, 128
    q, k, v = _inputs(63, b, n_kv, gqa, cap)
    span, ws = 50, 12
    base = oracle.decode_attention_f32(q, k, v, span, ws)
    perm = np.arange(cap)
    perm[ws:span] = ws + synth.randint(63, "perm", (span - ws,), 0, 10 ** 6).argsort()
    kp, vp = np.ascontiguousarray(k[:, :, perm]), np.ascontiguousarray(v[:, :, perm])
    assert rel(oracle.decode_attention_f32(q, kp, vp, span, ws), base) < 1e-6
    # large finite values outside [ws, span) change nothing
    ks, vs = k.copy(), v.copy()
    big = synth.f16_bits(np.float32(3e4))
    for t in (ks, vs):
        t[:, :, :ws] = big
        t[:, :, span:] = big
    assert np.array_equal(oracle.decode_attention_f32(q, ks, vs, span, ws), base)
