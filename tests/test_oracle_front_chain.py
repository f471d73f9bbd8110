"""Pins the oracle's codec front-half chain (oracle/codec_front.py: Codec::forward up to the
waveform stack, crates/qwen3tts/src/codec.rs:401-424) against an independent float64 numpy
restatement from the checkpoint-layout weights (tests/_front_ref.py) with f16 rounding at the
same storage points, at a small geometry with 2 transformer layers, a 5-frame window (so the
window bites) and two upsampling ratios; and the oracle's windowed prefill attention against
float64, with its window and causality invariants."""
import numpy as np

import oracle
from oracle import codec_front as ofront
from dtts import codec_front, synth

from _front_ref import TINY, front_f64
from _util import rel


def test_front_chain_matches_f64():
    geo = TINY
    hw = codec_front.random_weights(geo, 50)
    codes = synth.randint(50, "codes", (2, 11, geo.n_books), 0, geo.book_size - 1)
    got = synth.from_f16_bits(ofront.decode_f16(geo, hw, codes))
    want = front_f64(geo, hw, codes)
    assert got.shape == (2, 11 * 6, geo.latent_dim)
    assert rel(got, want)[1] < 2e-3  # f16 storage ties landing on either side (measured 9.5e-4)


def test_window_attention_against_f64_and_invariants():
    lanes, length, heads, n_kv, hd, window = 2, 23, 4, 2, 64, 6
    qkv = synth.f16_bits(synth.normal(51, "qkv", (lanes, length, (heads + 2 * n_kv) * hd)))
    cos_t, sin_t = oracle.rope_table_f32(length, hd, 1e4)
    scale = float(np.float32(1 / 8))
    got = synth.from_f16_bits(oracle.window_attention_prefill_f16(qkv, cos_t, sin_t, heads, n_kv, hd, window, scale))
    x = synth.from_f16_bits(qkv).astype(np.float64).reshape(lanes, length, heads + 2 * n_kv, hd)
    pos = np.arange(length)
    i = np.arange(hd // 2)
    ph = pos[:, None] * (1.0 / 1e4 ** (2.0 * i / hd))
    c, s = np.cos(ph), np.sin(ph)

    def rope(v):
        return np.concatenate([v[..., :hd // 2] * c - v[..., hd // 2:] * s, v[..., hd // 2:] * c + v[..., :hd // 2] * s], -1)

    want = np.zeros((lanes, length, heads, hd))
    for h in range(heads):
        kh = h // (heads // n_kv)
        sc = np.einsum("bid,bjd->bij", rope(x[:, :, h]), rope(x[:, :, heads + kh])) * scale
        a, b = np.meshgrid(pos, pos, indexing="ij")
        sc = np.where((b <= a) & (b > a - window), sc, -np.inf)
        e = np.exp(sc - sc.max(-1, keepdims=True))
        want[:, :, h] = np.einsum("bij,bjd->bid", e / e.sum(-1, keepdims=True), x[:, :, heads + n_kv + kh])
    assert rel(got, want.reshape(got.shape))[1] < 2e-3
    # position 0 attends only to itself: its output is its own v, rounded
    v0 = x[:, 0, heads + n_kv:].reshape(lanes, n_kv, hd)
    assert np.array_equal(got.reshape(lanes, length, heads, hd)[:, 0, 0], synth.from_f16_bits(synth.f16_bits(v0[:, 0])))
    # keys older than the window never matter
    q2 = qkv.reshape(lanes, length, heads + 2 * n_kv, hd).copy()
    q2[:, :10, heads:] = synth.f16_bits(np.float32(3.0))
    got2 = oracle.window_attention_prefill_f16(q2.reshape(qkv.shape), cos_t, sin_t, heads, n_kv, hd, window, scale)
    ref = oracle.window_attention_prefill_f16(qkv, cos_t, sin_t, heads, n_kv, hd, window, scale)
    assert np.array_equal(got2[:, 10 + window - 1:], ref[:, 10 + window - 1:])
