"""Pins the oracle's decoder-stack step (oracle.stack_decode_f32: Stack::forward at t = 1,
crates/qwen3tts/src/qwen3.rs:294-467, composed from the oracle's pinned rms_norm, projection,
QK-norm/RoPE/append, attention and SwiGLU restatements) against an independent float64 numpy
restatement with the f16 roundings at the same points, over several steps so the caches carry
history, with and without QK-norm, LayerScale and a sliding window; and against what the
mathematics fixes: with zero output and down projections the residual stream is x and the
result is rms_norm(x, norm) exactly, and cache slots other than each lane's position are never
written."""
import numpy as np
import pytest

import oracle
from dtts import stack, synth

from _stack_ref import SMALL, WINDOWED, inputs, stack_f64
from _util import rel


def _run_both(geo, seed, lanes, cap, steps):
    layers, fn = stack.random_weights(geo, seed)
    x, kc, vc = inputs(geo, seed, lanes, cap)
    kr, vr = [k.copy() for k in kc], [v.copy() for v in vc]
    start = synth.randint(seed, "stack.pos", (lanes,), 0, cap - steps).astype(np.int32)
    worst_out, worst_cache = 0.0, 0.0
    for s in range(steps):
        pos = start + s
        xs = x * np.float32(1.0 + 0.1 * s)
        got = oracle.stack_decode_f32(geo, layers, fn, xs, kc, vc, pos)
        want, kr, vr = stack_f64(geo, layers, fn, xs, kr, vr, pos)
        worst_out = max(worst_out, rel(got, want)[1])
        for li in range(geo.layers):
            for a, b in ((kc[li], kr[li]), (vc[li], vr[li])):
                worst_cache = max(worst_cache, rel(synth.from_f16_bits(a), synth.from_f16_bits(b))[1])
        # keep the f64 run on the oracle's caches so one rounding flip does not compound
        kr, vr = [k.copy() for k in kc], [v.copy() for v in vc]
    return worst_out, worst_cache


@pytest.mark.parametrize("geo,lanes,cap,steps", [(SMALL, 3, 64, 3), (WINDOWED, 4, 32, 9), (SMALL, 1, 64, 3),
                                                   (SMALL, 8, 64, 3)])
def test_stack_oracle_matches_f64(geo, lanes, cap, steps):
    out, cache = _run_both(geo, 80, lanes, cap, steps)
    assert out < 2e-4, out  # an f16 activation rounding may land on the other side of a tie
    assert cache < 1e-3, cache


def test_stack_oracle_residual_identity_and_untouched_slots():
    geo = SMALL
    layers, fn = stack.random_weights(geo, 81)
    for L in layers:
        L["wo"] = np.zeros_like(L["wo"])
        L["down"] = np.zeros_like(L["down"])
    lanes, cap = 4, 16
    x, kc, vc = inputs(geo, 81, lanes, cap)
    before = [(k.copy(), v.copy()) for k, v in zip(kc, vc)]
    pos = np.array([0, 15, 7, 3], np.int32)
    out = oracle.stack_decode_f32(geo, layers, fn, x, kc, vc, pos)
    assert np.array_equal(out, oracle.rms_norm_f32(x, fn, geo.eps))
    for (k0, v0), k1, v1 in zip(before, kc, vc):
        for i, p in enumerate(pos):
            mask = np.ones(cap, bool)
            mask[p] = False
            assert np.array_equal(k0[i, :, mask], k1[i, :, mask]) and np.array_equal(v0[i, :, mask], v1[i, :, mask])
            assert not np.array_equal(k0[i, :, p], k1[i, :, p])


def test_stack_oracle_window_hides_old_positions():
    """With a window of w, cache entries older than pos - w + 1 cannot change the result."""
    geo = WINDOWED
    layers, fn = stack.random_weights(geo, 82)
    lanes, cap = 2, 32
    x, kc, vc = inputs(geo, 82, lanes, cap)
    pos = np.array([20, 9], np.int32)
    k2, v2 = [k.copy() for k in kc], [v.copy() for v in vc]
    for li in range(geo.layers):
        for i, p in enumerate(pos):
            old = p + 1 - geo.window
            k2[li][i, :, :old] = synth.f16_bits(np.float32(7.0))
            v2[li][i, :, :old] = synth.f16_bits(np.float32(-7.0))
    a = oracle.stack_decode_f32(geo, layers, fn, x, kc, vc, pos)
    b = oracle.stack_decode_f32(geo, layers, fn, x, k2, v2, pos)
    assert np.array_equal(a, b)


def test_stack_oracle_routes_by_lane_count():
    """One lane takes candle's f16 matmul (its projection outputs rounded to f16); eight lanes the
    skinny GEMM (f32 outputs): the same lane's result differs between the two batch sizes, and the
    eight-lane batch equals eight one-lane-compatible rows only up to that rounding."""
    geo = SMALL
    layers, fn = stack.random_weights(geo, 83)
    x, kc, vc = inputs(geo, 83, 8, 16)
    pos = np.arange(8, dtype=np.int32)
    k1, v1 = [k[:1].copy() for k in kc], [v[:1].copy() for v in vc]
    eight = oracle.stack_decode_f32(geo, layers, fn, x, kc, vc, pos)
    one = oracle.stack_decode_f32(geo, layers, fn, np.ascontiguousarray(x[:1]), k1, v1, pos[:1])
    assert not np.array_equal(one[0], eight[0])
    assert rel(one[0], eight[0])[1] < 2e-3
