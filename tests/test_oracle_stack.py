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


# The f32 and Q8_0 weight kinds (Stack::load's `how`, qwen3.rs:228-250): f32 caches, f32
# projections in and out, the composed QK route. Against the float64 restatement: the f32 and
# unquantized-activation kinds differ by f32 rounding only (measured 1.2e-7 to 2.7e-7); W8A8 may
# also differ by an activation code that f32 and float64 evaluations put on different sides of a
# rounding boundary, each worth one code step of one block (none at these seeds: 1.8e-7 to 2.7e-7).
@pytest.mark.parametrize("weight,bar", [("f32", 2e-6), ("q8_0_a32", 2e-6), ("q8_0", 1e-4)])
@pytest.mark.parametrize("geo,lanes,cap,steps", [(SMALL, 3, 64, 3), (WINDOWED, 4, 32, 5), (SMALL, 8, 64, 2)])
def test_stack_oracle_weight_kinds_match_f64(weight, bar, geo, lanes, cap, steps):
    seed = 82
    layers, fn = stack.random_weights(geo, seed)
    x, kc, vc = inputs(geo, seed, lanes, cap, weight=weight)
    start = synth.randint(seed, "stack.pos", (lanes,), 0, cap - steps).astype(np.int32)
    worst_out, worst_cache = 0.0, 0.0
    for s in range(steps):
        pos = start + s
        xs = x * np.float32(1.0 + 0.1 * s)
        kr, vr = [k.copy() for k in kc], [v.copy() for v in vc]
        got = oracle.stack_decode_f32(geo, layers, fn, xs, kc, vc, pos, weight=weight)
        want, kr, vr = stack_f64(geo, layers, fn, xs, kr, vr, pos, weight=weight)
        worst_out = max(worst_out, rel(got, want)[1])
        for li in range(geo.layers):
            for a, b in ((kc[li], kr[li]), (vc[li], vr[li])):
                worst_cache = max(worst_cache, rel(a, b)[1])
    assert worst_out < bar, worst_out
    assert worst_cache < bar, worst_cache


def test_stack_oracle_weight_kinds_differ():
    """The kinds are distinguishable: on one step, f32 weights, the Q8_0 blocks with f32 activations
    and W8A8 give results further apart than the bars above (so a kind run as another fails)."""
    geo, lanes, cap = SMALL, 4, 16
    layers, fn = stack.random_weights(geo, 83)
    outs = {}
    for weight in ("f32", "q8_0_a32", "q8_0"):
        x, kc, vc = inputs(geo, 83, lanes, cap, weight=weight)
        outs[weight] = oracle.stack_decode_f32(geo, layers, fn, x, kc, vc, np.array([0, 5, 9, 15], np.int32),
                                               weight=weight)
    assert rel(outs["q8_0_a32"], outs["f32"])[1] > 1e-3
    assert rel(outs["q8_0"], outs["q8_0_a32"])[1] > 1e-3


def test_stack_oracle_f32_kinds_residual_identity_and_exact_cache():
    """With zero output and down projections the f32-cache step returns rms_norm(x) exactly, and the
    f32 caches hold each lane's roped k and its v at its position only."""
    geo = SMALL
    layers, fn = stack.random_weights(geo, 84)
    for L in layers:
        L["wo"] = np.zeros_like(L["wo"])
        L["down"] = np.zeros_like(L["down"])
    lanes, cap = 4, 16
    x, kc, vc = inputs(geo, 84, lanes, cap, weight="f32")
    before = [(k.copy(), v.copy()) for k, v in zip(kc, vc)]
    pos = np.array([0, 15, 7, 3], np.int32)
    out = oracle.stack_decode_f32(geo, layers, fn, x, kc, vc, pos, weight="f32")
    assert np.array_equal(out, oracle.rms_norm_f32(x, fn, geo.eps))
    for (k0, v0), k1, v1 in zip(before, kc, vc):
        for i, p in enumerate(pos):
            k0[i, :, p], v0[i, :, p] = k1[i, :, p], v1[i, :, p]
        assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
    # layer 0's v is the v rows of the f32 projection of rms_norm(x), stored unrounded
    a = oracle.rms_norm_f32(x, layers[0]["attn_norm"], geo.eps)
    v_rows = layers[0]["wv"]
    want_v = (a.astype(np.float64) @ v_rows.astype(np.float64).T).astype(np.float32).reshape(lanes, geo.n_kv, geo.head_dim)
    for i, p in enumerate(pos):
        assert np.array_equal(vc[0][i, :, p], want_v[i])
