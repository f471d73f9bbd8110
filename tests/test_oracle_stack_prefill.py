"""Pins the oracle's prefill branch (oracle.stack_prefill_f32: Stack::forward at t >= 2,
crates/qwen3tts/src/qwen3.rs:294-467) against an independent float64 restatement with the f16
roundings at the same points (including Proj::Half's row-count routing: f32 outputs from the
skinny GEMM, f16 outputs from candle's matmul), with and without QK-norm, LayerScale, a sliding
window and a cache prefix; and against what the mathematics fixes: later positions cannot change
earlier rows (causality), with zero output and down projections the result is rms_norm(x)
exactly and only slots start .. start + t - 1 are written, and cache entries the window excludes
cannot matter."""
import numpy as np
import pytest

import oracle
from dtts import stack, synth

from _stack_ref import SMALL, WINDOWED, inputs, stack_prefill_f64
from _util import rel


def _case(geo, seed, lanes, t, start, cap):
    layers, fn = stack.random_weights(geo, seed)
    _, kc, vc = inputs(geo, seed, lanes, cap)
    x = synth.normal(seed, "prefill.x", (lanes, t, geo.dim))
    return layers, fn, x, kc, vc


@pytest.mark.parametrize("geo,lanes,t,start,cap", [
    (SMALL, 3, 5, 0, 64),      # 15 rows: the f16-output matmul
    (SMALL, 8, 2, 0, 64),      # 16 rows: the skinny GEMM's f32 outputs
    (SMALL, 4, 3, 10, 64),     # a cache prefix
    (WINDOWED, 2, 9, 6, 32),   # windows reaching back into the prefix, no QK-norm, LayerScale
])
def test_prefill_oracle_matches_f64(geo, lanes, t, start, cap):
    layers, fn, x, kc, vc = _case(geo, 90, lanes, t, start, cap)
    kr, vr = [k.copy() for k in kc], [v.copy() for v in vc]
    got = oracle.stack_prefill_f32(geo, layers, fn, x, kc, vc, start)
    want, kr, vr = stack_prefill_f64(geo, layers, fn, x, kr, vr, start)
    # measured 3e-6 .. 1.3e-4 (an f16 rounding of an activation may land on the other side of a
    # tie); dropping the window mask alone gives 1.2e-2
    assert rel(got, want)[1] < 5e-4
    for li in range(geo.layers):
        for a, b in ((kc[li], kr[li]), (vc[li], vr[li])):
            assert rel(synth.from_f16_bits(a), synth.from_f16_bits(b))[1] < 2e-3


def test_prefill_oracle_is_causal():
    """Row ti depends on positions <= start + ti only: a shorter prefill gives the same rows (both
    with the f16-output projections: 12 and 18 rows)."""
    geo = SMALL
    layers, fn, x, kc, vc = _case(geo, 91, 3, 6, 5, 64)
    k2, v2 = [k.copy() for k in kc], [v.copy() for v in vc]
    full = oracle.stack_prefill_f32(geo, layers, fn, x, kc, vc, 5)
    part = oracle.stack_prefill_f32(geo, layers, fn, np.ascontiguousarray(x[:, :4]), k2, v2, 5)
    assert rel(part, full[:, :4])[1] < 1e-6
    for li in range(geo.layers):
        assert np.array_equal(kc[li][:, :, :9], k2[li][:, :, :9])


def test_prefill_oracle_residual_identity_and_untouched_slots():
    geo = SMALL
    layers, fn, x, kc, vc = _case(geo, 92, 2, 4, 7, 16)
    for L in layers:
        L["wo"] = np.zeros_like(L["wo"])
        L["down"] = np.zeros_like(L["down"])
    before = [(k.copy(), v.copy()) for k, v in zip(kc, vc)]
    out = oracle.stack_prefill_f32(geo, layers, fn, x, kc, vc, 7)
    assert np.array_equal(out, oracle.rms_norm_f32(x, fn, geo.eps))
    for (k0, v0), k1, v1 in zip(before, kc, vc):
        keep = np.ones(16, bool)
        keep[7:11] = False
        assert np.array_equal(k0[:, :, keep], k1[:, :, keep]) and np.array_equal(v0[:, :, keep], v1[:, :, keep])
        assert not np.array_equal(k0[:, :, 7:11], k1[:, :, 7:11])


def test_prefill_oracle_window_hides_old_positions():
    """With window w the first new position sees keys from start + 1 - w on: older cache entries
    cannot change the result."""
    geo = WINDOWED
    layers, fn, x, kc, vc = _case(geo, 93, 2, 3, 12, 32)
    k2, v2 = [k.copy() for k in kc], [v.copy() for v in vc]
    old = 12 + 1 - geo.window
    for li in range(geo.layers):
        k2[li][:, :, :old] = synth.f16_bits(np.float32(7.0))
        v2[li][:, :, :old] = synth.f16_bits(np.float32(-7.0))
    a = oracle.stack_prefill_f32(geo, layers, fn, x, kc, vc, 12)
    b = oracle.stack_prefill_f32(geo, layers, fn, x, k2, v2, 12)
    assert np.array_equal(a, b)


def test_prefill_oracle_shared_prefix_split():
    """validate.rs's "prefill.shared" claim (crates/qwen3tts/src/bin/validate.rs:210-245): the voice's
    positions prefilled once for one lane and copied into every lane's cache, then the rest of each
    prompt prefilled from there, give each lane's last hidden state within 1e-4 of one whole
    prefill (the prefix enters as f16 cache entries instead of f32)."""
    geo = SMALL
    layers, fn = stack.random_weights(geo, 94)
    lanes, n, shared, cap = 2, 12, 5, 16
    x = synth.normal(94, "prefill.shared.x", (lanes, n, geo.dim))
    x[1, :shared] = x[0, :shared]
    _, kc, vc = inputs(geo, 94, lanes, cap, fill=False)
    whole = oracle.stack_prefill_f32(geo, layers, fn, x, kc, vc, 0)
    _, k1, v1 = inputs(geo, 94, 1, cap, fill=False)
    oracle.stack_prefill_f32(geo, layers, fn, np.ascontiguousarray(x[:1, :shared]), k1, v1, 0)
    _, ks, vs = inputs(geo, 94, lanes, cap, fill=False)
    for li in range(geo.layers):
        ks[li][:, :, :shared] = k1[li][:, :, :shared]
        vs[li][:, :, :shared] = v1[li][:, :, :shared]
    split = oracle.stack_prefill_f32(geo, layers, fn, np.ascontiguousarray(x[:, shared:]), ks, vs, shared)
    assert rel(split[:, -1], whole[:, -1])[1] < 1e-4
    assert not np.array_equal(split[:, -1], whole[:, -1])  # the prefix's f16 rounding is visible
