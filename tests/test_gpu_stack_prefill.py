"""dtts_stack_prefill (Stack::forward at t >= 2, the prefill branch of crates/qwen3tts/src/
qwen3.rs:294-467) against the oracle's restatement (oracle.stack_prefill_f32) on the same seeded
weights, inputs and cache prefix: the normed outputs within max-rel 5e-4 (f32 sums in another
order, and an f16-rounded projection output may land on the other side of a tie), every cache
entry written at start .. start + t - 1 within max-rel 1e-3 and every other entry bit-identical.
Cases cover both routes of Proj::Half (the skinny GEMM's f32 outputs at <= 48 rows that are a
multiple of 8, the f16 matmul's outputs otherwise: from the A-sharing kernel up to 128 rows,
including the code predictor's 48 lanes x 2, and from the tile kernel past that),
a cache prefix, windows reaching into it, spans longer than a wave, and a decode step after the
prefill; plus the argument checks."""
from dataclasses import replace

import numpy as np
import pytest
import torch

import oracle
from dtts import DttsError, stack, synth

from _stack_ref import SMALL, WINDOWED, inputs, stack_prefill_f64
from _util import rel, to_dev, to_host

pytestmark = pytest.mark.gpu

LONG = replace(SMALL, capacity=160)


def _setup(dev, geo, seed, lanes, t, cap):
    layers, fn = stack.random_weights(geo, seed)
    _, kc, vc = inputs(geo, seed, lanes, cap)
    x = synth.normal(seed, "prefill.x", (lanes, t, geo.dim))
    st = stack.Stack(geo, layers, fn, dev)
    state = st.new_state(lanes, cap)
    for i in range(geo.layers):
        state.k[i].copy_(to_dev(kc[i], dev))
        state.v[i].copy_(to_dev(vc[i], dev))
    return layers, fn, x, kc, vc, st, state


def _check(geo, state, kc_before, vc_before, kc_want, vc_want, start, t):
    for li in range(geo.layers):
        for dev_t, want, old in ((state.k[li], kc_want[li], kc_before[li]), (state.v[li], vc_want[li], vc_before[li])):
            g = to_host(dev_t)
            keep = np.ones(g.shape[2], bool)
            keep[start:start + t] = False
            assert np.array_equal(g[:, :, keep], old[:, :, keep]), "a cache slot outside the new positions changed"
            assert rel(synth.from_f16_bits(g[:, :, ~keep]), synth.from_f16_bits(want[:, :, ~keep]))[1] < 1e-3


@pytest.mark.parametrize("geo,lanes,t,start,cap", [
    (SMALL, 3, 5, 0, 64),       # 15 rows: f16-output projections
    (SMALL, 8, 2, 0, 64),       # 16 rows: the skinny GEMM's f32 outputs
    (SMALL, 24, 2, 0, 32),      # 48 rows: skinny, the A-sharing kernel's k ranges
    (SMALL, 48, 2, 0, 17),      # the code predictor's per-frame prefill: 96 rows, f16 outputs
    (SMALL, 4, 3, 10, 64),      # a cache prefix
    (LONG, 2, 20, 100, 160),    # spans of 101 .. 120 keys (more than a wave)
    (WINDOWED, 2, 9, 6, 32),    # windows into the prefix, no QK-norm (scaled scores), D = 64
    (WINDOWED, 1, 30, 0, 32),   # t longer than the window
    (SMALL, 64, 2, 0, 16),      # 128 rows: the A-sharing kernel's largest row block
    (SMALL, 43, 3, 0, 16),      # 129 rows: the first count on the tile kernel
    (SMALL, 3, 50, 0, 64),      # 150 rows: the tile kernel's f16 outputs
    (WINDOWED, 5, 30, 2, 32),   # 150 rows, windowed
    # t >= 16: 32-query blocks on the f32 matrix cores
    (LONG, 2, 100, 20, 160),    # a 20-key f16 prefix: the first key block crosses start; a 4-query last block
    (replace(WINDOWED, capacity=96), 2, 70, 9, 96),  # D = 64, windows of 5 inside 32-query blocks, scaled scores
    # its LDS is the key blocks' scores (4352 B each) plus 512 B of static maxima and sums, within 64 KB
    (replace(SMALL, capacity=512), 1, 64, 380, 512),  # 444 keys: 14 key blocks
    (replace(SMALL, capacity=512), 1, 64, 384, 512),  # 448 keys: 14 full key blocks, 61,440 B, the most it takes
    (replace(SMALL, capacity=512), 1, 64, 416, 512),  # 480 keys: 15 blocks (65,792 B), the per-wave kernel
    (replace(SMALL, capacity=512), 1, 40, 460, 512),  # 500 keys: the per-wave kernel again
])
def test_prefill_matches_oracle(dev, geo, lanes, t, start, cap):
    layers, fn, x, kc, vc, st, state = _setup(dev, geo, 95, lanes, t, cap)
    kb, vb = [k.copy() for k in kc], [v.copy() for v in vc]
    print(f"prefill lanes={lanes} t={t} start={start} cap={cap} dim={geo.dim}", flush=True)
    want = oracle.stack_prefill_f32(geo, layers, fn, x, kc, vc, start)
    got = st.prefill(to_dev(x, dev), state, start)
    torch.cuda.synchronize()
    got = to_host(got)
    assert rel(got, want)[1] < 5e-4, rel(got, want)
    _check(geo, state, kb, vb, kc, vc, start, t)


def test_prefill_talker_widths(dev):
    """The talker's widths (dim 2048, 16/8 heads, D 128, ffn 6144), 2 of its 28 layers, 2 lanes x
    64 prompt positions: two 32-query blocks per (lane, head) on the matrix cores. Bar 1e-3 against
    the oracle, as for the decode step at these widths (an f16 rounding on the other side of a tie
    separates outputs by up to an f16 ulp of the rounded activation, 4.9e-4 relative), and the GPU
    no further from a float64 evaluation with the same f16 rounding points than the oracle is,
    within 2e-4."""
    geo = replace(stack.TALKER, layers=2, capacity=128)
    lanes, t, start = 2, 64, 0
    layers, fn, x, kc, vc, st, state = _setup(dev, geo, 96, lanes, t, 128)
    kb, vb = [k.copy() for k in kc], [v.copy() for v in vc]
    exact, _, _ = stack_prefill_f64(geo, layers, fn, x, kc, vc, start)
    want = oracle.stack_prefill_f32(geo, layers, fn, x, kc, vc, start)
    got = to_host(st.prefill(to_dev(x, dev), state, start))
    torch.cuda.synchronize()
    d_oracle, d_gpu, d_both = rel(want, exact)[1], rel(got, exact)[1], rel(got, want)[1]
    print(f"max-rel: oracle-f64 {d_oracle:.2e}, gpu-f64 {d_gpu:.2e}, gpu-oracle {d_both:.2e}")
    assert d_both < 1e-3
    assert d_gpu <= d_oracle + 2e-4
    _check(geo, state, kb, vb, kc, vc, start, t)


def test_prefill_then_decode(dev):
    """The per-frame pattern of the code predictor: a prefill of 2 positions, then decode steps
    over the cache it wrote (each side continuing from the GPU's cache)."""
    geo, lanes, cap = SMALL, 8, 17
    layers, fn, x, kc, vc, st, state = _setup(dev, geo, 96, lanes, 2, cap)
    for i in range(geo.layers):
        state.k[i].zero_()
        state.v[i].zero_()
    st.prefill(to_dev(x, dev), state, 0)
    torch.cuda.synchronize()
    kc = [to_host(k) for k in state.k]
    vc = [to_host(v) for v in state.v]
    for step in range(3):
        xs = synth.normal(96, f"prefill.step{step}", (lanes, geo.dim))
        pos = np.full(lanes, 2 + step, np.int32)
        want = oracle.stack_decode_f32(geo, layers, fn, xs, kc, vc, pos)
        got = to_host(st.decode(to_dev(xs, dev), state, pos))
        assert rel(got, want)[1] < 2e-4
        kc = [to_host(k) for k in state.k]
        vc = [to_host(v) for v in state.v]


def test_prefill_rejects_bad_arguments(dev):
    geo = SMALL
    st = stack.Stack(geo, *stack.random_weights(geo, 97), dev)
    state = st.new_state(2, 16)
    x = torch.zeros((2, 4, geo.dim), dtype=torch.float32, device=dev)
    with pytest.raises(DttsError, match="t >= 2"):
        st.prefill(torch.zeros((2, 1, geo.dim), dtype=torch.float32, device=dev), state, 0)
    with pytest.raises(DttsError, match="exceeds cache capacity 16"):
        st.prefill(x, state, 13)
    small = torch.empty(256, dtype=torch.uint8, device=dev)
    with pytest.raises(DttsError, match="workspace"):
        st.prefill(x, state, 0, workspace=small)
    before = [to_host(k) for k in state.k]
    torch.cuda.synchronize()
    assert all(np.array_equal(a, to_host(b)) for a, b in zip(before, state.k))


def test_prefill_shared_prefix_split(dev):
    """prefill_batch's shared voice prefix (crates/qwen3tts/src/talker.rs:1076-1113) as validate.rs
    checks it (bin/validate.rs:210-245): one lane's prefix prefilled once and copied into every
    lane's cache, then each lane's rest prefilled from `shared` on; each lane's last hidden state
    within 1e-4 of one whole prefill, and the split run matches the oracle's split run."""
    geo = SMALL
    layers, fn = stack.random_weights(geo, 94)
    lanes, n, shared, cap = 2, 12, 5, 16
    x = synth.normal(94, "prefill.shared.x", (lanes, n, geo.dim))
    x[1, :shared] = x[0, :shared]
    st = stack.Stack(geo, layers, fn, dev)
    whole_state = st.new_state(lanes, cap)
    whole = to_host(st.prefill(to_dev(x, dev), whole_state, 0))
    one = st.new_state(1, cap)
    st.prefill(to_dev(np.ascontiguousarray(x[:1, :shared]), dev), one, 0)
    split_state = st.new_state(lanes, cap)
    for li in range(geo.layers):  # State::fill_prefix: the one lane's prefix into every lane
        split_state.k[li][:, :, :shared].copy_(one.k[li][:, :, :shared].expand(lanes, -1, -1, -1))
        split_state.v[li][:, :, :shared].copy_(one.v[li][:, :, :shared].expand(lanes, -1, -1, -1))
    split = to_host(st.prefill(to_dev(np.ascontiguousarray(x[:, shared:]), dev), split_state, shared))
    torch.cuda.synchronize()
    assert rel(split[:, -1], whole[:, -1])[1] < 1e-4
    _, k1, v1 = inputs(geo, 94, 1, cap, fill=False)
    oracle.stack_prefill_f32(geo, layers, fn, np.ascontiguousarray(x[:1, :shared]), k1, v1, 0)
    _, ks, vs = inputs(geo, 94, lanes, cap, fill=False)
    for li in range(geo.layers):
        ks[li][:, :, :shared] = k1[li][:, :, :shared]
        vs[li][:, :, :shared] = v1[li][:, :, :shared]
    want = oracle.stack_prefill_f32(geo, layers, fn, np.ascontiguousarray(x[:, shared:]), ks, vs, shared)
    assert rel(split, want)[1] < 5e-4
