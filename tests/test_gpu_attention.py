"""dtts_decode_attention_{f16,f32} against the oracle's restatement of attn::decode_attention's
CPU path (crates/tts-nn/src/attn.rs:18-73), at the reference test's own shapes and bar
(attn.rs:389-420: q ~ 0.1 N(0,1), f16 caches ~ N(0,1), abs_and_rel's rel < 1e-5), plus per-lane
spans and windows (the batched-decode generalisation), f32 caches, D = 64, gqa up to 8, the
config-2 geometry, and the argument checks. The caches must come back untouched."""
import numpy as np
import pytest
import torch

import oracle
from dtts import DttsError, ops, synth

from _util import rel, to_dev, to_host

pytestmark = pytest.mark.gpu

REF_SHAPES = [(48, 8, 2, 400, 250, 0), (40, 8, 2, 17, 3, 0), (8, 8, 2, 300, 211, 90), (4, 8, 1, 64, 33, 0)]


def _inputs(seed, b, n_kv, gqa, cap, hd=128, f16=True):
    q = synth.normal(seed, "q", (b, n_kv, gqa, hd), 0, 0.1)
    k = synth.normal(seed, "k", (b, n_kv, cap, hd))
    v = synth.normal(seed, "v", (b, n_kv, cap, hd))
    if f16:
        k, v = synth.f16_bits(k), synth.f16_bits(v)
    return q, k, v


def _run(dev, q, k, v, span, ws, workspace=None):
    qd, kd, vd = to_dev(q, dev), to_dev(k, dev), to_dev(v, dev)
    out = ops.decode_attention(qd, kd, vd, span, ws, workspace=workspace)
    torch.cuda.synchronize()
    assert np.array_equal(to_host(kd), k) and np.array_equal(to_host(vd), v), "cache modified"
    return to_host(out)


@pytest.mark.parametrize("b,n_kv,gqa,cap,span,ws", REF_SHAPES)
def test_decode_attention_reference_shapes(dev, b, n_kv, gqa, cap, span, ws):
    q, k, v = _inputs(70, b, n_kv, gqa, cap)
    got = _run(dev, q, k, v, span, ws)
    want = oracle.decode_attention_f32(q, k, v, span, ws)
    assert rel(got, want)[1] < 1e-5


@pytest.mark.parametrize("hd,gqa,f16", [(128, 2, False), (64, 1, True), (64, 4, False), (128, 8, True),
                                        (128, 4, True)])
def test_decode_attention_per_lane_windows(dev, hd, gqa, f16):
    b, n_kv, cap = 7, 3, 300
    q, k, v = _inputs(71, b, n_kv, gqa, cap, hd, f16)
    span = np.array([1, 300, 17, 129, 2, 64, 250], np.int32)
    ws = np.array([0, 10, 16, 0, 1, 63, 3], np.int32)
    got = _run(dev, q, k, v, span, ws)
    want = oracle.decode_attention_f32(q, k, v, span, ws)
    assert rel(got, want)[1] < 1e-5


def test_decode_attention_ignores_slots_outside_the_window(dev):
    b, n_kv, gqa, cap = 4, 8, 2, 96
    q, k, v = _inputs(72, b, n_kv, gqa, cap)
    span, ws = 70, 20
    big = synth.f16_bits(np.float32(3e4))
    for t in (k, v):
        t[:, :, :ws] = big
        t[:, :, span:] = big
    got = _run(dev, q, k, v, span, ws)
    assert np.all(np.abs(got) < 10)
    assert rel(got, oracle.decode_attention_f32(q, k, v, span, ws))[1] < 1e-5


def test_decode_attention_config2_geometry(dev):
    """48 lanes, 16 query / 8 kv heads, D 128, cap 2048, each lane at its own position."""
    b, n_kv, gqa, cap = 48, 8, 2, 2048
    q, k, v = _inputs(73, b, n_kv, gqa, cap)
    span = synth.randint(73, "pos", (b,), 0, cap - 1).astype(np.int32) + 1
    got = _run(dev, q, k, v, span, 0)
    assert rel(got, oracle.decode_attention_f32(q, k, v, span, 0))[1] < 1e-5


def test_decode_attention_split_and_single_pass_agree(dev):
    """Windows past 512 positions split over workgroups when a workspace is given (merged by a
    second launch); without room for every chunk's state, one workgroup takes the whole span.
    Windows of 1500 (three chunks), 513 (a last chunk of one position), 700, 556 and 1."""
    b, n_kv, gqa, cap = 5, 4, 2, 1500
    q, k, v = _inputs(74, b, n_kv, gqa, cap)
    span = np.array([1500, 513, 1000, 600, 1], np.int32)
    ws = np.array([0, 0, 300, 44, 0], np.int32)
    need = ops.decode_attention_workspace_bytes(b, n_kv, gqa, 128, int(np.max(span - ws)))
    assert need == b * n_kv * 3 * gqa * 130 * 4  # three chunks of 512 for the 1500-position window
    want = oracle.decode_attention_f32(q, k, v, span, ws)
    split = _run(dev, q, k, v, span, ws)
    single = _run(dev, q, k, v, span, ws, workspace=torch.empty(need - 16, dtype=torch.uint8, device=dev))
    assert rel(split, want)[1] < 1e-5 and rel(single, want)[1] < 1e-5


def test_decode_attention_rejects_bad_arguments(dev):
    q = torch.zeros((2, 1, 2, 128), dtype=torch.float32, device=dev)
    k = torch.zeros((2, 1, 16, 128), dtype=torch.float16, device=dev)
    with pytest.raises(DttsError, match="exceeds capacity"):
        ops.decode_attention(q, k, k, 17)
    with pytest.raises(DttsError, match="empty range"):
        ops.decode_attention(q, k, k, 5, 5)
    with pytest.raises(DttsError, match="head_dim"):
        ops.decode_attention(q[..., :96].contiguous(), k[..., :96].contiguous(), k[..., :96].contiguous(), 4)
    big_q = torch.zeros((257, 1, 1, 64), dtype=torch.float32, device=dev)
    big_k = torch.zeros((257, 1, 4, 64), dtype=torch.float16, device=dev)
    with pytest.raises(DttsError, match="lanes"):
        ops.decode_attention(big_q, big_k, big_k, 4)


def test_decode_attention_split_past_eight_chunks(dev):
    """The merge requests up to eight chunks' states at once and loops past that: windows of
    4700 (ten chunks of 512), 4096 (eight) and 4097 (nine, the last of one position)."""
    b, n_kv, gqa, cap = 3, 2, 2, 4700
    q, k, v = _inputs(75, b, n_kv, gqa, cap)
    span = np.array([4700, 4096, 4200], np.int32)
    ws = np.array([0, 0, 103], np.int32)
    want = oracle.decode_attention_f32(q, k, v, span, ws)
    split = _run(dev, q, k, v, span, ws)
    assert rel(split, want)[1] < 1e-5
