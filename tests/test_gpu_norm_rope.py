"""RMSNorm, RoPE, QK-norm+RoPE+KV-append and KV append (a8-a11) on the GPU through the C ABI.

Bars: RoPE and both appends bit-exact against the oracle (the append must be, and RoPE's
products are rounded exactly as the oracle's); RMSNorm max-rel <= 1e-5 in f32 and within one
f16 ulp in f16 (the sum of squares is reduced in a different order); the fused QK kernel's q and
f32 k max-rel <= 1e-5, its cached k the RNE cast of its own f32 k and its cached v bit-exact;
every cache element outside the appended positions keeps its sentinel (qkrope.rs:245-257), and
the cached k is within one f16 ulp of the oracle's own cache bits. qkrope::apply's t-position form
is held to the reference test's three (b, t, start, lane offset) cases.
Shapes: config 2 (48 lanes, 16 q / 8 kv heads, D 128, cache [48, 8, 2048, 128], theta 1e6,
positions U[0, 2047]) and the reference test's (b, heads, n_kv, cap) = (8, 16, 8, 64).
"""
import numpy as np
import pytest
import torch

import oracle
from dtts import DttsError, ops, synth

from _util import f16_ulp_diff, rel, to_dev, to_host

pytestmark = pytest.mark.gpu

SENTINEL = 0x5555


@pytest.mark.parametrize("rows,dim", [(48, 1024), (8, 2048), (3, 7), (1, 64)])
def test_rms_norm_f32(dev, rows, dim):
    x = synth.normal(60, "x", (rows, dim))
    g = synth.uniform(60, "g", (dim,), 0.9, 1.1)
    got = to_host(ops.rms_norm(to_dev(x, dev), to_dev(g, dev), 1e-6))
    assert rel(got, oracle.rms_norm_f32(x, g, 1e-6))[1] < 1e-5


def test_rms_norm_f16_config2(dev):
    x = synth.f16_bits(synth.normal(61, "x", (48, 1, 1024)))
    g = synth.f16_bits(synth.uniform(61, "g", (1024,), 0.9, 1.1))
    got = to_host(ops.rms_norm(to_dev(x, dev), to_dev(g, dev), 1e-6))
    want = oracle.rms_norm_f16(x, g, 1e-6)
    assert f16_ulp_diff(got, want) <= 1
    assert rel(synth.from_f16_bits(got), synth.from_f16_bits(want))[1] < 1e-3


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_rope_config2_bit_exact(dev, dtype):
    c, s = oracle.rope_table_f32(2048, 128, 1e6)
    pos = synth.randint(62, "pos", (48,), 0, 2047).astype(np.int32)
    for heads in (16, 8):
        x = synth.normal(62, f"x{heads}", (48, heads, 128))
        if dtype == "f16":
            x = synth.f16_bits(x)
            want = oracle.rope_halfsplit_f16(x, c, s, pos)
        else:
            want = oracle.rope_halfsplit_f32(x, c, s, pos)
        got = to_host(ops.rope(to_dev(x, dev), to_dev(c, dev), to_dev(s, dev), pos))
        assert np.array_equal(got, want)


def _fill(shape, dev):
    return torch.full(shape, SENTINEL, dtype=torch.int16, device=dev).view(torch.float16)


def _untouched(cache_host, pos):
    mask = np.ones(cache_host.shape, bool)
    for bi, p in enumerate(pos):
        mask[bi, :, p] = False
    return np.all(cache_host[mask] == SENTINEL)


@pytest.mark.parametrize("b,heads,n_kv,cap", [(48, 16, 8, 2048), (8, 16, 8, 64), (4, 2, 1, 7)])
def test_qk_norm_rope_kv_append_f32(dev, b, heads, n_kv, cap):
    hd = 128
    c, s = oracle.rope_table_f32(cap, hd, 1e6)
    qkv = synth.normal(63, "qkv", (b, (heads + 2 * n_kv) * hd))
    norms = synth.uniform(63, "norms", (2, hd), 0.5, 1.5)
    pos = synth.randint(63, "pos", (b,), 0, cap - 1).astype(np.int32)
    kc, vc = _fill((b, n_kv, cap, hd), dev), _fill((b, n_kv, cap, hd), dev)
    q, k = ops.qk_norm_rope_kv_append(to_dev(qkv, dev), to_dev(norms, dev), to_dev(c, dev), to_dev(s, dev),
                                      pos, kc, vc, heads, 1e-6, f32_k=True)
    okc = np.full((b, n_kv, cap, hd), SENTINEL, np.uint16)
    ovc = okc.copy()
    want_q, want_k = oracle.qk_norm_rope_append_f32(qkv, norms, c, s, pos, okc, ovc, heads, n_kv, 1e-6)
    gq, gk = to_host(q), to_host(k)
    assert rel(gq, want_q)[1] < 1e-5
    assert rel(gk, want_k)[1] < 1e-5
    hk, hv = to_host(kc), to_host(vc)
    for bi in range(b):
        assert np.array_equal(hk[bi, :, pos[bi]], synth.f16_bits(gk[bi]))  # RNE of its own f32 k
        assert np.array_equal(hv[bi, :, pos[bi]], ovc[bi, :, pos[bi]])      # v: bit-exact
        # against the oracle's own cache bits: within one f16 ulp (its f32 k is within 1e-5)
        assert f16_ulp_diff(hk[bi, :, pos[bi]], okc[bi, :, pos[bi]]) <= 1
    assert _untouched(hk, pos) and _untouched(hv, pos)


def test_qk_norm_rope_kv_append_f16(dev):
    b, heads, n_kv, cap, hd = 48, 16, 8, 2048, 128
    c, s = oracle.rope_table_f32(cap, hd, 1e6)
    qkv = synth.f16_bits(synth.normal(64, "qkv", (b, (heads + 2 * n_kv) * hd)))
    norms = synth.uniform(64, "norms", (2, hd), 0.5, 1.5)
    pos = synth.randint(64, "pos", (b,), 0, cap - 1).astype(np.int32)
    kc, vc = _fill((b, n_kv, cap, hd), dev), _fill((b, n_kv, cap, hd), dev)
    q, k = ops.qk_norm_rope_kv_append(to_dev(qkv, dev), to_dev(norms, dev), to_dev(c, dev), to_dev(s, dev),
                                      pos, kc, vc, heads, 1e-6, f32_k=True)
    okc = np.full((b, n_kv, cap, hd), SENTINEL, np.uint16)
    ovc = okc.copy()
    want_q, want_k = oracle.qk_norm_rope_append_f32(synth.from_f16_bits(qkv), norms, c, s, pos, okc, ovc,
                                                    heads, n_kv, 1e-6)
    assert f16_ulp_diff(to_host(q), synth.f16_bits(want_q)) <= 1
    assert rel(to_host(k), want_k)[1] < 1e-5
    hk, hv = to_host(kc), to_host(vc)
    gk = to_host(k)
    for bi in range(b):
        assert np.array_equal(hk[bi, :, pos[bi]], synth.f16_bits(gk[bi]))
        assert np.array_equal(hv[bi, :, pos[bi]], ovc[bi, :, pos[bi]])
        assert f16_ulp_diff(hk[bi, :, pos[bi]], okc[bi, :, pos[bi]]) <= 1
    assert _untouched(hk, pos) and _untouched(hv, pos)


@pytest.mark.parametrize("b,t,start,off", [(8, 1, 37, 2), (4, 5, 0, 1), (4, 7, 10, 0)])
def test_qkrope_apply_reference_cases_on_a_lane_window(dev, b, t, start, off):
    """qkrope::apply's own test (crates/tts-nn/src/qkrope.rs:191-260): t positions from start on a
    lane window of a (b + 3)-lane cache; q and f32 k within rel 1e-5, f32 v within 1e-6 (here
    exact), the cached values within 1e-3 (here: v bit-exact, k within an ulp of the oracle's
    bits and the RNE of the kernel's own f32 k), nothing outside the window touched."""
    heads, n_kv, hd, cap, eps = 16, 8, 128, 64, 1e-6
    c, s = oracle.rope_table_f32(cap, hd, 1e6)
    norms = synth.uniform(65, "norms", (2, hd), 0.5, 1.5)
    qkv = synth.normal(65, f"qkv{b}.{t}", (b, t, (heads + 2 * n_kv) * hd))
    kc, vc = _fill((b + 3, n_kv, cap, hd), dev), _fill((b + 3, n_kv, cap, hd), dev)
    q, (k, v) = ops.qkrope_apply(to_dev(qkv, dev), to_dev(norms, dev), to_dev(c, dev), to_dev(s, dev),
                                 kc.narrow(0, off, b), vc.narrow(0, off, b), heads, start, eps, f32_kv=True)
    okc = np.full((b + 3, n_kv, cap, hd), SENTINEL, np.uint16)
    ovc = okc.copy()
    wq, (wk, wv) = oracle.qkrope_apply_f32(qkv, norms, c, s, okc[off:off + b], ovc[off:off + b], heads, start, eps)
    gq, gk, gv = to_host(q), to_host(k), to_host(v)
    assert gq.shape == (b, heads, t, hd) and gk.shape == gv.shape == (b, n_kv, t, hd)
    assert rel(gq, wq)[1] < 1e-5
    assert rel(gk, wk)[1] < 1e-5
    assert np.array_equal(gv, wv)
    hk, hv = to_host(kc), to_host(vc)
    win = (slice(off, off + b), slice(None), slice(start, start + t))
    assert np.array_equal(hk[win], synth.f16_bits(gk))
    assert f16_ulp_diff(hk[win], okc[win]) <= 1
    assert rel(synth.from_f16_bits(hk[win]), synth.from_f16_bits(okc[win]))[1] < 1e-3
    assert np.array_equal(hv[win], ovc[win])
    mask = np.ones(hk.shape, bool)
    mask[win] = False
    assert np.all(hk[mask] == SENTINEL) and np.all(hv[mask] == SENTINEL), "writes escaped the lane window"


def test_qkrope_apply_refuses_positions_past_the_cache(dev):
    heads, n_kv, hd, cap = 4, 2, 128, 16
    c, s = oracle.rope_table_f32(cap, hd, 1e6)
    qkv = to_dev(synth.normal(66, "qkv", (2, 5, (heads + 2 * n_kv) * hd)), dev)
    norms = to_dev(synth.uniform(66, "n", (2, hd), 0.5, 1.5), dev)
    kc, vc = _fill((2, n_kv, cap, hd), dev), _fill((2, n_kv, cap, hd), dev)
    with pytest.raises(DttsError, match="17 positions exceed 16"):
        ops.qkrope_apply(qkv, norms, to_dev(c, dev), to_dev(s, dev), kc, vc, heads, 12, 1e-6)
    torch.cuda.synchronize()
    assert np.all(to_host(kc) == SENTINEL) and np.all(to_host(vc) == SENTINEL)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_kv_append_bit_exact_config2(dev, dtype):
    b, n_kv, cap, hd = 48, 8, 2048, 128
    k = synth.normal(65, "k", (b, n_kv, hd))
    v = synth.normal(65, "v", (b, n_kv, hd))
    pos = synth.randint(65, "pos", (b,), 0, cap - 1).astype(np.int32)
    pos[0], pos[1] = 0, cap - 1  # both ends of the cache
    kc, vc = _fill((b, n_kv, cap, hd), dev), _fill((b, n_kv, cap, hd), dev)
    okc = np.full((b, n_kv, cap, hd), SENTINEL, np.uint16)
    ovc = okc.copy()
    if dtype == "f16":
        k, v = synth.f16_bits(k), synth.f16_bits(v)
        oracle.kv_append_f16(k, v, pos, okc, ovc)
    else:
        oracle.kv_append_f32(k, v, pos, okc, ovc)
    ops.kv_append(to_dev(k, dev), to_dev(v, dev), pos, kc, vc)
    assert np.array_equal(to_host(kc), okc)
    assert np.array_equal(to_host(vc), ovc)


def test_append_rejects_positions_past_capacity(dev):
    k = torch.zeros((2, 1, 8), device=dev)
    kc = _fill((2, 1, 4, 8), dev)
    with pytest.raises(DttsError, match="capacity"):
        ops.kv_append(k, k, [0, 4], kc, kc.clone())
    torch.cuda.synchronize()
    assert np.all(to_host(kc) == SENTINEL)  # nothing was enqueued
