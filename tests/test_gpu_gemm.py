"""Decode-shape f16 GEMMs, SwiGLU and Q8_0 projections (a12-a15) through the C ABI.

Bars: f16 GEMM max-abs <= 2e-2 at unit-scale activations and max-rel (abs_and_rel) <= 1e-4
against the oracle's f32-accumulated GEMM of the same f16 operands (the reference's own check,
crates/tts-nn/src/skinny.rs:175-202, allows 2e-3 against candle); SwiGLU within 2e-6 of f64
scaled by max(|g u|, 1) (fused.rs:2310-2322); Q8_0 dequant bit-exact; W8A8 max-rel <= 1e-5
against the oracle's vec_dot restatement (same integer dots and scale products, different f32
summation order); W8A16 max-abs <= 2e-2 and max-rel <= 1e-3 against f64 on the dequantized
weights. Shapes: the reference test's, and configs 3 and 4.
"""
import numpy as np
import pytest
import torch

import oracle
from dtts import ops, synth

from _util import rel, to_dev, to_host

pytestmark = pytest.mark.gpu

SKINNY = [(48, 2048, 4096), (48, 2048, 6144), (48, 6144, 2048), (48, 1024, 3072), (40, 3072, 1024),
          (32, 1024, 2048), (8, 1024, 4096),                        # skinny.rs:175-202
          (48, 1024, 4096), (48, 3072, 1024),                       # config 3
          (1, 1024, 1024), (64, 128, 48), (5, 100, 24), (3, 64, 16)]  # edges + the direct kernel


def _ab(seed, m, k, n):
    a = synth.f16_bits(synth.normal(seed, "a", (m, k)))
    w = synth.f16_bits(synth.normal(seed, "w", (n, k), 0, 0.02))  # [out, in]
    return a, w


@pytest.mark.parametrize("m,k,n", SKINNY)
def test_gemm_nt_and_kn_match_oracle(dev, m, k, n):
    a, w = _ab(80, m, k, n)
    b_kn = np.ascontiguousarray(w.T)
    want = oracle.gemm_f16_f32acc(a, b_kn)
    for got in (to_host(ops.matmul_nt(to_dev(a, dev), to_dev(w, dev))),
                to_host(ops.skinny_matmul(to_dev(a, dev), to_dev(b_kn, dev)))):
        ab, rl = rel(got, want)
        assert ab <= 2e-2 and rl <= 1e-4, (ab, rl)


@pytest.mark.parametrize("m,k,n,gateup", [(48, 3072, 1024, False), (40, 6144, 1024, False), (48, 3072, 512, True),
                                           (8, 8192, 256, False)])
def test_gemm_k_split_over_workgroups_matches_single_pass(dev, m, k, n, gateup):
    """Few output columns: with a workspace, k splits over workgroups too and a second launch sums
    the splits in order; without one, each column group's workgroup takes all of k."""
    need = ops.gemm_workspace_bytes(m, k, n, gateup)
    assert need > 0
    a, w = _ab(82, m, k, 2 * n if gateup else n)
    ad, wd = to_dev(a, dev), to_dev(w, dev)
    fn = ops.gateup_silu if gateup else ops.matmul_nt
    split = to_host(fn(ad, wd, torch.empty(need, dtype=torch.uint8, device=dev)))
    single = to_host(fn(ad, wd, torch.empty(1, dtype=torch.uint8, device=dev)))
    gu = oracle.gemm_f16_f32acc(a, np.ascontiguousarray(w.T))
    want = oracle.swiglu_mul_f32(gu[:, :n].copy(), gu[:, n:].copy()) if gateup else gu
    for got in (split, single):
        ab, rl = rel(got, want)
        assert ab <= 2e-2 and rl <= 1e-4, (ab, rl)


def test_short_k_projections_take_one_launch_without_workspace():
    """k * ceil(m/16) <= 3072 (config 3's QKV and gate|up, the predictor's projections): one
    launch with k over the waves of a workgroup, so the entry points ask for no workspace; the
    talker's k = 2048 at 48 rows and config 3's down projection keep the split and its merge."""
    for m, k, n, gu in ((48, 1024, 4096, False), (48, 1024, 3072, True), (8, 3072, 1024, False),
                        (16, 2048, 2048, False), (64, 128, 48, False)):
        assert ops.gemm_workspace_bytes(m, k, n, gu) == 0, (m, k, n, gu)
    for m, k, n, gu in ((48, 3072, 1024, False), (48, 2048, 4096, False), (48, 2048, 6144, True)):
        assert ops.gemm_workspace_bytes(m, k, n, gu) > 0, (m, k, n, gu)


@pytest.mark.parametrize("m,k,ffn", [(48, 1024, 3072), (8, 1024, 3072), (48, 2048, 6144), (3, 64, 16)])
def test_gateup_silu_matches_oracle(dev, m, k, ffn):
    a, w = _ab(81, m, k, 2 * ffn)
    got = to_host(ops.gateup_silu(to_dev(a, dev), to_dev(w, dev)))
    gu = oracle.gemm_f16_f32acc(a, np.ascontiguousarray(w.T))
    want = oracle.swiglu_mul_f32(gu[:, :ffn].copy(), gu[:, ffn:].copy())
    ab, rl = rel(got, want)
    assert ab <= 2e-2 and rl <= 1e-4, (ab, rl)


def test_swiglu_sweep_accuracy(dev):
    n = 8 * 4096
    gs = (-30.0 + 60.0 * (np.arange(n) % 4096) / 4095).astype(np.float32)
    us = (-4.0 + 8.0 * (np.arange(n) % 4096) / 4095).astype(np.float32)
    got = to_host(ops.swiglu_mul(to_dev(gs, dev), to_dev(us, dev)))
    g64, u64 = gs.astype(np.float64), us.astype(np.float64)
    want = g64 / (1.0 + np.exp(-g64)) * u64
    assert np.max(np.abs(got - want) / np.maximum(np.abs(g64 * u64), 1.0)) < 2e-6


Q8_SHAPES = [(m, k, n) for (k, n) in ((1024, 6144), (3072, 1024)) for m in (1, 8, 48)]


@pytest.mark.parametrize("k,n", [(1024, 6144), (3072, 1024)])
def test_q8_0_dequant_bit_exact(dev, k, n):
    w = synth.normal(82, "w", (n, k), 0, 0.02)
    blocks = ops.q8_0_quantize(w)
    got = to_host(ops.q8_0_dequantize(torch.from_numpy(blocks).to(dev), k))
    assert np.array_equal(got, oracle.q8_0_dequantize(blocks, k))


@pytest.mark.parametrize("m,k,n", Q8_SHAPES)
def test_q8_0_matmul(dev, m, k, n):
    w = synth.normal(83, "w", (n, k), 0, 0.02)
    blocks = ops.q8_0_quantize(w)
    xb = synth.f16_bits(synth.normal(83, "x", (m, k)))
    x = synth.from_f16_bits(xb)
    xd, bd = to_dev(xb, dev), torch.from_numpy(blocks).to(dev)
    got8 = to_host(ops.q8_0_matmul(xd, bd, "w8a8"))
    assert rel(got8, oracle.q8_0_matmul_w8a8(x, blocks))[1] <= 1e-5
    got16 = to_host(ops.q8_0_matmul(xd, bd, "w8a16"))
    ab, rl = rel(got16, oracle.q8_0_matmul_f64(x, blocks))
    assert ab <= 2e-2 and rl <= 1e-3, (ab, rl)


@pytest.mark.parametrize("m,k,n", Q8_SHAPES + [(33, 512, 128)])
def test_q8_0_matmul_workspace_path(dev, m, k, n):
    """dtts_gemm_q8_0_ws: for m > 16, workgroups of 64 columns share the activation slab in LDS and
    k splits into ranges merged in order -- the same bars against the oracle as the workspace-free
    kernel, and without room for the ranges (or at m <= 16) it is that kernel bit for bit."""
    w = synth.normal(84, "w", (n, k), 0, 0.02)
    blocks = ops.q8_0_quantize(w)
    xb = synth.f16_bits(synth.normal(84, "x", (m, k)))
    x = synth.from_f16_bits(xb)
    xd, bd = to_dev(xb, dev), torch.from_numpy(blocks).to(dev)
    got8 = to_host(ops.q8_0_matmul(xd, bd, "w8a8", workspace="auto"))
    assert rel(got8, oracle.q8_0_matmul_w8a8(x, blocks))[1] <= 1e-5
    got16 = to_host(ops.q8_0_matmul(xd, bd, "w8a16", workspace="auto"))
    ab, rl = rel(got16, oracle.q8_0_matmul_f64(x, blocks))
    assert ab <= 2e-2 and rl <= 1e-3, (ab, rl)
    tiny = torch.empty(16, dtype=torch.uint8, device=dev)
    if ops.q8_0_workspace_bytes(m, k, n) > 16:
        assert np.array_equal(to_host(ops.q8_0_matmul(xd, bd, "w8a16", workspace=tiny)),
                              to_host(ops.q8_0_matmul(xd, bd, "w8a16")))


def _repack_host(blocks, k):
    """The packed layout restated on the host: per row, weights 8g .. 8g+7 of block b at
    g * nb * 8 + b * 8, then the nb f16 scales."""
    n, nb = blocks.shape[0], k // 32
    b = blocks.reshape(n, nb, 34)
    qs = b[:, :, 2:].reshape(n, nb, 4, 8).transpose(0, 2, 1, 3).reshape(n, k)
    return np.concatenate([qs, b[:, :, :2].reshape(n, 2 * nb)], axis=1).reshape(-1)


@pytest.mark.parametrize("m,k,n", Q8_SHAPES + [(33, 512, 128)])
def test_q8_0_packed_layout(dev, m, k, n):
    """dtts_q8_0_repack writes the documented layout byte for byte; dtts_gemm_q8_0_packed on it meets
    the oracle bars of the other Q8_0 paths and, where dtts_gemm_q8_0_ws runs the same A-sharing
    kernel on the GGML blocks (m > 16), equals it bit for bit."""
    w = synth.normal(85, "w", (n, k), 0, 0.02)
    blocks = ops.q8_0_quantize(w)
    bd = torch.from_numpy(blocks).to(dev)
    packed = ops.q8_0_repack(bd, k)
    assert np.array_equal(to_host(packed), _repack_host(blocks, k))
    xb = synth.f16_bits(synth.normal(85, "x", (m, k)))
    x, xd = synth.from_f16_bits(xb), to_dev(xb, dev)
    got8 = to_host(ops.q8_0_matmul_packed(xd, packed, n, "w8a8"))
    assert rel(got8, oracle.q8_0_matmul_w8a8(x, blocks))[1] <= 1e-5
    got16 = to_host(ops.q8_0_matmul_packed(xd, packed, n, "w8a16"))
    ab, rl = rel(got16, oracle.q8_0_matmul_f64(x, blocks))
    assert ab <= 2e-2 and rl <= 1e-3, (ab, rl)
    if m > 16:
        for mode, got in (("w8a8", got8), ("w8a16", got16)):
            assert np.array_equal(got, to_host(ops.q8_0_matmul(xd, bd, mode, workspace="auto"))), mode


# ---------------------------------------------------------------- Q8_0 on f32 activations
# Proj::forward hands QMatMul::forward the f32 hidden state (crates/tts-nn/src/lib.rs:509-531).
# Bars: W8A8 max-rel <= 1e-5 against the oracle's vec_dot restatement on the same f32 values
# (no f16 rounding first); W8A32 max-rel <= 1e-5 against float64 on the dequantized weights.

def _q8_f32_paths(xd, bd, packed, n, mode):
    return {
        "plain": ops.q8_0_matmul(xd, bd, mode),
        "ws": ops.q8_0_matmul(xd, bd, mode, workspace="auto"),
        "packed": ops.q8_0_matmul_packed(xd, packed, n, mode),
    }


@pytest.mark.parametrize("m,k,n", Q8_SHAPES + [(33, 512, 128), (64, 1024, 1024)])
def test_q8_0_f32_activations(dev, m, k, n):
    w = synth.normal(86, "w", (n, k), 0, 0.02)
    blocks = ops.q8_0_quantize(w)
    x = synth.normal(86, "x32", (m, k)).astype(np.float32)
    assert not np.array_equal(x, synth.from_f16_bits(synth.f16_bits(x)))  # not f16 values
    xd, bd = torch.from_numpy(x).to(dev), torch.from_numpy(blocks).to(dev)
    packed = ops.q8_0_repack(bd, k)
    want8 = oracle.q8_0_matmul_w8a8(x, blocks)
    want32 = oracle.q8_0_matmul_f64(x, blocks)
    got8 = {p: to_host(y) for p, y in _q8_f32_paths(xd, bd, packed, n, "w8a8").items()}
    got32 = {p: to_host(y) for p, y in _q8_f32_paths(xd, bd, packed, n, "w8a32").items()}
    for p in got8:
        assert rel(got8[p], want8)[1] <= 1e-5, (p, rel(got8[p], want8))
        assert rel(got32[p], want32)[1] <= 1e-5, (p, rel(got32[p], want32))
    if m > 16:  # the A-sharing kernel behind both: the same sums bit for bit
        assert np.array_equal(got8["ws"], got8["packed"]) and np.array_equal(got32["ws"], got32["packed"])


def test_q8_0_f32_w8a8_near_ties(dev):
    """f32 activations just below an x.5 tie that f16 rounding lands on (test_oracle_gemm_q8's
    block): every path quantizes the f32 values, matching the oracle, and lands far from the
    f16-first route."""
    from test_oracle_gemm_q8 import near_tie_activations

    m, k, n = 48, 1024, 1024
    x = near_tie_activations(m, k)
    w = synth.normal(87, "w", (n, k), 0, 0.02)
    blocks = ops.q8_0_quantize(w)
    xd, bd = torch.from_numpy(x).to(dev), torch.from_numpy(blocks).to(dev)
    want = oracle.q8_0_matmul_w8a8(x, blocks)
    via_f16 = oracle.q8_0_matmul_w8a8(synth.from_f16_bits(synth.f16_bits(x)), blocks)
    assert rel(via_f16, want)[1] > 1e-3
    for p, y in _q8_f32_paths(xd, bd, ops.q8_0_repack(bd, k), n, "w8a8").items():
        got = to_host(y)
        assert rel(got, want)[1] <= 1e-5, p
        assert rel(got, via_f16)[1] > 1e-3, p


def test_q8_0_w8a32_dynamic_range(dev):
    """W8A32 scales each activation block by a power of two before its f16 hi + lo split: rows far
    outside f16's range (1e6, 1e30) or deep in its subnormals (1e-6, 1e-30), a row whose blocks
    differ by 1e12, and a zero row all meet 1e-5 of their own row's magnitude."""
    m, k, n = 48, 1024, 1024
    x = synth.normal(88, "x32", (m, k)).astype(np.float32)
    scales = np.ones(m, np.float32)
    scales[1:6] = [1e6, 1e30, 1e-6, 1e-30, 6e4]
    x *= scales[:, None]
    x[6, 512:] *= np.float32(1e12)
    x[7] = 0.0
    w = synth.normal(88, "w", (n, k), 0, 0.02)
    blocks = ops.q8_0_quantize(w)
    xd, bd = torch.from_numpy(x).to(dev), torch.from_numpy(blocks).to(dev)
    want = oracle.q8_0_matmul_f64(x, blocks)
    for p, y in _q8_f32_paths(xd, bd, ops.q8_0_repack(bd, k), n, "w8a32").items():
        got = to_host(y)
        assert np.all(got[7] == 0.0), p
        for r in range(m):
            if r == 7:
                continue
            err = np.max(np.abs(got[r].astype(np.float64) - want[r])) / np.max(np.abs(want[r]))
            assert err <= 1e-5, (p, r, err)


def test_q8_0_mode_and_dtype_refusals(dev):
    """W8A16 names an f16 operand (refused for f32 x); W8A32 is an f32 mode (refused for f16 x)."""
    k, n = 256, 64
    bd = torch.from_numpy(ops.q8_0_quantize(synth.normal(89, "w", (n, k), 0, 0.02))).to(dev)
    x32 = torch.ones((8, k), dtype=torch.float32, device=dev)
    x16 = x32.half()
    for xx, mode in ((x32, "w8a16"), (x16, "w8a32")):
        for ws in (None, "auto"):
            with pytest.raises(ops.DttsError, match="not taken with"):
                ops.q8_0_matmul(xx, bd, mode, workspace=ws)
        with pytest.raises(ops.DttsError, match="not taken with"):
            ops.q8_0_matmul_packed(xx, ops.q8_0_repack(bd, k), n, mode)


# ---------------------------------------------------------------- f32 projections (Proj::Dense)

@pytest.mark.parametrize("m,k,n", [(48, 1024, 4096), (48, 1024, 3072), (48, 3072, 1024), (1, 2048, 6144),
                                   (8, 256, 64), (64, 512, 128), (33, 96, 192)])
def test_gemm_f32_nt(dev, m, k, n):
    """dtts_gemm_f32_nt against float64 on the same f32 operands: max-rel <= 1e-5 (f32 products
    and sums on the matrix cores, in another order), and split and single-range runs agree."""
    x = synth.normal(100, "x32", (m, k)).astype(np.float32)
    w = synth.normal(100, "w32", (n, k), 0, 0.02).astype(np.float32)
    got = to_host(ops.gemm_f32_nt(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev)))
    want = x.astype(np.float64) @ w.astype(np.float64).T
    ab, rl = rel(got, want)
    assert rl <= 1e-5, (ab, rl)


def test_gemm_f32_nt_refusals(dev):
    x = torch.zeros((8, 100), device=dev)
    with pytest.raises(ops.DttsError, match="multiple of 32"):
        ops.gemm_f32_nt(x, torch.zeros((64, 100), device=dev))
    x = torch.zeros((65, 128), device=dev)
    with pytest.raises(ops.DttsError, match="m <= 64"):
        ops.gemm_f32_nt(x, torch.zeros((64, 128), device=dev))


# ---------------------------------------------------------------- one-launch kernels at their edges
# gemm_row_nt (k * ceil(m/16) <= 3072: two or three 64-k chunks per wave, up to 16 waves) and
# gemm_q8_row (4, 6, 8 or 12 blocks per wave, up to 8 waves): every row-block count, the chunk
# choices and the last k each takes, against the same oracle bars as the split kernels.

@pytest.mark.parametrize("m,k,n,gateup", [
    (1, 128, 64, False), (16, 2048, 256, False), (16, 3072, 128, False), (17, 1536, 512, False),
    (33, 1024, 192, False), (48, 1024, 96, True), (64, 768, 128, False), (64, 256, 64, True), (5, 2880, 80, False),
])
def test_one_launch_projection_edges(dev, m, k, n, gateup):
    assert ops.gemm_workspace_bytes(m, k, n, gateup) == 0  # the one-launch kernel takes these
    a, w = _ab(90, m, k, 2 * n if gateup else n)
    ad, wd = to_dev(a, dev), to_dev(w, dev)
    gu = oracle.gemm_f16_f32acc(a, np.ascontiguousarray(w.T))
    if gateup:
        got, want = to_host(ops.gateup_silu(ad, wd)), oracle.swiglu_mul_f32(gu[:, :n].copy(), gu[:, n:].copy())
    else:
        got, want = to_host(ops.matmul_nt(ad, wd)), gu
    ab, rl = rel(got, want)
    assert ab <= 2e-2 and rl <= 1e-4, (ab, rl)


@pytest.mark.parametrize("m,k,n", [(1, 256, 64), (16, 768, 128), (1, 1536, 64), (1, 2048, 128), (16, 3072, 64),
                                   (9, 2304, 64)])
def test_q8_0_one_launch_edges(dev, m, k, n):
    """W8A16 on GGML blocks and the packed layout, W8A32 on the packed layout, at the one-launch
    kernel's block-per-wave choices (4, 6, 8, 12); where both layouts take it (4 blocks per wave:
    k <= 1024 at these m) the packed and GGML W8A16 results agree bit for bit."""
    w = synth.normal(91, "w", (n, k), 0, 0.02)
    blocks = ops.q8_0_quantize(w)
    bd = torch.from_numpy(blocks).to(dev)
    packed = ops.q8_0_repack(bd, k) if k % 256 == 0 else None
    xb = synth.f16_bits(synth.normal(91, "x", (m, k)))
    x16 = synth.from_f16_bits(xb)
    want16 = oracle.q8_0_matmul_f64(x16, blocks)
    g16 = to_host(ops.q8_0_matmul(to_dev(xb, dev), bd, "w8a16"))
    ab, rl = rel(g16, want16)
    assert ab <= 2e-2 and rl <= 1e-3, (ab, rl)
    if packed is not None:
        p16 = to_host(ops.q8_0_matmul_packed(to_dev(xb, dev), packed, n, "w8a16"))
        ab, rl = rel(p16, want16)
        assert ab <= 2e-2 and rl <= 1e-3, (ab, rl)
        if k <= 1024:
            assert np.array_equal(p16, g16)
        x32 = synth.normal(91, "x32", (m, k)).astype(np.float32)
        g32 = to_host(ops.q8_0_matmul_packed(torch.from_numpy(x32).to(dev), packed, n, "w8a32"))
        assert rel(g32, oracle.q8_0_matmul_f64(x32, blocks))[1] <= 1e-5


# The one-launch kernels are instantiated for some (row blocks, chunks per wave) pairs only: three
# 64-k chunks per wave (k a multiple of 192, not of 128) for one 16-row block; 6 Q8_0 blocks per
# wave up to two row blocks, 8 and 12 for one. Shapes outside those pairs take the k-split kernels,
# and every row of the result is computed (a shape routed to a kernel of fewer row blocks or
# blocks per wave would leave rows or k unreduced).

@pytest.mark.parametrize("m,k,n,gateup", [(48, 576, 128, False), (33, 192, 64, True), (20, 1344, 64, False),
                                          (17, 960, 32, False), (64, 576, 64, True)])
def test_projection_shapes_off_the_one_launch_instances(dev, m, k, n, gateup):
    a, w = _ab(92, m, k, 2 * n if gateup else n)
    ad, wd = to_dev(a, dev), to_dev(w, dev)
    gu = oracle.gemm_f16_f32acc(a, np.ascontiguousarray(w.T))
    if gateup:
        got, want = to_host(ops.gateup_silu(ad, wd)), oracle.swiglu_mul_f32(gu[:, :n].copy(), gu[:, n:].copy())
    else:
        got, want = to_host(ops.matmul_nt(ad, wd)), gu
    ab, rl = rel(got, want)
    assert ab <= 2e-2 and rl <= 1e-4, (ab, rl)


@pytest.mark.parametrize("m,k,n", [(24, 1280, 64), (32, 1280, 128), (40, 768, 64)])
def test_q8_0_shapes_off_the_one_launch_instances(dev, m, k, n):
    """k = 1280 takes 8 blocks per wave, instantiated for one row block only: at 17-32 rows the
    packed W8A16 product goes to the A-sharing kernel; the GGML and packed results agree with
    float64 on the dequantized weights."""
    w = synth.normal(93, "w", (n, k), 0, 0.02)
    blocks = ops.q8_0_quantize(w)
    bd = torch.from_numpy(blocks).to(dev)
    packed = ops.q8_0_repack(bd, k)
    xb = synth.f16_bits(synth.normal(93, "x", (m, k)))
    want = oracle.q8_0_matmul_f64(synth.from_f16_bits(xb), blocks)
    for got in (to_host(ops.q8_0_matmul(to_dev(xb, dev), bd, "w8a16")),
                to_host(ops.q8_0_matmul_packed(to_dev(xb, dev), packed, n, "w8a16"))):
        ab, rl = rel(got, want)
        assert ab <= 2e-2 and rl <= 1e-3, (ab, rl)
