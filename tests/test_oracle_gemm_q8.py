"""Pins the oracle's f16 GEMM, SwiGLU and Q8_0 restatements (float64, closed forms, exact cases),
and checks the library's host Q8_0 quantizer against the oracle bit for bit."""
import numpy as np
import pytest

import oracle
from dtts import ops, synth


def test_gemm_f16_oracle_matches_f64():
    a = synth.f16_bits(synth.normal(70, "a", (48, 1024)))
    b = synth.f16_bits(synth.normal(70, "b", (1024, 256), 0, 0.02))
    got = oracle.gemm_f16_f32acc(a, b)
    want = synth.from_f16_bits(a).astype(np.float64) @ synth.from_f16_bits(b).astype(np.float64)
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-5
    assert np.max(np.abs(oracle.gemm_f16_f64(a, b) - want)) < 1e-10


def test_swiglu_oracle_matches_f64_sweep():
    # crates/tts-nn/src/fused.rs:2310-2322: g over +-30, u over +-4, error / max(|g u|, 1) < 2e-6
    n = 8 * 4096
    gs = (-30.0 + 60.0 * (np.arange(n) % 4096) / 4095).astype(np.float32)
    us = (-4.0 + 8.0 * (np.arange(n) % 4096) / 4095).astype(np.float32)
    got = oracle.swiglu_mul_f32(gs, us)
    g64, u64 = gs.astype(np.float64), us.astype(np.float64)
    want = g64 / (1.0 + np.exp(-g64)) * u64
    assert np.max(np.abs(got - want) / np.maximum(np.abs(g64 * u64), 1.0)) < 2e-6


def _edge_weights():
    w = synth.normal(71, "w", (6, 128), 0, 0.02)
    w[1, :32] = 0.0                       # an all-zero block: d = 0, id = 0
    w[2, :32] = np.linspace(-1, 1, 32)    # amax exactly at both ends
    w[3, 32:64] = 0.5                     # constant block: every q = 127
    w[4, :32] = np.arange(32) - 15.5      # halves land on x.5 boundaries
    return w.astype(np.float32)


def test_q8_0_oracle_closed_form_and_library_quantizer_agree():
    w = _edge_weights()
    blocks = oracle.q8_0_quantize(w)
    assert blocks.shape == (6, 4, 34)
    d = synth.from_f16_bits(blocks[..., :2].copy().view(np.uint16)[..., 0])
    q = blocks[..., 2:].view(np.int8).astype(np.int32)
    amax = np.abs(w.reshape(6, 4, 32)).max(-1)
    assert np.array_equal(synth.f16_bits(amax / 127.0), blocks[..., :2].copy().view(np.uint16)[..., 0])
    assert np.all(np.abs(q) <= 127)
    assert np.all(q[1, 0] == 0) and d[1, 0] == 0.0
    assert np.all(q[3, 1] == 127)
    deq = oracle.q8_0_dequantize(blocks, 128)
    assert np.array_equal(deq, (q * d[..., None]).reshape(6, 128).astype(np.float32))
    assert np.all(np.abs(deq - w) <= np.repeat(d, 32, -1) * 0.5 + 1e-3 * np.abs(w) + 1e-9)
    # the library's host quantizer writes the same bytes
    assert np.array_equal(ops.q8_0_quantize(w), blocks)


# A block whose amax is exactly 127 has d = 127/127 = 1 and id = 1, so x * id is x itself and
# every x.5 below is an exact tie. ggml's quantize_row_q8_0 (roundf) and candle's
# BlockQ8_0::from_float (f32::round) round ties away from zero; round-half-even would give
# 2, -2, 0, 0, 4, -6, 126, -126 for the first eight, so this pins the rule.
TIE_VALUES = np.array([2.5, -2.5, 0.5, -0.5, 4.5, -6.5, 126.5, -126.5, 1.5, -1.5, 3.5, 127.0], np.float32)
TIE_CODES = np.array([3, -3, 1, -1, 5, -7, 127, -127, 2, -2, 4, 127], np.int32)


def tie_block_weights():
    w = np.zeros((2, 64), np.float32)
    w[0, :12] = TIE_VALUES
    w[1, 32:44] = TIE_VALUES * 0.5  # amax 63.5: d = 0.5 exactly in f16, id = 2, the same ties
    return w


def test_q8_0_ties_round_half_away_from_zero():
    # the block discriminates: round-half-even (numpy's rint) disagrees on 8 of the 12 codes
    assert int(np.sum(np.rint(TIE_VALUES).astype(np.int32) != TIE_CODES)) == 8
    w = tie_block_weights()
    blocks = oracle.q8_0_quantize(w)
    d = synth.from_f16_bits(blocks[..., :2].copy().view(np.uint16)[..., 0])
    q = blocks[..., 2:].view(np.int8).astype(np.int32)
    assert d[0, 0] == 1.0 and d[1, 1] == 0.5
    assert np.array_equal(q[0, 0, :12], TIE_CODES) and np.all(q[0, 0, 12:] == 0)
    assert np.array_equal(q[1, 1, :12], TIE_CODES) and np.all(q[1, 1, 12:] == 0)
    assert np.array_equal(ops.q8_0_quantize(w), blocks)  # the library's host quantizer


def test_q8_0_w8a8_is_exact_on_prequantized_activations():
    # activations that are already Q8_0 values quantize to themselves, so the w8a8 result is the
    # exact block dot up to the f32 scale products
    k, n, m = 256, 32, 3
    w = synth.normal(72, "w", (n, k), 0, 0.02)
    blocks = oracle.q8_0_quantize(w)
    qx = synth.randint(72, "qx", (m, k), -127, 127).astype(np.float32)
    qx[:, ::32] = 127.0  # each block's amax is 127 * dx
    dx = np.float32(0.03125)  # a power of two: d = amax/127 = dx exactly, 1/d exact
    x = qx * dx
    got = oracle.q8_0_matmul_w8a8(x, blocks)
    want = oracle.q8_0_matmul_f64(x, blocks)
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-6


def test_q8_0_w8a8_close_to_unquantized_activations():
    w = synth.normal(73, "w", (64, 1024), 0, 0.02)
    blocks = oracle.q8_0_quantize(w)
    x = synth.from_f16_bits(synth.f16_bits(synth.normal(73, "x", (8, 1024))))
    got = oracle.q8_0_matmul_w8a8(x, blocks)
    want = oracle.q8_0_matmul_f64(x, blocks)
    assert oracle.abs_and_rel(got, want)[1] < 2e-2  # activation quantization noise, ~1/254 per term


# f32 activations just below an x.5 tie that f16 rounding lands on: in a block whose amax is 127
# (d = 1, id = 1) each f32 value quantizes toward zero and its f16 image (2.5, 4.5, -6.5, ...)
# away from zero. Proj::forward hands QMatMul::forward the f32 hidden state
# (crates/tts-nn/src/lib.rs:509-531), so a route that rounds x to f16 first gets other codes.
NEAR_TIE = np.array([127.0, 2.4999, 4.4999, -6.4999, 0.49999, 10.4999, -1.4999, 126.4999], np.float32)
NEAR_TIE_CODES_F32 = np.array([127, 2, 4, -6, 0, 10, -1, 126], np.int32)
NEAR_TIE_CODES_F16 = np.array([127, 3, 5, -7, 1, 11, -2, 127], np.int32)


def near_tie_activations(m, k, seed=74):
    """[m, k] f32 ~ N(0, 1) whose first block in every row opens with NEAR_TIE (amax 127)."""
    x = synth.normal(seed, "x.neartie", (m, k)).astype(np.float32)
    x[:, :8] = NEAR_TIE
    return x


def test_q8_0_w8a8_quantizes_f32_activations_without_f16_rounding():
    x = near_tie_activations(4, 64)
    x16 = synth.from_f16_bits(synth.f16_bits(x))
    codes = oracle.q8_0_quantize(x)[:, 0, 2:10].view(np.int8).astype(np.int32)
    codes16 = oracle.q8_0_quantize(x16)[:, 0, 2:10].view(np.int8).astype(np.int32)
    assert np.array_equal(codes, np.tile(NEAR_TIE_CODES_F32, (4, 1)))
    assert np.array_equal(codes16, np.tile(NEAR_TIE_CODES_F16, (4, 1)))
    # the W8A8 product on the f32 values is the one the oracle's vec_dot restatement gives, and
    # the f16-first route misses it by far more than the 1e-5 parity bar
    w = synth.normal(74, "w.neartie", (64, 64), 0, 0.02)
    blocks = oracle.q8_0_quantize(w)
    y = oracle.q8_0_matmul_w8a8(x, blocks)
    y16 = oracle.q8_0_matmul_w8a8(x16, blocks)
    assert oracle.abs_and_rel(y16, y)[1] > 1e-3
    # and it is the exact block arithmetic: integer dots of those codes times the f16 scales
    xq = oracle.q8_0_quantize(x)
    qx = xq[..., 2:].view(np.int8).astype(np.int64)
    dx = synth.from_f16_bits(xq[..., :2].copy().view(np.uint16)[..., 0]).astype(np.float64)
    qw = blocks[..., 2:].view(np.int8).astype(np.int64)
    dw = synth.from_f16_bits(blocks[..., :2].copy().view(np.uint16)[..., 0]).astype(np.float64)
    want = np.einsum("mbj,nbj->mnb", qx, qw).astype(np.float64) * dx[:, None, :] * dw[None, :, :]
    assert np.max(np.abs(y - want.sum(-1))) <= 1e-5 * np.max(np.abs(want.sum(-1)))
