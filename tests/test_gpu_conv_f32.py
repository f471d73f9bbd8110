"""The channel-major f32 conv and the im2col gather (a6/a7), and config 1 end to end.

Bars (the reference's, crates/tts-nn/src/lib.rs:1330-1366, nlc.rs:264-405): max-rel <= 1e-5
against the oracle's im2col + GEMM + bias route and against torch's float64 conv1d; the gather
bit-exact. Config 1: one residual unit [1, 512, 4800] f32, snake(alpha1) -> conv k7 d3 pad 9
-> snake(alpha2) -> conv k1 -> + x, Kaiming-normal weights, biases N(0, 0.01), from seed 0.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from dtts import nlc, synth

from _util import rel, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cin,length,k,dil,pad", [(3, 11, 3, 1, 2), (8, 17, 7, 3, 18), (6, 9, 1, 1, 0),
                                                  (4, 15, 3, 1, 1), (8, 64, 7, 3, 9), (2, 65, 11, 5, 25),
                                                  (128, 444, 3, 1, 1)])
def test_im2col_bit_exact(dev, cin, length, k, dil, pad):
    # im2col.rs:177-239 shapes, causal and centred
    x = synth.normal(90, f"x{cin}", (cin, length))
    got = to_host(nlc.im2col_tap_major(to_dev(x, dev), k, dil, pad))
    assert np.array_equal(got, oracle.im2col_tap_major_f32(x, k, dil, pad))


@pytest.mark.parametrize("cout,cin,length,k,dil", [(8, 4, 15, 3, 1), (8, 8, 64, 7, 3), (4, 4, 65, 11, 5),
                                                   (128, 128, 444, 3, 1), (64, 32, 1000, 7, 9),
                                                   (512, 512, 300, 7, 3), (128, 64, 257, 1, 1)])
def test_centered_conv_matches_oracle_and_torch(dev, cout, cin, length, k, dil):
    # lib.rs:1330-1366 shapes plus the tiled kernel's
    pad = (k - 1) * dil // 2
    x = synth.normal(91, "x", (2, cin, length))
    w = synth.normal(91, "w", (cout, cin, k), 0, 0.1)
    b = synth.normal(91, "b", (cout,))
    w_tm = oracle.tap_major_weight_f32(w)
    got = to_host(nlc.conv1d_ncl_f32(to_dev(x, dev), to_dev(nlc.tap_major_weight(w), dev), to_dev(b, dev), k=k, dilation=dil,
                                     pad_left=pad))
    assert rel(got, oracle.conv1d_ncl_gemm_f32(x, w_tm, b, k, dil, pad))[1] < 1e-5
    want = F.conv1d(torch.from_numpy(x).double(), torch.from_numpy(w).double(), torch.from_numpy(b).double(),
                    padding=pad, dilation=dil).numpy()
    assert rel(got, want)[1] < 1e-5


def test_causal_conv_with_snake_and_residual(dev):
    cin = cout = 64
    length, k, dil = 700, 7, 9
    x = synth.normal(92, "x", (1, cin, length))
    res = synth.normal(92, "res", (1, cout, length))
    w = synth.normal(92, "w", (cout, cin, k), 0, 0.1)
    b = synth.normal(92, "b", (cout,), 0, 0.1)
    a1, r1 = synth.uniform(92, "a1", (cin,), 0.5, 1.5), synth.uniform(92, "r1", (cin,), 0.5, 1.5)
    a2, r2 = synth.uniform(92, "a2", (cout,), 0.5, 1.5), synth.uniform(92, "r2", (cout,), 0.5, 1.5)
    w_tm = oracle.tap_major_weight_f32(w)
    y_pre, y = nlc.conv1d_ncl_f32(to_dev(x, dev), to_dev(nlc.tap_major_weight(w), dev), to_dev(b, dev), k=k, dilation=dil,
                                  snake_in=(to_dev(a1, dev), to_dev(r1, dev)), residual=to_dev(res, dev),
                                  snake_out=(to_dev(a2, dev), to_dev(r2, dev)), want_pre=True)
    s = oracle.snake_ncl_f32(x, a1, r1)
    want_pre = oracle.conv1d_ncl_gemm_f32(s, w_tm, b, k, dil, (k - 1) * dil) + res
    assert rel(to_host(y_pre), want_pre)[1] < 1e-5
    assert rel(to_host(y), oracle.snake_ncl_f32(want_pre, a2, r2))[1] < 1e-5


def config1():
    c, length = 512, 4800
    x = synth.normal(0, "cfg1.x", (1, c, length))
    a1 = synth.uniform(0, "cfg1.alpha1", (c,), 0.5, 1.5)
    a2 = synth.uniform(0, "cfg1.alpha2", (c,), 0.5, 1.5)
    w1 = synth.kaiming_normal(0, "cfg1.w1", (c, c, 7), c * 7)
    b1 = synth.normal(0, "cfg1.b1", (c,), 0, 0.01)
    w2 = synth.kaiming_normal(0, "cfg1.w2", (c, c, 1), c)
    b2 = synth.normal(0, "cfg1.b2", (c,), 0, 0.01)
    return x, a1, a2, w1, b1, w2, b2


def test_config1_residual_unit(dev):
    x, a1, a2, w1, b1, w2, b2 = config1()
    r1, r2 = (1.0 / a1).astype(np.float32), (1.0 / a2).astype(np.float32)
    w1t, w2t = oracle.tap_major_weight_f32(w1), oracle.tap_major_weight_f32(w2)
    xd = to_dev(x, dev)
    h = nlc.conv1d_ncl_f32(xd, to_dev(nlc.tap_major_weight(w1), dev), to_dev(b1, dev), k=7, dilation=3, pad_left=9,
                           snake_in=(to_dev(a1, dev), to_dev(r1, dev)),
                           snake_out=(to_dev(a2, dev), to_dev(r2, dev)))
    y = to_host(nlc.conv1d_ncl_f32(h, to_dev(nlc.tap_major_weight(w2), dev), to_dev(b2, dev), k=1, residual=xd))
    s1 = oracle.snake_ncl_f32(x, a1, r1)
    h_ref = oracle.conv1d_ncl_gemm_f32(s1, w1t, b1, 7, 3, 9)
    s2 = oracle.snake_ncl_f32(h_ref, a2, r2)
    want = oracle.conv1d_ncl_gemm_f32(s2, w2t, b2, 1, 1, 0) + x
    assert rel(y, want)[1] < 1e-5
