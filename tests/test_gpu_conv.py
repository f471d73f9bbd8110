"""Channels-last conv (a3-a5) through the C ABI against the CPU oracle's f16-storage conv.

Both sides hold activations, weights and bias in f16, snake outputs rounded to f16, f32
accumulation and one rounding of the output; they differ only in summation order. Bar: max-abs
<= 2e-2 at unit-scale activations (the f16 GEMM tolerance), and at most a few f16 ulps. The
transposed conv is also held to the f64 scatter definition of ConvTranspose1d.
"""
import numpy as np
import pytest
import torch

import oracle
from dtts import nlc, synth

from _util import f16_ulp_diff, rel, to_dev, to_host  # noqa: F401

pytestmark = pytest.mark.gpu


def _case(seed, lanes, length, cin, cout, k, wscale=None):
    x = synth.f16_bits(synth.normal(seed, "x", (lanes, length, cin)))
    std = wscale if wscale is not None else np.sqrt(2.0 / (cin * k))  # Kaiming normal
    w = synth.normal(seed, "w", (cout, cin, k), 0, std)
    wb = synth.f16_bits(w)
    b = synth.f16_bits(synth.normal(seed, "b", (cout,), 0, 0.01))
    return x, w, wb, b


def _elementwise(got_bits, want_bits):
    """Per element: one f16 ulp of the value plus the f32 summation-order error (~1e-4 here)."""
    g = synth.from_f16_bits(got_bits).astype(np.float64)
    w = synth.from_f16_bits(want_bits).astype(np.float64)
    bad = np.abs(g - w) > np.abs(w) * 2.0 ** -10 + 1e-4
    assert not bad.any(), f"{int(bad.sum())} elements off, worst {np.max(np.abs(g - w)):.3e}"


def _close(got_bits, want_bits, tol=2e-2):
    g = synth.from_f16_bits(got_bits)
    w = synth.from_f16_bits(want_bits)
    err = float(np.max(np.abs(g - w))) if g.size else 0.0
    assert err <= tol, f"max abs {err:.3e}"
    return err


@pytest.mark.parametrize("lanes,cin,cout,length,k,dil", [
    (2, 8, 12, 40, 7, 1), (1, 16, 16, 33, 7, 3), (2, 6, 9, 20, 1, 1),            # nlc.rs:294-328 (direct)
    (1, 96, 96, 4200, 7, 9), (2, 32, 96, 4096, 7, 1), (1, 128, 192, 5000, 7, 3),  # nlc.rs:362-398
    (2, 64, 96, 4097, 1, 1),
    (3, 96, 96, 700, 7, 9), (2, 192, 192, 513, 7, 3), (2, 384, 384, 300, 7, 1),   # codec RU shapes
    (2, 768, 768, 250, 1, 1), (2, 1024, 1536, 250, 7, 1),                         # RU k1, head conv
    (2, 64, 64, 100, 7, 2), (2, 32, 32, 65, 3, 4),                                 # BN 64 / 32 tiles
    (2, 96, 384, 300, 1, 1), (1, 160, 192, 257, 1, 1),                             # cin off the 64-chunk tile
    (1, 384, 192, 1500, 2, 1), (2, 96, 192, 300, 7, 3),                            # k=2 and k=7 at 192 columns
])
def test_causal_conv_matches_oracle(dev, lanes, cin, cout, length, k, dil):
    x, w, wb, b = _case(40, lanes, length, cin, cout, k)
    w_tm = nlc.tap_major_weight(wb)
    got = to_host(nlc.causal_conv1d(to_dev(x, dev), to_dev(w_tm, dev), to_dev(b, dev), dil))
    want = oracle.conv1d_nlc_f16(x, oracle.tap_weight_f32(synth.from_f16_bits(wb)).astype(np.float32)
                                 .astype(np.float16).view(np.uint16), b, dil)
    _close(got, want)
    _elementwise(got, want)


@pytest.mark.parametrize("lanes,c,length,k,dil,pre", [
    (2, 96, 3000, 1, 1, False), (2, 192, 1100, 7, 3, True), (1, 96, 2049, 7, 9, True),
    (2, 384, 300, 7, 1, False),
])
def test_fused_prologue_epilogue(dev, lanes, c, length, k, dil, pre):
    """snake on load + residual (snake_conv_residual), plus the epilogue snake and y_pre."""
    x, w, wb, b = _case(41, lanes, length, c, c, k)
    res = synth.f16_bits(synth.normal(41, "res", (lanes, length, c)))
    a1 = synth.uniform(41, "a1", (c,), 0.5, 1.5)
    r1 = (1.0 / a1).astype(np.float32)
    a2 = synth.uniform(41, "a2", (c,), 0.5, 1.5)
    r2 = (1.0 / a2).astype(np.float32)
    w_tm = nlc.tap_major_weight(wb)
    w_tap = oracle.tap_weight_f32(synth.from_f16_bits(wb)).astype(np.float16).view(np.uint16)
    y_pre, y = nlc.conv1d(to_dev(x, dev), to_dev(w_tm, dev), to_dev(b, dev), k=k, dilation=dil,
                          snake_in=(to_dev(a1, dev), to_dev(r1, dev)), residual=to_dev(res, dev),
                          snake_out=(to_dev(a2, dev), to_dev(r2, dev)), want_pre=True)
    want_pre = oracle.conv1d_nlc_f16(x, w_tap, b, dil, snake=(a1, r1), res_bits=res)
    _close(to_host(y_pre), want_pre)
    # the epilogue snake applied to the kernel's own rounded sum is exactly the oracle's snake
    got_y = to_host(y)
    assert f16_ulp_diff(got_y, oracle.snake_nlc_f16(to_host(y_pre), a2, r2)) <= 1
    _close(got_y, oracle.snake_nlc_f16(want_pre, a2, r2), tol=3e-2)


@pytest.mark.parametrize("cin,cout,length,stride", [(1536, 768, 20, 8), (768, 384, 40, 5),
                                                    (384, 192, 64, 4), (192, 96, 128, 3),
                                                    (32, 32, 9, 2)])
def test_transposed_conv_matches_definition(dev, cin, cout, length, stride):
    lanes, k = 2, 2 * stride
    x = synth.f16_bits(synth.normal(42, "x", (lanes, length, cin)))
    w = synth.normal(42, "w", (cin, cout, k), 0, np.sqrt(2.0 / (cout * k)))
    wb = synth.f16_bits(w)
    b = synth.f16_bits(synth.normal(42, "b", (cout,), 0, 0.01))
    w_tm = nlc.transpose_tap_major_weight(wb, stride)
    b_rep = nlc.transpose_bias(b, stride)
    got = to_host(nlc.causal_conv_transpose1d(to_dev(x, dev), to_dev(w_tm, dev), to_dev(b_rep, dev), stride))
    assert got.shape == (lanes, length * stride, cout)
    for li in range(lanes):
        want = oracle.conv_transpose1d_causal_f64(synth.from_f16_bits(x[li]), synth.from_f16_bits(wb),
                                                  synth.from_f16_bits(b), stride)
        err = np.abs(synth.from_f16_bits(got[li]) - want)
        assert np.max(err) <= 2e-2
        assert np.all(err <= np.abs(want) * 2.0 ** -10 + 1e-3)


@pytest.mark.parametrize("cin,k,dil,length", [(96, 7, 1, 1500), (64, 7, 3, 777), (128, 7, 9, 300), (32, 3, 1, 129),
                                               (40, 7, 1, 500)])
def test_tanh_output_conv_single_channel(dev, cin, k, dil, length):
    """The decoder's output conv, 96 -> 1, k=7, tanh, and the single-output-channel kernel's other
    channel counts, dilations and lengths (partial last tiles)."""
    x, w, wb, b = _case(43, 2, length, cin, 1, k)
    w_tm = nlc.tap_major_weight(wb)
    w_tap = oracle.tap_weight_f32(synth.from_f16_bits(wb)).astype(np.float16).view(np.uint16)
    y = to_host(nlc.conv1d(to_dev(x, dev), to_dev(w_tm, dev), to_dev(b, dev), k=k, dilation=dil, act="tanh"))
    want = oracle.conv1d_nlc_f16(x, w_tap, b, dil, act_tanh=True)
    _close(y, want, tol=2e-3)
    _elementwise(y, want)


@pytest.mark.parametrize("lanes,cin,length,k,dil", [(2, 96, 1000, 7, 1), (1, 40, 300, 5, 9), (3, 160, 257, 7, 3)])
def test_single_channel_conv_operands(dev, lanes, cin, length, k, dil):
    """The single-output-channel kernel with the prologue snake, residual, pre-snake store and output
    SnakeBeta, then with the clamp: channel counts with a partial last 32-channel chunk, halos to 54."""
    x, w, wb, b = _case(45, lanes, length, cin, 1, k)
    res = synth.f16_bits(synth.normal(45, "res", (lanes, length, 1)))
    a1 = synth.uniform(45, "a1", (cin,), 0.5, 1.5)
    r1 = (1.0 / a1).astype(np.float32)
    a2 = synth.uniform(45, "a2", (1,), 0.5, 1.5)
    r2 = (1.0 / a2).astype(np.float32)
    w_tm = nlc.tap_major_weight(wb)
    w_tap = oracle.tap_weight_f32(synth.from_f16_bits(wb)).astype(np.float16).view(np.uint16)
    y_pre, y = nlc.conv1d(to_dev(x, dev), to_dev(w_tm, dev), to_dev(b, dev), k=k, dilation=dil,
                          snake_in=(to_dev(a1, dev), to_dev(r1, dev)), residual=to_dev(res, dev),
                          snake_out=(to_dev(a2, dev), to_dev(r2, dev)), want_pre=True)
    want_pre = oracle.conv1d_nlc_f16(x, w_tap, b, dil, snake=(a1, r1), res_bits=res)
    _close(to_host(y_pre), want_pre)
    _elementwise(to_host(y_pre), want_pre)
    assert f16_ulp_diff(to_host(y), oracle.snake_nlc_f16(to_host(y_pre), a2, r2)) <= 1
    got = to_host(nlc.conv1d(to_dev(x, dev), to_dev(w_tm, dev), to_dev(b, dev), k=k, dilation=dil, act="clamp"))
    want = oracle.conv1d_nlc_f16(x, w_tap, b, dil, act="clamp")
    _close(got, want)
    _elementwise(got, want)


@pytest.mark.parametrize("lanes,cin,length,dil", [(2, 96, 1000, 1), (1, 64, 300, 9), (3, 160, 257, 3)])
def test_single_channel_k7_kernels_agree(dev, lanes, cin, length, dil):
    """The k = 7 single-output-channel kernel (32-channel multiples, no prologue SnakeBeta) with the
    residual, pre-snake store and output SnakeBeta against the oracle, and bit for bit against the
    generic kernel on the same operands (weights 8 bytes past a 16-byte boundary take that one)."""
    k = 7
    x, w, wb, b = _case(48, lanes, length, cin, 1, k)
    res = synth.f16_bits(synth.normal(48, "res", (lanes, length, 1)))
    a2 = synth.uniform(48, "a2", (1,), 0.5, 1.5)
    r2 = (1.0 / a2).astype(np.float32)
    w_tm = nlc.tap_major_weight(wb)
    w_tap = oracle.tap_weight_f32(synth.from_f16_bits(wb)).astype(np.float16).view(np.uint16)
    wd = to_dev(w_tm, dev)
    wbuf = torch.zeros(w_tm.size + 4, dtype=torch.float16, device=dev)
    wbuf[4:4 + w_tm.size] = wd.reshape(-1)
    w_off = wbuf[4:4 + w_tm.size].view(wd.shape)
    assert w_off.data_ptr() % 16 == 8
    outs = []
    for wt in (wd, w_off):
        outs.append([to_host(t) for t in nlc.conv1d(to_dev(x, dev), wt, to_dev(b, dev), k=k, dilation=dil,
                                                     residual=to_dev(res, dev), snake_out=(to_dev(a2, dev), to_dev(r2, dev)),
                                                     want_pre=True)])
    (pre_f, y_f), (pre_g, y_g) = outs
    assert np.array_equal(pre_f.view(np.uint16), pre_g.view(np.uint16))
    assert np.array_equal(y_f.view(np.uint16), y_g.view(np.uint16))
    want_pre = oracle.conv1d_nlc_f16(x, w_tap, b, dil, res_bits=res)
    _close(pre_f, want_pre)
    _elementwise(pre_f, want_pre)
    assert f16_ulp_diff(y_f, oracle.snake_nlc_f16(pre_f, a2, r2)) <= 1


def test_conv_rejects_bad_shapes(dev):
    from dtts import DttsError

    x = torch.zeros((1, 10, 32), dtype=torch.float16, device=dev)
    w = torch.zeros((32, 7 * 32), dtype=torch.float16, device=dev)
    with pytest.raises(DttsError, match="pad_left"):
        nlc.conv1d(x, w, None, k=7, dilation=1, pad_left=7)
    with pytest.raises(DttsError, match="shape"):
        nlc.conv1d(x, w[:, :100].contiguous(), None, k=7)


@pytest.mark.parametrize("lanes,c,length,dil,out_snake,k", [
    (2, 96, 3000, 9, True, 7), (3, 96, 700, 1, False, 7), (2, 192, 1100, 3, True, 7), (1, 192, 257, 9, False, 7),
    (2, 96, 900, 3, True, 7), (2, 192, 600, 1, False, 7), (2, 96, 500, 2, True, 7), (1, 192, 300, 5, False, 7),
    (2, 192, 800, 4, True, 3), (2, 96, 600, 2, False, 5), (1, 192, 300, 1, False, 1), (2, 96, 520, 1, True, 1)])
def test_fused_residual_unit_matches_composed_chain(dev, lanes, c, length, dil, out_snake, k):
    """dtts_residual_unit_nlc_f16 against the oracle's unfused chain with the same f16 storage
    points: h = conv_k(snake1(x)); h2 = snake2(h); y = conv1(h2) + x; [snake_out(y)]. The codec's
    k = 7 and dilations (1, 3, 9) at both widths, other dilations (2, 5) a caller may pass, and
    k = 1, 3, 5 (the kernel form with the tap count at run time)."""
    x = synth.f16_bits(synth.normal(44, "x", (lanes, length, c)))
    w1 = synth.f16_bits(synth.normal(44, "w1", (c, c, k), 0, np.sqrt(1.0 / (c * k))))
    w2 = synth.f16_bits(synth.normal(44, "w2", (c, c, 1), 0, np.sqrt(1.0 / c)))
    b1 = synth.f16_bits(synth.normal(44, "b1", (c,), 0, 0.01))
    b2 = synth.f16_bits(synth.normal(44, "b2", (c,), 0, 0.01))
    acts = [synth.uniform(44, f"a{i}", (c,), 0.5, 1.5) for i in range(3)]
    pairs = [(a, (1.0 / a).astype(np.float32)) for a in acts]
    dv = lambda p: (to_dev(p[0], dev), to_dev(p[1], dev))
    y_pre, y = nlc.residual_unit(to_dev(x, dev), dv(pairs[0]), to_dev(nlc.tap_major_weight(w1), dev), to_dev(b1, dev),
                                 dv(pairs[1]), to_dev(nlc.tap_major_weight(w2), dev), to_dev(b2, dev), k=k,
                                 dilation=dil, snake_out=dv(pairs[2]) if out_snake else None, want_pre=True)
    tap = lambda w: oracle.tap_weight_f32(synth.from_f16_bits(w)).astype(np.float16).view(np.uint16)
    h = oracle.conv1d_nlc_f16(x, tap(w1), b1, dil, snake=pairs[0])
    h2 = oracle.snake_nlc_f16(h, *pairs[1])
    want = oracle.conv1d_nlc_f16(h2, tap(w2), b2, 1, res_bits=x)
    got_pre = to_host(y_pre)
    _close(got_pre, want)
    g, w = synth.from_f16_bits(got_pre).astype(np.float64), synth.from_f16_bits(want).astype(np.float64)
    assert np.sqrt(np.mean((g - w) ** 2)) < 1e-3 * np.sqrt(np.mean(w ** 2))
    if out_snake:
        assert f16_ulp_diff(to_host(y), oracle.snake_nlc_f16(got_pre, *pairs[2])) <= 1
    else:
        assert np.array_equal(to_host(y), got_pre)


@pytest.mark.parametrize("act", ["tanh", "clamp", "gelu"])
@pytest.mark.parametrize("lanes,cin,cout,length,k,dil", [(2, 96, 96, 1100, 7, 3), (2, 64, 128, 300, 2, 1),
                                                        (2, 128, 128, 257, 1, 1)])
def test_general_epilogue_activation_and_scale(dev, act, lanes, cin, cout, length, k, dil):
    """The tile's general epilogue form (an activation and/or a per-channel scale; the plain form
    serves neither): each activation with and without the scale and the residual, at a k=7, a k=2
    and a k=1 tile, and a scale off 16-byte alignment, which the direct kernel takes instead."""
    x, w, wb, b = _case(46, lanes, length, cin, cout, k)
    w_tm = to_dev(nlc.tap_major_weight(wb), dev)
    w_tap = oracle.tap_weight_f32(synth.from_f16_bits(wb)).astype(np.float16).view(np.uint16)
    res = synth.f16_bits(synth.normal(46, "res", (lanes, length, cout)))
    scale = synth.uniform(46, "scale", (cout,), 0.1, 2.0)
    xd, bd = to_dev(x, dev), to_dev(b, dev)
    got = to_host(nlc.conv1d(xd, w_tm, bd, k=k, dilation=dil, act=act))
    want = oracle.conv1d_nlc_f16(x, w_tap, b, dil, act=act)
    _close(got, want)
    _elementwise(got, want)
    got = to_host(nlc.conv1d(xd, w_tm, bd, k=k, dilation=dil, act=act, residual=to_dev(res, dev),
                             scale=to_dev(scale, dev)))
    want = oracle.conv1d_nlc_f16(x, w_tap, b, dil, act=act, res_bits=res, scale=scale)
    _close(got, want)
    _elementwise(got, want)
    # the same scale one float past a 16-byte boundary: the direct kernel, the same values
    buf = torch.zeros(cout + 4, dtype=torch.float32, device=dev)
    buf[1:1 + cout] = to_dev(scale, dev)
    got_u = to_host(nlc.conv1d(xd, w_tm, bd, k=k, dilation=dil, act=act, residual=to_dev(res, dev),
                               scale=buf[1:1 + cout]))
    _close(got_u, want)
    _elementwise(got_u, want)


@pytest.mark.parametrize("lanes,length", [(3, 1), (2, 5), (1, 256), (2, 513)])
def test_single_channel_conv_short_and_exact_lengths(dev, lanes, length):
    """The single-output-channel kernels, f16 and f32, at lengths shorter than the halo, one tile
    exactly and one past a tile boundary."""
    cin, k, dil = 96, 7, 9
    x, w, wb, b = _case(47, lanes, length, cin, 1, k)
    w_tap = oracle.tap_weight_f32(synth.from_f16_bits(wb)).astype(np.float16).view(np.uint16)
    got = to_host(nlc.conv1d(to_dev(x, dev), to_dev(nlc.tap_major_weight(wb), dev), to_dev(b, dev), k=k,
                             dilation=dil, act="tanh"))
    want = oracle.conv1d_nlc_f16(x, w_tap, b, dil, act_tanh=True)
    assert got.shape == (lanes, length, 1)
    _close(got, want, tol=2e-3)
    xf = synth.from_f16_bits(x).astype(np.float32)
    got32 = to_host(nlc.conv1d(to_dev(xf, dev), to_dev(nlc.tap_major_weight(w), dev), to_dev(synth.from_f16_bits(b).astype(np.float32), dev),
                               k=k, dilation=dil, act="tanh"))
    want32 = np.tanh(oracle.conv1d_nlc_f32(xf, oracle.tap_weight_f32(w), synth.from_f16_bits(b).astype(np.float32), dil))
    assert rel(got32, want32)[1] < 1e-5
