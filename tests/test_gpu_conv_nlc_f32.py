"""The channels-last conv at NlcConv's own precision (dtts_conv1d_nlc_f32_ex) through the C ABI.

NlcConv is f32-only (crates/tts-nn/src/nlcconv.rs:185-198). Bars are the reference's own:
abs_and_rel max-rel < 1e-5 (nlc.rs:294-405) against the oracle's NlcConv::cpu_fwd restatement
(oracle.conv1d_nlc_f32, itself pinned to torch's float64 conv1d) and against torch's float64
conv1d directly. Shapes: nlc.rs:294-328's direct cases (odd channel counts: the direct kernel),
nlc.rs:362-398's fused-conv shapes, the codec's own stages (several lanes, per-lane zero
boundaries), the transposed conv's polyphase form, and the fused prologue/epilogue operands.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from dtts import nlc, synth

from _util import rel, to_dev, to_host

pytestmark = pytest.mark.gpu


def _case(seed, lanes, length, cin, cout, k):
    x = synth.normal(seed, "x", (lanes, length, cin))
    w = synth.normal(seed, "w", (cout, cin, k), 0, np.sqrt(2.0 / (cin * k)))
    b = synth.normal(seed, "b", (cout,), 0, 0.01)
    return x, w, b


def _torch_f64(x, w, b, dil, pad_left, snake=None):
    xt = torch.from_numpy(x).double().transpose(1, 2)  # [lanes, cin, L]
    if snake is not None:
        a = torch.from_numpy(np.asarray(snake[0], np.float64))[None, :, None]
        r = torch.from_numpy(np.asarray(snake[1], np.float64))[None, :, None]
        xt = xt + r * torch.sin(a * xt) ** 2
    k = w.shape[2]
    pad_right = (k - 1) * dil - pad_left
    y = F.conv1d(F.pad(xt, (pad_left, pad_right)), torch.from_numpy(w).double(), torch.from_numpy(b).double(),
                 dilation=dil)
    return y.transpose(1, 2).numpy()


@pytest.mark.parametrize("lanes,cin,cout,length,k,dil", [
    (1, 8, 12, 40, 7, 1), (1, 16, 16, 33, 7, 3), (1, 6, 9, 20, 1, 1),             # nlc.rs:294-328
    (1, 96, 96, 4200, 7, 9), (1, 32, 96, 4096, 7, 1), (1, 128, 192, 5000, 7, 3),  # nlc.rs:362-398
    (1, 64, 96, 4097, 1, 1),
    (3, 96, 96, 700, 7, 9), (2, 192, 192, 513, 7, 3), (2, 384, 384, 300, 7, 1),   # codec stages
    (2, 768, 768, 250, 1, 1), (2, 1024, 1536, 60, 7, 1), (2, 96, 1, 900, 7, 1),
    (2, 64, 160, 300, 7, 3), (1, 32, 32, 500, 1, 1), (1, 64, 64, 400, 5, 2),     # each tile width (32, 64, 96)
    (2, 96, 96, 333, 3, 4), (1, 40, 64, 129, 2, 3),                               # and taps below 7
])
def test_causal_conv_f32_matches_oracle_and_torch(dev, lanes, cin, cout, length, k, dil):
    x, w, b = _case(100, lanes, length, cin, cout, k)
    got = to_host(nlc.conv1d(to_dev(x, dev), to_dev(nlc.tap_major_weight(w), dev), to_dev(b, dev), k=k,
                             dilation=dil))
    want = oracle.conv1d_nlc_f32(x, oracle.tap_weight_f32(w), b, dil)
    assert rel(got, want)[1] < 1e-5
    assert rel(got, _torch_f64(x, w, b, dil, (k - 1) * dil))[1] < 1e-5


def test_centered_pad_f32(dev):
    """pad_left below (k-1)*dil: the centred form (config 1's k=7, d=3, pad 9) channels-last."""
    x, w, b = _case(101, 2, 600, 64, 64, 7)
    got = to_host(nlc.conv1d(to_dev(x, dev), to_dev(nlc.tap_major_weight(w), dev), to_dev(b, dev), k=7,
                             dilation=3, pad_left=9))
    assert rel(got, oracle.conv1d_nlc_f32(x, oracle.tap_weight_f32(w), b, 3, pad_left=9))[1] < 1e-5
    assert rel(got, _torch_f64(x, w, b, 3, 9))[1] < 1e-5


@pytest.mark.parametrize("lanes,c,length,k,dil", [(2, 96, 3000, 7, 9), (1, 192, 1100, 1, 1), (2, 384, 300, 7, 3),
                                                   (1, 160, 700, 7, 1), (2, 64, 400, 5, 3)])
def test_fused_snake_residual_f32(dev, lanes, c, length, k, dil):
    """NlcConv's has_snake / has_res (nlc::snake_conv_residual, nlc.rs:40-68) plus the epilogue
    SnakeBeta and y_pre the codec uses."""
    x, w, b = _case(102, lanes, length, c, c, k)
    res = synth.normal(102, "res", (lanes, length, c))
    a1 = synth.uniform(102, "a1", (c,), 0.5, 1.5)
    a2 = synth.uniform(102, "a2", (c,), 0.5, 1.5)
    r1, r2 = (1.0 / a1).astype(np.float32), (1.0 / a2).astype(np.float32)
    y_pre, y = nlc.conv1d(to_dev(x, dev), to_dev(nlc.tap_major_weight(w), dev), to_dev(b, dev), k=k, dilation=dil,
                          snake_in=(to_dev(a1, dev), to_dev(r1, dev)), residual=to_dev(res, dev),
                          snake_out=(to_dev(a2, dev), to_dev(r2, dev)), want_pre=True)
    want_pre = oracle.conv1d_nlc_f32(x, oracle.tap_weight_f32(w), b, dil, snake=(a1, r1), res=res)
    assert rel(to_host(y_pre), want_pre)[1] < 1e-5
    assert rel(to_host(y_pre), _torch_f64(x, w, b, dil, (k - 1) * dil, snake=(a1, r1)) + res)[1] < 1e-5
    assert rel(to_host(y), oracle.snake_nlc_f32(want_pre, a2, r2))[1] < 1e-5


def test_activations_and_scale_f32(dev):
    x, w, b = _case(103, 2, 700, 96, 96, 7)
    scale = synth.uniform(103, "s", (96,), 0.1, 2.0)
    res = synth.normal(103, "res", (2, 700, 96))
    w_tm = to_dev(nlc.tap_major_weight(w), dev)
    plain = oracle.conv1d_nlc_f32(x, oracle.tap_weight_f32(w), b, 1)
    got = to_host(nlc.conv1d(to_dev(x, dev), w_tm, to_dev(b, dev), k=7, act="tanh"))
    assert rel(got, np.tanh(plain))[1] < 1e-5
    got = to_host(nlc.conv1d(to_dev(x, dev), w_tm, to_dev(b, dev), k=7, act="clamp"))
    assert rel(got, np.clip(plain, -1, 1))[1] < 1e-5
    got = to_host(nlc.conv1d(to_dev(x, dev), w_tm, to_dev(b, dev), k=7, residual=to_dev(res, dev),
                             scale=to_dev(scale, dev)))
    assert rel(got, res + scale * plain)[1] < 1e-5


@pytest.mark.parametrize("cin,cout,length,stride", [(1536, 768, 20, 8), (768, 384, 40, 5), (384, 192, 64, 4),
                                                    (192, 96, 128, 3), (8, 6, 12, 2), (12, 8, 9, 5), (16, 16, 50, 2)])
def test_transposed_conv_f32_matches_definition(dev, cin, cout, length, stride):
    """The polyphase transposed conv at f32 against the scatter definition (nlc.rs:329-360 shapes
    and the codec's four)."""
    lanes, k = 2, 2 * stride
    x = synth.normal(104, "x", (lanes, length, cin))
    w = synth.normal(104, "w", (cin, cout, k), 0, np.sqrt(2.0 / (cout * k)))
    b = synth.normal(104, "b", (cout,), 0, 0.01)
    w_tm = nlc.transpose_tap_major_weight(w, stride)
    got = to_host(nlc.causal_conv_transpose1d(to_dev(x, dev), to_dev(w_tm, dev),
                                              to_dev(nlc.transpose_bias(b, stride), dev), stride))
    for li in range(lanes):
        want = oracle.conv_transpose1d_causal_f64(x[li], w, b, stride)
        assert rel(got[li], want)[1] < 1e-5


@pytest.mark.parametrize("lanes,cin,length,k,dil,pad,ops", [
    (2, 96, 900, 7, 1, None, "tanh"), (3, 96, 1000, 7, 3, None, "clamp"), (1, 64, 257, 7, 9, None, "snake_res"),
    (2, 32, 300, 3, 21, None, "pre_snake_out"), (1, 128, 513, 1, 1, None, "bias"), (2, 96, 700, 7, 2, 5, "tanh"),
])
def test_single_output_channel_f32(dev, lanes, cin, length, k, dil, pad, ops):
    """cin -> 1 (the waveform conv at f32): the window kernel against the oracle and torch f64, with
    each epilogue and prologue operand, several lanes, halos up to 64 and partial last tiles."""
    pad = (k - 1) * dil if pad is None else pad
    x, w, b = _case(105, lanes, length, cin, 1, k)
    kw = dict(k=k, dilation=dil, pad_left=pad)
    w_tm = to_dev(nlc.tap_major_weight(w), dev)
    want = oracle.conv1d_nlc_f32(x, oracle.tap_weight_f32(w), b, dil, pad_left=pad)
    exact = _torch_f64(x, w, b, dil, pad)
    if ops in ("tanh", "clamp"):
        got = to_host(nlc.conv1d(to_dev(x, dev), w_tm, to_dev(b, dev), act=ops, **kw))
        f = np.tanh if ops == "tanh" else (lambda v: np.clip(v, -1, 1))
        assert rel(got, f(want))[1] < 1e-5 and rel(got, f(exact))[1] < 1e-5
    elif ops == "snake_res":
        a1 = synth.uniform(105, "a1", (cin,), 0.5, 1.5)
        r1 = (1.0 / a1).astype(np.float32)
        res = synth.normal(105, "res", (lanes, length, 1))
        got = to_host(nlc.conv1d(to_dev(x, dev), w_tm, to_dev(b, dev), snake_in=(to_dev(a1, dev), to_dev(r1, dev)),
                                 residual=to_dev(res, dev), **kw))
        want = oracle.conv1d_nlc_f32(x, oracle.tap_weight_f32(w), b, dil, pad_left=pad, snake=(a1, r1), res=res)
        assert rel(got, want)[1] < 1e-5
        assert rel(got, _torch_f64(x, w, b, dil, pad, snake=(a1, r1)) + res)[1] < 1e-5
    elif ops == "pre_snake_out":
        a2 = synth.uniform(105, "a2", (1,), 0.5, 1.5)
        r2 = (1.0 / a2).astype(np.float32)
        y_pre, y = nlc.conv1d(to_dev(x, dev), w_tm, to_dev(b, dev), snake_out=(to_dev(a2, dev), to_dev(r2, dev)),
                              want_pre=True, **kw)
        assert rel(to_host(y_pre), want)[1] < 1e-5
        assert rel(to_host(y), oracle.snake_nlc_f32(want, a2, r2))[1] < 1e-5
    else:
        got = to_host(nlc.conv1d(to_dev(x, dev), w_tm, to_dev(b, dev), **kw))
        assert rel(got, want)[1] < 1e-5 and rel(got, exact)[1] < 1e-5


# ---------------------------------------------------------------- the split route
# dtts_conv1d_nlc_f32_split: the same f32 NlcConv at f32 accuracy on the f16 matrix cores (x and the
# residual split into f16 hi/lo pairs, the weight scaled by 2^s and split once at load, three f16
# products per term, xl*wl dropped). Held to NlcConv's own bar, max-rel < 1e-5 (nlc.rs:294-405),
# against the oracle's NlcConv restatement and torch float64, at nlc.rs:362-398's fused-conv shapes
# and the codec's stages.

SPLIT_SHAPES = [
    (1, 96, 96, 4200, 7, 9), (1, 32, 96, 4096, 7, 1), (1, 128, 192, 5000, 7, 3), (1, 64, 96, 4097, 1, 1),  # nlc.rs
    (3, 96, 96, 700, 7, 9), (2, 192, 192, 513, 7, 3), (2, 384, 384, 300, 7, 1), (2, 768, 768, 250, 1, 1),   # codec
    (2, 1024, 1536, 60, 7, 1), (2, 192, 192, 600, 1, 1), (2, 384, 384, 300, 1, 1),
]


@pytest.mark.parametrize("lanes,cin,cout,length,k,dil", SPLIT_SHAPES)
def test_split_conv_matches_oracle_and_torch(dev, lanes, cin, cout, length, k, dil):
    x, w, b = _case(110, lanes, length, cin, cout, k)
    w3, inv = nlc.split_weight(to_dev(nlc.tap_major_weight(w), dev), k)
    got = to_host(nlc.conv1d_f32_split(to_dev(x, dev), w3, inv, to_dev(b, dev), k=k, dilation=dil))
    want = oracle.conv1d_nlc_f32(x, oracle.tap_weight_f32(w), b, dil)
    assert rel(got, want)[1] < 1e-5, rel(got, want)
    assert rel(got, _torch_f64(x, w, b, dil, (k - 1) * dil))[1] < 1e-5


@pytest.mark.parametrize("lanes,c,length,k,dil", [(2, 96, 3000, 7, 9), (1, 192, 1100, 1, 1), (2, 384, 300, 7, 3)])
def test_split_conv_residual_snake_out(dev, lanes, c, length, k, dil):
    """The codec's epilogue on the split route: bias, residual, y_pre and the output SnakeBeta at
    full precision, and a centred pad."""
    x, w, b = _case(111, lanes, length, c, c, k)
    res = synth.normal(111, "res", (lanes, length, c))
    a2 = synth.uniform(111, "a2", (c,), 0.5, 1.5)
    r2 = (1.0 / a2).astype(np.float32)
    w3, inv = nlc.split_weight(to_dev(nlc.tap_major_weight(w), dev), k)
    pad = (k - 1) * dil // 2
    y_pre, y = nlc.conv1d_f32_split(to_dev(x, dev), w3, inv, to_dev(b, dev), k=k, dilation=dil, pad_left=pad,
                                    residual=to_dev(res, dev), snake_out=(to_dev(a2, dev), to_dev(r2, dev)),
                                    want_pre=True)
    want_pre = oracle.conv1d_nlc_f32(x, oracle.tap_weight_f32(w), b, dil, pad_left=pad, res=res)
    assert rel(to_host(y_pre), want_pre)[1] < 1e-5
    assert rel(to_host(y_pre), _torch_f64(x, w, b, dil, pad) + res)[1] < 1e-5
    assert rel(to_host(y), oracle.snake_nlc_f32(want_pre, a2, r2))[1] < 1e-5


def test_split_conv_snake_out_past_the_reduction_range(dev):
    """Every eighth channel's alpha puts |alpha * y_pre| past 2^20, where the epilogue's group of
    eight takes the library sine for all eight values: the far channels keep y - y_pre in [0, r]
    (at alpha 3e9 their sine turns on y_pre's last bits, which the split store rounds), the other
    channels (the far ones' neighbours in the same groups) are SnakeBeta of y_pre within 1e-5 of
    max(|y_pre|, r, 1) (fused.rs:2356-2391's scale; y_pre is stored split, to 2^-22 of itself)."""
    lanes, c, length, k = 1, 96, 700, 7
    x, w, b = _case(113, lanes, length, c, c, k)
    a2 = synth.uniform(113, "a2", (c,), 0.5, 1.5)
    a2[3::8] = 3.0e9
    r2 = (1.0 / synth.uniform(113, "b2", (c,), 0.5, 1.5)).astype(np.float32)
    w3, inv = nlc.split_weight(to_dev(nlc.tap_major_weight(w), dev), k)
    y_pre, y = nlc.conv1d_f32_split(to_dev(x, dev), w3, inv, to_dev(b, dev), k=k, dilation=1,
                                    snake_out=(to_dev(a2, dev), to_dev(r2, dev)), want_pre=True)
    y_pre, y = to_host(y_pre).astype(np.float64), to_host(y).astype(np.float64)
    big = np.zeros(c, bool)
    big[3::8] = True
    assert (np.abs(a2 * y_pre) > 2.0 ** 20)[..., big].mean() > 0.99
    scale = np.maximum(np.maximum(np.abs(y_pre), r2), 1.0)
    want = y_pre + r2 * np.sin(a2 * y_pre) ** 2
    assert np.max((np.abs(y - want) / scale)[..., ~big]) < 1e-5
    d = (y - y_pre)[..., big]
    tol = 1e-6 * scale[..., big]
    assert np.all(d >= -tol) and np.all(d <= r2[big] + tol)


def test_split_conv_refuses_what_it_has_no_kernel_for(dev):
    """A prologue SnakeBeta, an activation or a shape off the split tiles: DTTS_ERR_UNSUPPORTED,
    nothing written (the shim then calls dtts_conv1d_nlc_f32_ex). A bias off 16-byte alignment or
    a w_inv that is not a power of two: DTTS_ERR_INVALID, nothing written."""
    import ctypes

    from dtts import DttsError
    from dtts._lib import call, stream_handle

    x, w, b = _case(112, 1, 300, 96, 96, 7)
    w3, inv = nlc.split_weight(to_dev(nlc.tap_major_weight(w), dev), 7)
    xd = to_dev(x, dev)
    y = torch.full((1, 300, 96), 7.0, dtype=torch.float32, device=dev)
    alpha = torch.ones(96, dtype=torch.float32, device=dev)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=dev)
    for in_alpha, act in ((alpha, 0), (None, 1)):
        d = nlc.ConvDesc(1, 300, 96, 96, 7, 1, 6, xd.data_ptr(), w3.data_ptr(), None,
                         None if in_alpha is None else in_alpha.data_ptr(),
                         None if in_alpha is None else in_alpha.data_ptr(), None, None, None, None, y.data_ptr(),
                         act, None)
        with pytest.raises(DttsError, match="no split kernel"):
            call("dtts_conv1d_nlc_f32_split", ctypes.byref(d), ctypes.c_float(inv), ws.data_ptr(), ws.numel(),
                 stream_handle())
    x40, w40, _ = _case(112, 1, 300, 40, 96, 7)
    w3b, invb = nlc.split_weight(to_dev(nlc.tap_major_weight(w40), dev), 7)
    with pytest.raises(DttsError, match="no split kernel"):
        nlc.conv1d_f32_split(to_dev(x40, dev), w3b, invb, k=7)
    bias = torch.zeros(100, dtype=torch.float32, device=dev)
    for bias_ptr, w_inv, msg in ((bias.data_ptr() + 4, inv, "16-byte aligned"), (None, inv * 1.5, "power of two")):
        d = nlc.ConvDesc(1, 300, 96, 96, 7, 1, 6, xd.data_ptr(), w3.data_ptr(), bias_ptr, None, None, None, None,
                         None, None, y.data_ptr(), 0, None)
        with pytest.raises(DttsError, match=msg):
            call("dtts_conv1d_nlc_f32_split", ctypes.byref(d), ctypes.c_float(w_inv), ws.data_ptr(), ws.numel(),
                 stream_handle())
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
