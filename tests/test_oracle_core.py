"""Pins the CPU oracle's conversion, snake, gather, conv and transposed-conv restatements.

Each check is independent of the oracle's own formula: numpy's float16 cast, double-precision
definitions, torch's CPU conv1d / conv_transpose1d in float64 (library routines), and the
reference's own test constructions (pad, narrow, cat) rebuilt in numpy. Shapes are the
reference's known-answer-test shapes, cited per test.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from dtts import synth

from _util import rel


# ---------------------------------------------------------------- f16 storage points

def test_f16_to_f32_exhaustive_matches_numpy():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, 1e-8, 2.0 ** -24, 2.0 ** -25,
                     2.0 ** -25 * 1.0000001, 3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 * (1 - 2 ** -11),
                     np.inf, -np.inf, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 0.1, -0.1],
                    dtype=np.float32)
    x = np.concatenate([bits.view(np.float32), edge])
    x = x[~np.isnan(x)]
    got = oracle.f32_to_f16(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- snake

def _snake_f64(x, a, r):
    return x + r * np.sin(a * x) ** 2


def test_snake_matches_double_precision_over_generator_range():
    # crates/tts-nn/src/fused.rs:2356-2391: c=8, len=2048, x over +-12, alpha 0.03..2.33,
    # brecip 0.5 + j; error scaled by max(|x|, r, 1) < 1e-6.
    c, length = 8, 2048
    xs = (-12.0 + 24.0 * (np.arange(c * length) % length) / (length - 1)).astype(np.float32)
    al = np.array([0.03 + 2.3 * j / (c - 1) for j in range(c)], np.float32)
    br = np.array([0.5 + j for j in range(c)], np.float32)
    x = xs.reshape(1, c, length)
    got = oracle.snake_ncl_f32(x, al, br)
    want = _snake_f64(x.astype(np.float64), al.astype(np.float64)[None, :, None],
                      br.astype(np.float64)[None, :, None])
    scale = np.maximum(np.maximum(np.abs(x), br[None, :, None]), 1.0)
    assert np.max(np.abs(got - want) / scale) < 1e-6


def test_snake_wide_sweep_within_2e6():
    # crates/tts-nn/src/fused.rs:2227-2337: x over +-30, alpha 0.05..2.55, bound 2e-6.
    c, length = 8, 4096
    xs = (-30.0 + 60.0 * (np.arange(c * length) % length) / (length - 1)).astype(np.float32)
    al = np.array([0.05 + 2.5 * j / (c - 1) for j in range(c)], np.float32)
    br = np.array([0.5 + j for j in range(c)], np.float32)
    x = xs.reshape(length, c)  # channels-last, as qwen3tts's codec calls it
    got = oracle.snake_nlc_f32(x, al, br)
    want = oracle.snake_nlc_f64(x, al, br)
    scale = np.maximum(np.maximum(np.abs(x), br[None, :]), 1.0)
    assert np.max(np.abs(got - want) / scale) < 2e-6


def test_snake_layouts_agree_and_zero_is_fixed():
    x = synth.normal(1, "x", (3, 7, 33), 0, 2)
    a = np.exp(synth.normal(1, "a", (7,)))
    r = np.exp(synth.normal(1, "r", (7,)))
    ncl = oracle.snake_ncl_f32(x, a, r)
    nlc = oracle.snake_nlc_f32(np.ascontiguousarray(x.transpose(0, 2, 1)), a, r)
    assert np.array_equal(ncl, nlc.transpose(0, 2, 1))
    assert np.all(oracle.snake_nlc_f32(np.zeros((4, 7), np.float32), a, r) == 0)


def _sweep(c, length, lo, hi):
    return (lo + (hi - lo) * (np.arange(c * length) % length) / (length - 1)).astype(np.float32)


def test_folded_snakes_match_double_precision_over_wide_sweep():
    # crates/tts-nn/src/fused.rs:2227-2283 ("snake_folded", "snake (alpha)"): x over +-30, alpha
    # 0.05..2.55, error scaled by max(|x|, 1) resp. max(|alpha x|, 1), bound 2e-6 (fused.rs:2332).
    c, length = 8, 4096
    x = _sweep(c, length, -30.0, 30.0).reshape(1, c, length)
    al = np.array([0.05 + 2.5 * j / (c - 1) for j in range(c)], np.float32)
    xd = x.astype(np.float64)
    got = oracle.snake_folded_f32(x)
    assert np.max(np.abs(got - (xd + np.sin(xd) ** 2)) / np.maximum(np.abs(xd), 1.0)) < 2e-6
    u = al.astype(np.float64)[None, :, None] * xd
    got = oracle.snake_alpha_f32(x, al)
    assert np.max(np.abs(got - (u + np.sin(u) ** 2)) / np.maximum(np.abs(u), 1.0)) < 2e-6
    # the output is u + sin^2(u), not x + sin^2(u) (SnakeBeta with r = 1): a dropped alpha fails
    assert np.max(np.abs(got - (xd + np.sin(u) ** 2))) > 1.0


def test_folded_snakes_reduce_to_each_other_and_to_snake_beta():
    """snake_forms_agree (fused.rs:2429-2446) plus the identities that fix the forms exactly:
    snake_alpha at alpha = 1 and SnakeBeta at alpha = 1, 1/beta = 1 are x + sin^2(x) bit for bit,
    and snake_alpha(x, a) is snake_folded of the f32 product a x."""
    x = synth.normal(3, "x", (2, 7, 33), 0, 2)
    a = synth.normal(3, "a", (7,))
    folded = oracle.snake_folded_f32(x)
    composed = (x + np.sin(x) ** 2).astype(np.float32)  # numpy's f32 sin, the candle composed form
    assert np.max(np.abs(folded - composed)) < 1e-5
    one = np.ones(7, np.float32)
    assert np.array_equal(oracle.snake_alpha_f32(x, one), folded)
    assert np.array_equal(oracle.snake_ncl_f32(x, one, one), folded)
    ax = (x * a[None, :, None]).astype(np.float32)
    assert np.array_equal(oracle.snake_alpha_f32(x, a), oracle.snake_folded_f32(ax))
    assert np.all(oracle.snake_folded_f32(np.zeros(5, np.float32)) == 0)


def test_snake_f16_is_one_rounding_of_f32():
    x = synth.normal(2, "x", (64, 96), 0, 3)
    xb = synth.f16_bits(x)
    a = synth.uniform(2, "a", (96,), 0.5, 1.5)
    r = 1.0 / a
    got = oracle.snake_nlc_f16(xb, a, r)
    want = synth.f16_bits(oracle.snake_nlc_f32(synth.from_f16_bits(xb), a, r))
    assert np.array_equal(got, want)
    ncl = oracle.snake_ncl_f16(np.ascontiguousarray(xb.reshape(1, 64, 96).transpose(0, 2, 1)), a, r)
    assert np.array_equal(ncl.transpose(0, 2, 1).reshape(64, 96), got)


# ---------------------------------------------------------------- im2col (bit-exact)

def _cat_matrix(x, k, dil, pad_l):
    cin, length = x.shape
    pad_r = (k - 1) * dil - pad_l
    xp = np.pad(x, ((0, 0), (pad_l, max(pad_r, 0))))
    return np.concatenate([xp[:, t * dil: t * dil + length] for t in range(k)], axis=0)


@pytest.mark.parametrize("cin,length,k,dil", [(3, 11, 3, 1), (8, 17, 7, 3), (6, 9, 1, 1)])
def test_im2col_matches_cat_matrix(cin, length, k, dil):
    # crates/tts-nn/src/im2col.rs:177-199
    x = synth.normal(3, f"im2col{cin}", (cin, length))
    got = oracle.im2col_tap_major_f32(x, k, dil, (k - 1) * dil)
    assert np.array_equal(got, _cat_matrix(x, k, dil, (k - 1) * dil))


@pytest.mark.parametrize("cin,length,k,dil,pad", [(4, 15, 3, 1, 1), (8, 64, 7, 3, 9),
                                                   (2, 65, 11, 5, 25), (128, 444, 3, 1, 1)])
def test_im2col_centered_matches_windows(cin, length, k, dil, pad):
    # crates/tts-nn/src/im2col.rs:204-239
    x = synth.normal(4, f"cent{cin}", (cin, length))
    got = oracle.im2col_tap_major_f32(x, k, dil, pad)
    assert np.array_equal(got, _cat_matrix(x, k, dil, pad))


# ---------------------------------------------------------------- weight layouts

def test_weight_layouts_are_the_stated_permutations():
    w = synth.normal(5, "w", (6, 4, 7))  # torch [out, in, k]
    assert np.array_equal(oracle.tap_weight_f32(w), w.transpose(2, 1, 0))
    assert np.array_equal(oracle.tap_major_weight_f32(w), w.transpose(0, 2, 1).reshape(6, 28))
    b = synth.normal(5, "b", (5,))
    assert np.array_equal(oracle.transpose_bias_f32(b, 3), np.tile(b, 3))


# ---------------------------------------------------------------- convs against torch f64

def _torch_causal_nlc(x, w_oik, b, dil, pad_left=None):
    """x [lanes, L, cin] -> [lanes, L, cout] through torch's conv1d (f64), padding (pl, pr)."""
    cout, cin, k = w_oik.shape
    pl = (k - 1) * dil if pad_left is None else pad_left
    pr = (k - 1) * dil - pl
    xt = torch.from_numpy(np.ascontiguousarray(x.transpose(0, 2, 1))).double()
    xt = F.pad(xt, (pl, pr))
    y = F.conv1d(xt, torch.from_numpy(w_oik).double(),
                 None if b is None else torch.from_numpy(b).double(), dilation=dil)
    return y.numpy().transpose(0, 2, 1)


@pytest.mark.parametrize("cin,cout,length,k,dil", [
    (8, 12, 40, 7, 1), (16, 16, 33, 7, 3), (6, 9, 20, 1, 1),          # nlc.rs:294-328
    (96, 96, 4200, 7, 9), (32, 96, 4096, 7, 1), (64, 96, 4097, 1, 1),  # nlc.rs:362-398
])
def test_nlc_conv_matches_torch_f64(cin, cout, length, k, dil):
    x = synth.normal(6, f"x{cin}{length}", (2, length, cin))
    w = synth.normal(6, f"w{cin}{cout}{k}", (cout, cin, k), 0, 0.1)
    b = synth.normal(6, f"b{cout}", (cout,), 0, 0.1)
    got = oracle.conv1d_nlc_f32(x, oracle.tap_weight_f32(w), b, dil)
    want = _torch_causal_nlc(x, w, b, dil)
    assert rel(got, want)[1] < 1e-5
    got64 = oracle.conv1d_nlc_f64(x, oracle.tap_weight_f32(w), b, dil)
    assert np.max(np.abs(got64 - want)) < 1e-10


@pytest.mark.parametrize("length,c,k,dil", [(5000, 96, 1, 1), (4100, 192, 7, 3)])
def test_snake_conv_residual_is_the_composition(length, c, k, dil):
    # crates/tts-nn/src/nlc.rs:264-288: res + conv(snake(x)) against the three ops.
    x = synth.normal(7, "x", (1, length, c))
    res = synth.normal(7, "res", (1, length, c))
    w = (synth.normal(7, "w", (c, c, k)) / np.sqrt(k * c)).astype(np.float32)
    b = synth.normal(7, "b", (c,), 0, 0.1)
    a = synth.uniform(7, "a", (c,), 0.5, 2.0)
    r = synth.uniform(7, "r", (c,), 0.2, 1.5)
    wt = oracle.tap_weight_f32(w)
    got = oracle.conv1d_nlc_f32(x, wt, b, dil, snake=(a, r), res=res)
    snaked = oracle.snake_nlc_f32(x, a, r)
    want = _torch_causal_nlc(snaked, w, b, dil) + res
    assert rel(got, want)[1] < 1e-5


@pytest.mark.parametrize("cin,cout,length,stride,mult", [
    (8, 6, 12, 2, 1), (8, 6, 12, 2, 2), (12, 8, 9, 5, 2), (10, 7, 11, 3, 2), (9, 5, 7, 4, 1),
])
def test_transposed_conv_is_one_causal_conv(cin, cout, length, stride, mult):
    # crates/tts-nn/src/nlc.rs:329-360: the polyphase rewrite against the transposed conv.
    k = mult * stride
    x = synth.normal(8, f"x{cin}", (1, length, cin))
    w = synth.normal(8, f"w{cin}{cout}", (cin, cout, k), 0, 0.1)
    b = synth.normal(8, f"b{cout}", (cout,), 0, 0.1)
    # torch's ConvTranspose1d, then drop the trailing k - stride (lib.rs:962-982)
    yt = F.conv_transpose1d(torch.from_numpy(np.ascontiguousarray(x.transpose(0, 2, 1))).double(),
                            torch.from_numpy(w).double(), torch.from_numpy(b).double(), stride=stride)
    want = yt.numpy()[:, :, : length * stride].transpose(0, 2, 1)[0]
    scatter = oracle.conv_transpose1d_causal_f64(x[0], w, b, stride)
    assert np.max(np.abs(scatter - want)) < 1e-12
    wtap = oracle.transpose_tap_weight_f32(w, stride)
    btap = oracle.transpose_bias_f32(b, stride)
    y = oracle.conv1d_nlc_f32(x, wtap, btap, 1)  # [1, L, stride*cout]
    got = y.reshape(length * stride, cout)
    assert rel(got, want)[1] < 1e-5


@pytest.mark.parametrize("cout,cin,length,k,dil", [(8, 4, 15, 3, 1), (8, 8, 64, 7, 3),
                                                   (4, 4, 65, 11, 5), (128, 128, 444, 3, 1)])
def test_centered_ncl_gemm_matches_torch(cout, cin, length, k, dil):
    # crates/tts-nn/src/lib.rs:1330-1366
    pad = (k - 1) * dil // 2
    x = synth.normal(9, f"x{cin}{length}", (1, cin, length))
    w = synth.normal(9, f"w{cout}{k}", (cout, cin, k), 0, 0.1)
    b = synth.normal(9, f"b{cout}", (cout,))
    want = F.conv1d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                    torch.from_numpy(b).double(), padding=pad, dilation=dil).numpy()
    got = oracle.conv1d_ncl_gemm_f32(x, oracle.tap_major_weight_f32(w), b, k, dil, pad)
    assert rel(got, want)[1] < 1e-5


def test_cat_gemm_route_matches_direct():
    x = synth.normal(10, "x", (1, 777, 64))
    w = synth.normal(10, "w", (48, 64, 7), 0, 0.1)
    b = synth.normal(10, "b", (48,))
    wt = oracle.tap_weight_f32(w)
    direct = oracle.conv1d_nlc_f32(x, wt, b, 3)
    cat = oracle.conv1d_nlc_cat_gemm_f32(x[0], wt, b, 3)
    assert rel(cat, direct[0])[1] < 1e-5


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (7, 13, 5), (97, 33, 300), (6, 16, 256), (200, 3100, 70)])
def test_sgemm_matches_f64(m, n, k):
    a = synth.normal(11, f"a{m}{k}", (m, k))
    b = synth.normal(11, f"b{k}{n}", (k, n))
    got = oracle.sgemm(a, b)
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert rel(got, want)[1] < 1e-5


def test_f16_conv_storage_points():
    # f16 form: with f16 inputs widened exactly, f32 accumulation and one rounding, the result is
    # within half an ulp of the f64 conv of the same (f16) values, plus accumulation error.
    x = synth.f16_bits(synth.normal(12, "x", (2, 300, 32)))
    w = synth.normal(12, "w", (48, 32, 7), 0, 0.05)
    wt = synth.f16_bits(oracle.tap_weight_f32(w))
    b = synth.f16_bits(synth.normal(12, "b", (48,), 0, 0.01))
    res = synth.f16_bits(synth.normal(12, "res", (2, 300, 48)))
    a = synth.uniform(12, "a", (32,), 0.5, 1.5)
    r = (1.0 / a).astype(np.float32)
    got = synth.from_f16_bits(oracle.conv1d_nlc_f16(x, wt, b, 3, snake=(a, r), res_bits=res))
    sn = synth.from_f16_bits(oracle.snake_nlc_f16(x, a, r))
    want = oracle.conv1d_nlc_f64(sn, synth.from_f16_bits(wt), synth.from_f16_bits(b), 3,
                                 res=synth.from_f16_bits(res))
    err = np.abs(got - want)
    assert np.all(err <= np.abs(want) * 2.0 ** -11 + 1e-4)
