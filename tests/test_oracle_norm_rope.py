"""Pins the oracle's RMSNorm, RoPE, QK-norm+RoPE+append and KV append restatements against
float64, closed forms and invariants (rotation preserves pair norms; position 0 is the identity;
positions compose), and the library's host RoPE table against the oracle's."""
import numpy as np

import oracle
from dtts import ops, synth


def test_rms_norm_f32_matches_f64_and_f16_rounding_points():
    x = synth.normal(50, "x", (48, 1024))
    g = synth.uniform(50, "g", (1024,), 0.9, 1.1)
    got = oracle.rms_norm_f32(x, g, 1e-6)
    want = oracle.rms_norm_f64(x, g, 1e-6)
    assert np.max(np.abs(got - want) / np.max(np.abs(want))) < 1e-6
    # numpy restatement in f64 of the closed form
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2, -1, keepdims=True) + 1e-6) * g
    assert np.max(np.abs(want - ref)) < 1e-12
    xb, gb = synth.f16_bits(x), synth.f16_bits(g)
    got16 = synth.from_f16_bits(oracle.rms_norm_f16(xb, gb, 1e-6))
    want16 = oracle.rms_norm_f64(synth.from_f16_bits(xb), synth.from_f16_bits(gb), 1e-6)
    # three f16 roundings (m, x/m, *gamma), each at most half an ulp (2^-11 relative)
    assert np.all(np.abs(got16 - want16) <= np.abs(want16) * 3.05 * 2.0 ** -11 + 1e-7)


def test_rope_table_closed_form_and_library_agrees():
    c, s = oracle.rope_table_f32(2048, 128, 1e6)
    t = np.arange(2048)[:, None].astype(np.float64)
    inv = 1.0 / 1e6 ** (2.0 * np.arange(64) / 128.0)
    assert np.max(np.abs(c - np.cos(t * inv))) < 1e-7
    assert np.max(np.abs(s - np.sin(t * inv))) < 1e-7
    lc, ls = ops.rope_table_f32(2048, 128, 1e6)
    assert np.array_equal(lc, c) and np.array_equal(ls, s)


def test_rope_invariants():
    c, s = oracle.rope_table_f32(4096, 128, 1e6)
    x = synth.normal(51, "x", (6, 4, 128))
    y0 = oracle.rope_halfsplit_f32(x, c, s, np.zeros(6, np.int32))
    assert np.array_equal(y0, x)  # position 0: cos 1, sin 0
    pos = synth.randint(51, "pos", (6,), 0, 2047).astype(np.int32)
    y = oracle.rope_halfsplit_f32(x, c, s, pos)
    n_in = x[..., :64] ** 2 + x[..., 64:] ** 2
    n_out = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert np.max(np.abs(n_in - n_out) / (n_in + 1e-3)) < 1e-5
    # composition: rotating by p1 then p2 == rotating by p1 + p2 (to f32 accuracy)
    p2 = synth.randint(51, "p2", (6,), 0, 2047).astype(np.int32)
    yy = oracle.rope_halfsplit_f32(y, c, s, p2)
    direct = oracle.rope_halfsplit_f32(x, c, s, pos + p2)
    assert np.max(np.abs(yy - direct)) < 5e-4
    # the half-split pairing (not interleaved): element i pairs with i + 64
    e = np.zeros((1, 1, 128), np.float32)
    e[0, 0, 3] = 1.0
    r = oracle.rope_halfsplit_f32(e, c, s, np.array([5], np.int32))
    assert set(np.nonzero(r[0, 0])[0]) <= {3, 67}


def test_qk_oracle_matches_numpy_composition_and_append_placement():
    b, heads, n_kv, hd, cap = 5, 4, 2, 128, 64
    c, s = oracle.rope_table_f32(cap, hd, 1e6)
    qkv = synth.normal(52, "qkv", (b, (heads + 2 * n_kv) * hd))
    norms = synth.uniform(52, "n", (2, hd), 0.5, 1.5)
    pos = synth.randint(52, "pos", (b,), 0, cap - 1).astype(np.int32)
    kc = np.full((b, n_kv, cap, hd), 0x5555, np.uint16)
    vc = np.full((b, n_kv, cap, hd), 0x5555, np.uint16)
    q, k = oracle.qk_norm_rope_append_f32(qkv, norms, c, s, pos, kc, vc, heads, n_kv, 1e-6)
    x = qkv.reshape(b, heads + 2 * n_kv, hd).astype(np.float64)

    def norm_rope(v, w, p):
        v = v / np.sqrt(np.mean(v ** 2, -1, keepdims=True) + 1e-6) * w
        cc, ss = c[p][:, None, :], s[p][:, None, :]
        return np.concatenate([v[..., :64] * cc - v[..., 64:] * ss, v[..., 64:] * cc + v[..., :64] * ss], -1)

    assert np.max(np.abs(q - norm_rope(x[:, :heads], norms[0], pos))) < 1e-5
    assert np.max(np.abs(k - norm_rope(x[:, heads:heads + n_kv], norms[1], pos))) < 1e-5
    for bi in range(b):
        assert np.array_equal(kc[bi, :, pos[bi]], synth.f16_bits(k[bi]))
        assert np.array_equal(vc[bi, :, pos[bi]], synth.f16_bits(x[bi, heads + n_kv:].astype(np.float32)))
    mask = np.ones(kc.shape, bool)
    for bi in range(b):
        mask[bi, :, pos[bi]] = False
    assert np.all(kc[mask] == 0x5555) and np.all(vc[mask] == 0x5555)


def test_kv_append_places_exactly():
    b, n_kv, hd, cap = 4, 3, 16, 10
    k = synth.normal(53, "k", (b, n_kv, hd))
    v = synth.normal(53, "v", (b, n_kv, hd))
    pos = np.array([0, 9, 3, 3], np.int32)
    kc = np.zeros((b, n_kv, cap, hd), np.uint16)
    vc = np.zeros_like(kc)
    oracle.kv_append_f32(k, v, pos, kc, vc)
    want = np.zeros_like(kc)
    for bi in range(b):
        want[bi, :, pos[bi]] = k[bi].astype(np.float16).view(np.uint16)
    assert np.array_equal(kc, want)


# qkrope.rs:191-260's cases: (b, t, start, lane offset) on a lane window of a (b + 3)-lane cache
QKROPE_CASES = [(8, 1, 37, 2), (4, 5, 0, 1), (4, 7, 10, 0)]


def _qkrope_f64(qkv, norms, c, s, heads, n_kv, start, eps):
    """An independent float64 evaluation of the composed path: norm, heads first, rope."""
    b, t, _ = qkv.shape
    hd = norms.shape[-1]
    x = qkv.reshape(b, t, heads + 2 * n_kv, hd).astype(np.float64).transpose(0, 2, 1, 3)  # [b, h, t, D]
    cc = c[start:start + t].astype(np.float64)[None, None]
    ss = s[start:start + t].astype(np.float64)[None, None]
    half = hd // 2

    def norm_rope(v, w):
        v = v / np.sqrt(np.mean(v ** 2, -1, keepdims=True) + eps) * w.astype(np.float64)
        return np.concatenate([v[..., :half] * cc - v[..., half:] * ss, v[..., half:] * cc + v[..., :half] * ss], -1)

    return norm_rope(x[:, :heads], norms[0]), norm_rope(x[:, heads:heads + n_kv], norms[1]), x[:, heads + n_kv:]


def test_qkrope_apply_oracle_matches_f64_at_the_reference_cases():
    heads, n_kv, hd, cap, eps = 16, 8, 128, 64, 1e-6
    c, s = oracle.rope_table_f32(cap, hd, 1e6)
    norms = synth.uniform(54, "norms", (2, hd), 0.5, 1.5)
    for b, t, start, off in QKROPE_CASES:
        qkv = synth.normal(54, f"qkv{b}.{t}", (b, t, (heads + 2 * n_kv) * hd))
        kc = np.full((b + 3, n_kv, cap, hd), 0x5555, np.uint16)
        vc = kc.copy()
        q, (k, v) = oracle.qkrope_apply_f32(qkv, norms, c, s, kc[off:off + b], vc[off:off + b], heads, start, eps)
        wq, wk, wv = _qkrope_f64(qkv, norms, c, s, heads, n_kv, start, eps)
        assert q.shape == (b, heads, t, hd) and k.shape == v.shape == (b, n_kv, t, hd)
        assert oracle.abs_and_rel(q.ravel(), wq.astype(np.float32).ravel())[1] < 1e-6
        assert oracle.abs_and_rel(k.ravel(), wk.astype(np.float32).ravel())[1] < 1e-6
        assert np.array_equal(v, wv.astype(np.float32))  # v passes through untouched
        win_k, win_v = kc[off:off + b, :, start:start + t], vc[off:off + b, :, start:start + t]
        assert np.array_equal(win_k, synth.f16_bits(k)) and np.array_equal(win_v, synth.f16_bits(v))
        mask = np.ones(kc.shape, bool)
        mask[off:off + b, :, start:start + t] = False
        assert np.all(kc[mask] == 0x5555) and np.all(vc[mask] == 0x5555), "writes escaped the window"


def test_qkrope_apply_oracle_at_one_position_is_the_decode_form():
    """t = 1 with every lane at `start` is the per-lane decode restatement bit for bit."""
    b, heads, n_kv, hd, cap, start = 6, 4, 2, 128, 32, 19
    c, s = oracle.rope_table_f32(cap, hd, 1e6)
    qkv = synth.normal(55, "qkv", (b, 1, (heads + 2 * n_kv) * hd))
    norms = synth.uniform(55, "n", (2, hd), 0.5, 1.5)
    kc1 = np.zeros((b, n_kv, cap, hd), np.uint16)
    vc1, kc2, vc2 = kc1.copy(), kc1.copy(), kc1.copy()
    q1, (k1, _) = oracle.qkrope_apply_f32(qkv, norms, c, s, kc1, vc1, heads, start, 1e-6)
    q2, k2 = oracle.qk_norm_rope_append_f32(qkv[:, 0], norms, c, s, np.full(b, start, np.int32), kc2, vc2,
                                            heads, n_kv, 1e-6)
    assert np.array_equal(q1[:, :, 0], q2) and np.array_equal(k1[:, :, 0], k2)
    assert np.array_equal(kc1, kc2) and np.array_equal(vc1, vc2)
