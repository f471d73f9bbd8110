"""Shared pieces of the decoder-stack tests: small geometries, seeded inputs, and an independent
float64 restatement of Stack::forward's decode step (crates/qwen3tts/src/qwen3.rs:294-467) in
numpy, with the reference's f16 roundings at the same points (projection inputs, weights, cache
entries, and projection outputs where Proj::Half takes candle's f16 matmul) and everything else in
float64."""
from dataclasses import replace

import numpy as np

from dtts import stack, synth

SMALL = stack.Geometry(dim=256, layers=2, heads=4, n_kv=2, head_dim=128, ffn=512, capacity=64)
# no QK-norm, LayerScale, a sliding window, D = 64, one query head per kv head
WINDOWED = stack.Geometry(dim=128, layers=2, heads=4, n_kv=4, head_dim=64, ffn=256, eps=1e-5,
                          rope_base=10_000.0, qk_norm=False, layer_scale=True, window=5, capacity=32)


def with_layers(geo, n):
    return replace(geo, layers=n)


def inputs(geo, seed, lanes, cap, fill=True, weight="f16"):
    """x [lanes, dim] f32 and per-layer caches, pre-filled with N(0,1) history when fill is set:
    uint16 f16 bits for an f16 stack, float32 for the other weight kinds (Stack::load's kv dtype)."""
    x = synth.normal(seed, "stack.x", (lanes, geo.dim))
    shape = (lanes, geo.n_kv, cap, geo.head_dim)
    f16 = weight == "f16"
    kc, vc = [], []
    for i in range(geo.layers):
        if fill:
            k, v = synth.normal(seed, f"stack.k{i}", shape), synth.normal(seed, f"stack.v{i}", shape)
            kc.append(synth.f16_bits(k) if f16 else k.astype(np.float32))
            vc.append(synth.f16_bits(v) if f16 else v.astype(np.float32))
        else:
            kc.append(np.zeros(shape, np.uint16 if f16 else np.float32))
            vc.append(np.zeros(shape, np.uint16 if f16 else np.float32))
    return x, kc, vc


def _q8(w):
    """Q8_0 blocks of an [n, k] weight as ggml's quantize_row_q8_0 forms them, in numpy: per 32-block
    amax, d = amax / 127 and id = 1 / d in f32, codes rounded half away from zero, d stored in f16.
    Returns (codes [n, k/32, 32] float64, d [n, k/32] float64)."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    wb = w.reshape(n, k // 32, 32)
    d = (np.abs(wb).max(-1) / np.float32(127)).astype(np.float32)
    inv = np.zeros_like(d)
    np.divide(np.float32(1), d, out=inv, where=d != 0)
    t = (wb * inv[..., None]).astype(np.float32).astype(np.float64)
    q = np.sign(t) * np.floor(np.abs(t) + 0.5)
    return q, d.astype(np.float16).astype(np.float64)


def proj_kind_f64(a, w, weight):
    """Proj::forward for the f32 and Q8_0 weight kinds in float64 (crates/tts-nn/src/lib.rs:509-531):
    the dense product, the dequantized weight times the activations (q8_0_a32), or both sides
    quantized per block and the integer block dots scaled by the two f16 scales (q8_0)."""
    a = np.asarray(a, np.float64)
    if weight == "f32":
        return a @ np.asarray(w, np.float64).T
    qw, dw = _q8(w)
    if weight == "q8_0_a32":
        deq = (qw * dw[..., None]).reshape(w.shape)
        return a @ deq.T
    qa, da = _q8(a.astype(np.float32))
    dots = np.einsum("mbj,nbj->mnb", qa, qw)
    return (dots * da[:, None, :] * dw[None, :, :]).sum(-1)


def _eligible(m, k, n):
    """skinny::eligible (crates/tts-nn/src/skinny.rs:123-131): f32 output; else candle's f16 matmul."""
    return m <= 48 and m % 8 == 0 and k % 32 == 0 and n % 64 == 0


def _h(a):
    """Round to f16 (numpy's conversion is round-to-nearest-even) and back, in float64."""
    return np.asarray(a, np.float64).astype(np.float16).astype(np.float64)


def _rms(x, g, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * g


def _rope(x, pos, geo):
    half = geo.head_dim // 2
    i = np.arange(half, dtype=np.float64)
    freq = 1.0 / geo.rope_base ** (2.0 * i / geo.head_dim)
    ph = pos[:, None, None].astype(np.float64) * freq  # [b, 1, half]
    c, s = np.cos(ph), np.sin(ph)
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)


def stack_f64(geo, layers, final_norm, x, kc, vc, pos, weight="f16"):
    """Returns (out [b, dim] float64, kc, vc) with the caches as new arrays (uint16 f16 bits for an
    f16 stack; float32 for the other weight kinds, whose step rounds nothing to f16)."""
    if weight != "f16":
        return _stack_dense_f64(geo, layers, final_norm, x, kc, vc, pos, weight)
    b = x.shape[0]
    hd, heads, n_kv = geo.head_dim, geo.heads, geo.n_kv
    qw, kvw, gqa = heads * hd, n_kv * hd, heads // n_kv
    pos = np.broadcast_to(np.asarray(pos, np.int64), (b,))
    kc = [k.copy() for k in kc]
    vc = [v.copy() for v in vc]
    h = np.asarray(x, np.float64)

    def out(y, k, n):  # Proj::Half's routing by lane count (skinny.rs:123-131)
        return y if _eligible(b, k, n) else _h(y)

    for li, L in enumerate(layers):
        a = _h(_rms(h, L["attn_norm"], geo.eps))
        wqkv = _h(np.concatenate([L["wq"], L["wk"], L["wv"]], 0))
        qkv = out(a @ wqkv.T, geo.dim, wqkv.shape[0])
        q = qkv[:, :qw].reshape(b, heads, hd)
        k = qkv[:, qw:qw + kvw].reshape(b, n_kv, hd)
        v = qkv[:, qw + kvw:].reshape(b, n_kv, hd)
        if geo.qk_norm:
            q = _rms(q, np.float64(L["q_norm"]) / np.sqrt(hd), geo.eps)
            k = _rms(k, L["k_norm"], geo.eps)
        q, k = _rope(q, pos, geo), _rope(k, pos, geo)
        if not geo.qk_norm:
            q = q / np.sqrt(hd)
        for i in range(b):
            kc[li][i, :, pos[i]] = synth.f16_bits(k[i])
            vc[li][i, :, pos[i]] = synth.f16_bits(v[i])
        att = np.empty((b, heads, hd))
        for i in range(b):
            hi = pos[i] + 1
            lo = hi - geo.window if geo.window and hi > geo.window else 0
            kk = synth.from_f16_bits(kc[li][i, :, lo:hi]).astype(np.float64)  # [n_kv, n, hd]
            vv = synth.from_f16_bits(vc[li][i, :, lo:hi]).astype(np.float64)
            qg = q[i].reshape(n_kv, gqa, hd)
            s = np.einsum("hgd,hnd->hgn", qg, kk)
            e = np.exp(s - s.max(-1, keepdims=True))
            att[i] = np.einsum("hgn,hnd->hgd", e / e.sum(-1, keepdims=True), vv).reshape(heads, hd)
        o = out(_h(att.reshape(b, qw)) @ _h(L["wo"]).T, qw, geo.dim)
        if geo.layer_scale:
            o = o * L["attn_scale"]
        h = h + o
        a = _h(_rms(h, L["ffn_norm"], geo.eps))
        g, u = out(a @ _h(L["gate"]).T, geo.dim, geo.ffn), out(a @ _h(L["up"]).T, geo.dim, geo.ffn)
        t = _h(g / (1.0 + np.exp(-g)) * u)
        m = out(t @ _h(L["down"]).T, geo.ffn, geo.dim)
        if geo.layer_scale:
            m = m * L["mlp_scale"]
        h = h + m
    return _rms(h, final_norm, geo.eps), kc, vc


def _stack_dense_f64(geo, layers, final_norm, x, kc, vc, pos, weight):
    b = x.shape[0]
    hd, heads, n_kv = geo.head_dim, geo.heads, geo.n_kv
    qw, kvw, gqa = heads * hd, n_kv * hd, heads // n_kv
    pos = np.broadcast_to(np.asarray(pos, np.int64), (b,))
    kc = [k.copy() for k in kc]
    vc = [v.copy() for v in vc]
    h = np.asarray(x, np.float64)
    for li, L in enumerate(layers):
        a = _rms(h, L["attn_norm"], geo.eps)
        qkv = proj_kind_f64(a, np.concatenate([L["wq"], L["wk"], L["wv"]], 0), weight)
        q = qkv[:, :qw].reshape(b, heads, hd)
        k = qkv[:, qw:qw + kvw].reshape(b, n_kv, hd)
        v = qkv[:, qw + kvw:].reshape(b, n_kv, hd)
        if geo.qk_norm:
            q = _rms(q, np.float64(L["q_norm"]) / np.sqrt(hd), geo.eps)
            k = _rms(k, L["k_norm"], geo.eps)
        q, k = _rope(q, pos, geo), _rope(k, pos, geo)
        if not geo.qk_norm:
            q = q / np.sqrt(hd)
        for i in range(b):
            kc[li][i, :, pos[i]] = k[i]
            vc[li][i, :, pos[i]] = v[i]
        att = np.empty((b, heads, hd))
        for i in range(b):
            hi = pos[i] + 1
            lo = hi - geo.window if geo.window and hi > geo.window else 0
            kk = kc[li][i, :, lo:hi].astype(np.float64)
            vv = vc[li][i, :, lo:hi].astype(np.float64)
            qg = q[i].reshape(n_kv, gqa, hd)
            sc = np.einsum("hgd,hnd->hgn", qg, kk)
            e = np.exp(sc - sc.max(-1, keepdims=True))
            att[i] = np.einsum("hgn,hnd->hgd", e / e.sum(-1, keepdims=True), vv).reshape(heads, hd)
        o = proj_kind_f64(att.reshape(b, qw), L["wo"], weight)
        if geo.layer_scale:
            o = o * L["attn_scale"]
        h = h + o
        a = _rms(h, L["ffn_norm"], geo.eps)
        g, u = proj_kind_f64(a, L["gate"], weight), proj_kind_f64(a, L["up"], weight)
        m = proj_kind_f64(g / (1.0 + np.exp(-g)) * u, L["down"], weight)
        if geo.layer_scale:
            m = m * L["mlp_scale"]
        h = h + m
    return _rms(h, final_norm, geo.eps), kc, vc


def stack_prefill_f64(geo, layers, final_norm, x, kc, vc, start):
    """Stack::forward's prefill branch (t >= 2, qwen3.rs:294-467) in float64 with the reference's
    f16 roundings: projection inputs and weights; projection outputs where Proj::Half takes the f16
    matmul (more than 48 rows, or rows not a multiple of 8); cache entries. The new positions'
    own k and v enter the attention unrounded. x [b, t, dim]; returns (out [b, t, dim], kc, vc)."""
    b, t, dim = x.shape
    rows = b * t
    hd, heads, n_kv = geo.head_dim, geo.heads, geo.n_kv
    qw, kvw, gqa = heads * hd, n_kv * hd, heads // n_kv
    kc = [k.copy() for k in kc]
    vc = [v.copy() for v in vc]
    pos = start + np.arange(t)

    def proj(a, w):
        y = _h(a) @ _h(w).T
        return y if _eligible(rows, a.shape[1], w.shape[0]) else _h(y)

    h = np.asarray(x, np.float64).reshape(rows, dim)
    n = start + t
    rr, cc = pos[:, None], np.arange(n)[None, :]
    lo = np.maximum(rr + 1 - geo.window, 0) if geo.window else np.zeros_like(rr)
    allowed = (cc <= rr) & (cc >= lo)                                                # [t, n]
    for li, L in enumerate(layers):
        qkv = proj(_rms(h, L["attn_norm"], geo.eps), np.concatenate([L["wq"], L["wk"], L["wv"]], 0))
        qkv = qkv.reshape(b, t, -1)
        q = qkv[..., :qw].reshape(b, t, heads, hd)
        k = qkv[..., qw:qw + kvw].reshape(b, t, n_kv, hd)
        v = qkv[..., qw + kvw:].reshape(b, t, n_kv, hd)
        if geo.qk_norm:
            q = _rms(q, np.float64(L["q_norm"]) / np.sqrt(hd), geo.eps)
            k = _rms(k, L["k_norm"], geo.eps)
        # rope over [b, t, heads, hd] at positions start + ti
        q = np.stack([_rope(q[:, ti], np.full(b, pos[ti]), geo) for ti in range(t)], 1)
        k = np.stack([_rope(k[:, ti], np.full(b, pos[ti]), geo) for ti in range(t)], 1)
        kc[li][:, :, start:n] = synth.f16_bits(k.transpose(0, 2, 1, 3))
        vc[li][:, :, start:n] = synth.f16_bits(v.transpose(0, 2, 1, 3))
        kk = np.concatenate([synth.from_f16_bits(kc[li][:, :, :start]).astype(np.float64),
                             k.transpose(0, 2, 1, 3)], 2)                              # [b, n_kv, n, hd]
        vv = np.concatenate([synth.from_f16_bits(vc[li][:, :, :start]).astype(np.float64),
                             v.transpose(0, 2, 1, 3)], 2)
        att = np.empty((b, t, heads, hd))
        for hh in range(heads):
            kh = hh // gqa
            s = np.einsum("btd,bnd->btn", q[:, :, hh], kk[:, kh])
            if not geo.qk_norm:
                s = s / np.sqrt(hd)
            s = np.where(allowed[None], s, -np.inf)
            e = np.exp(s - s.max(-1, keepdims=True))
            att[:, :, hh] = np.einsum("btn,bnd->btd", e / e.sum(-1, keepdims=True), vv[:, kh])
        o = proj(att.reshape(rows, qw), L["wo"])
        if geo.layer_scale:
            o = o * L["attn_scale"]
        h = h + o
        a = _rms(h, L["ffn_norm"], geo.eps)
        g, u = proj(a, L["gate"]), proj(a, L["up"])
        m = proj(g / (1.0 + np.exp(-g)) * u, L["down"])
        if geo.layer_scale:
            m = m * L["mlp_scale"]
        h = h + m
    return _rms(h, final_norm, geo.eps).reshape(b, t, dim), kc, vc
