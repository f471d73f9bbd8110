"""An independent float64 restatement of the codec's front half (Codec::forward up to the waveform
stack, crates/qwen3tts/src/codec.rs:401-424) in numpy, from the checkpoint-layout weights, with
f16 rounding at the same storage points the oracle and the GPU keep. Used to pin the oracle's
chain (oracle/codec_front.py) at small geometries."""
from dataclasses import replace

import numpy as np

from dtts import codec_front

TINY = replace(codec_front.CODEC, n_books=4, book_size=40, book_dim=16, codebook_dim=32, latent_dim=64,
               tf_dim=64, tf_layers=2, tf_heads=4, tf_n_kv=2, tf_head_dim=64, tf_ffn=128, tf_window=5,
               up_ratios=(2, 3), max_frames=64)


def _h(a):
    return np.asarray(a, np.float64).astype(np.float16).astype(np.float64)


def _conv_causal(x, w_oik, b):
    """x [lanes, L, cin]; w [cout, cin, k] (torch layout): causal conv, zero left padding."""
    lanes, length, cin = x.shape
    cout, _, k = w_oik.shape
    xp = np.concatenate([np.zeros((lanes, k - 1, cin)), x], 1)
    y = np.zeros((lanes, length, cout))
    for t in range(k):
        y += xp[:, t:t + length] @ w_oik[:, :, t].T.astype(np.float64)
    return y + (0 if b is None else b)


def _rope(x, pos, base):
    d = x.shape[-1]
    i = np.arange(d // 2)
    ph = pos[:, None] * (1.0 / base ** (2.0 * i / d))
    c, s = np.cos(ph), np.sin(ph)
    x1, x2 = x[..., :d // 2], x[..., d // 2:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)


def _rms(x, g, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * g


def front_f64(geo, hw, codes):
    codes = np.asarray(codes)
    lanes, frames, nb = codes.shape
    books = hw.codebooks.astype(np.float64)
    pick = np.stack([books[b][codes[:, :, b]] for b in range(nb)], 2)  # [lanes, T, nb, dim]
    sem = _h(pick[:, :, :geo.n_first].sum(2))
    ac = _h(pick[:, :, geo.n_first:].sum(2))
    q = _h(sem @ hw.out_proj_sem[:, :, 0].T + ac @ hw.out_proj_ac[:, :, 0].T)
    h = _h(_conv_causal(q, _h(hw.pre_w), _h(hw.pre_b)))
    h = _h(h @ _h(hw.in_w).T + _h(hw.in_b))
    hd, heads, n_kv = geo.tf_head_dim, geo.tf_heads, geo.tf_n_kv
    pos = np.arange(frames, dtype=np.float64)
    for L in hw.layers:
        a = _h(_rms(h, L["attn_norm"], geo.tf_eps))
        qq = _h(a @ _h(L["wq"]).T).reshape(lanes, frames, heads, hd)
        kk = _h(a @ _h(L["wk"]).T).reshape(lanes, frames, n_kv, hd)
        vv = _h(a @ _h(L["wv"]).T).reshape(lanes, frames, n_kv, hd)
        att = np.zeros((lanes, frames, heads, hd))
        for hh in range(heads):
            kh = hh // (heads // n_kv)
            qr = _rope(qq[:, :, hh], pos, geo.tf_rope_base)
            kr = _rope(kk[:, :, kh], pos, geo.tf_rope_base)
            s = np.einsum("bid,bjd->bij", qr, kr) / np.sqrt(hd)
            i, j = np.meshgrid(np.arange(frames), np.arange(frames), indexing="ij")
            s = np.where((j <= i) & (j > i - geo.tf_window), s, -np.inf)
            e = np.exp(s - s.max(-1, keepdims=True))
            att[:, :, hh] = np.einsum("bij,bjd->bid", e / e.sum(-1, keepdims=True), vv[:, :, kh])
        att = _h(att.reshape(lanes, frames, heads * hd))
        h = _h(h + (att @ _h(L["wo"]).T) * L["attn_scale"])
        a = _h(_rms(h, L["ffn_norm"], geo.tf_eps))
        g, u = _h(a @ _h(L["gate"]).T), _h(a @ _h(L["up"]).T)
        t = _h(g / (1 + np.exp(-g)) * u)
        h = _h(h + (t @ _h(L["down"]).T) * L["mlp_scale"])
    a = _h(_rms(h, hw.tf_norm, geo.tf_eps))
    x = _h(a @ _h(hw.out_w).T + _h(hw.out_b))
    from math import erf
    verf = np.vectorize(erf)
    for i, U in enumerate(hw.up):
        r = geo.up_ratios[i]
        lanes_, length, c = x.shape
        # ConvTranspose1d with kernel = stride: output l*r + p = x[l] . W[:, :, p] + b
        u = np.einsum("blc,cop->blpo", x, _h(U["up_w"])) + _h(U["up_b"])
        u = _h(u.reshape(lanes_, length * r, c))
        d = _conv_depthwise(u, U["dw_w"][:, 0, :]) + U["dw_b"]
        m = d.mean(-1, keepdims=True)
        v = ((d - m) ** 2).mean(-1, keepdims=True)
        dn = _h((d - m) / np.sqrt(v + geo.ln_eps) * U["ln_w"] + U["ln_b"])
        p = dn @ _h(U["pw1_w"]).T + _h(U["pw1_b"])
        p = _h(0.5 * p * (1 + verf(p / np.sqrt(2))))
        x = _h(u + (p @ _h(U["pw2_w"]).T + _h(U["pw2_b"])) * U["gamma"])
    return x


def _conv_depthwise(x, taps):
    lanes, length, c = x.shape
    k = taps.shape[1]
    xp = np.concatenate([np.zeros((lanes, k - 1, c)), x], 1)
    return sum(xp[:, t:t + length] * taps[:, t] for t in range(k))
