"""A codec checkpoint in the reference's tensor naming (crates/qwen3tts/src/codec.rs:262-399:
"decoder.quantizer.rvq_first.*", "decoder.pre_conv.*", "decoder.pre_transformer.*",
"decoder.upsample.<i>.*", "decoder.decoder.<i>.*"), written with the safetensors package from
seeded random parameters, together with the host weights those parameters fold to -- the inputs
of the Python-built models a loaded model is compared against.

SnakeBeta is stored as logs and folded as alpha = exp(a), brecip = 1 / (exp(b) + 1e-9)
(codec.rs:60-68), each exp rounded once to f32 from float64; the codebooks as embedding_sum and
cluster_usage, folded as sum / max(usage, 1e-5) in f32 (codec.rs:275-282). Extra tensors the
decoder does not read (the RVQ input projections, an encoder weight) are included so the loader is
seen to ignore them."""
from __future__ import annotations

from dataclasses import replace

import numpy as np

from dtts import codec, codec_front, synth

from _doc_ref import TINY, TINY_WAVE  # noqa: F401


def _round(a, dtype):
    a = np.asarray(a, np.float32)
    if dtype == "BF16":
        import torch
        return torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    if dtype == "F16":
        return a.astype(np.float16).astype(np.float32)
    return a


def _snake_fold(alog, blog):
    alpha = np.exp(alog.astype(np.float64)).astype(np.float32)
    eb = np.exp(blog.astype(np.float64)).astype(np.float32)
    return alpha, (np.float32(1.0) / (eb + np.float32(1e-9))).astype(np.float32)


def build(fg, wg, seed=0, dtype="F32"):
    """-> (tensors: name -> f32 array already rounded to `dtype`, front HostWeights, wave HostWeights)."""
    T = {}

    def put(name, a):
        T[name] = _round(a, dtype)
        return T[name]

    def w(tag, shape, fan_in):
        return synth.normal(seed, "ck." + tag, shape, 0.0, float(1.0 / np.sqrt(fan_in)))

    def b(tag, n):
        return synth.normal(seed, "ck." + tag, (n,), 0.0, 0.01)

    def u(tag, n, lo=0.9, hi=1.1):
        return synth.uniform(seed, "ck." + tag, (n,), lo, hi)

    def logs(tag, n):
        return (synth.uniform(seed, "ck." + tag + ".a", (n,), np.log(0.5), np.log(1.5)),
                synth.uniform(seed, "ck." + tag + ".b", (n,), np.log(0.5), np.log(1.5)))

    # ---- front half
    fw = codec_front.HostWeights()
    q = "decoder.quantizer."
    books = []
    for i in range(fg.n_books):
        first = i < fg.n_first
        p = f"{q}{'rvq_first' if first else 'rvq_rest'}.vq.layers.{i if first else i - fg.n_first}._codebook."
        s = put(p + "embedding_sum", synth.normal(seed, f"ck.book{i}.sum", (fg.book_size, fg.book_dim)))
        us = put(p + "cluster_usage", synth.uniform(seed, f"ck.book{i}.usage", (fg.book_size,), 0.5, 2.0))
        books.append(codec_front.fold_codebook(s, us))
    fw.codebooks = np.stack(books)
    fw.out_proj_sem = put(q + "rvq_first.output_proj.weight", w("osem", (fg.codebook_dim, fg.book_dim, 1), fg.book_dim))
    fw.out_proj_ac = put(q + "rvq_rest.output_proj.weight", w("oac", (fg.codebook_dim, fg.book_dim, 1), fg.book_dim))
    put(q + "rvq_first.input_proj.weight", w("isem", (fg.book_dim, fg.codebook_dim, 1), fg.codebook_dim))
    put(q + "rvq_rest.input_proj.weight", w("iac", (fg.book_dim, fg.codebook_dim, 1), fg.codebook_dim))
    put("encoder.conv.weight", w("enc", (8, 1, 7), 7))
    fw.pre_w = put("decoder.pre_conv.conv.weight",
                   w("pre", (fg.latent_dim, fg.codebook_dim, fg.pre_kernel), fg.codebook_dim * fg.pre_kernel))
    fw.pre_b = put("decoder.pre_conv.conv.bias", b("preb", fg.latent_dim))
    t = "decoder.pre_transformer."
    fw.in_w = put(t + "input_proj.weight", w("in", (fg.tf_dim, fg.latent_dim), fg.latent_dim))
    fw.in_b = put(t + "input_proj.bias", b("inb", fg.tf_dim))
    qw, kvw, d = fg.tf_heads * fg.tf_head_dim, fg.tf_n_kv * fg.tf_head_dim, fg.tf_dim
    for i in range(fg.tf_layers):
        p = f"{t}layers.{i}."
        L = dict(attn_norm=put(p + "input_layernorm.weight", u(f"l{i}.an", d)),
                 ffn_norm=put(p + "post_attention_layernorm.weight", u(f"l{i}.fn", d)),
                 attn_scale=put(p + "self_attn_layer_scale.scale", u(f"l{i}.as", d, 0.05, 0.15)),
                 mlp_scale=put(p + "mlp_layer_scale.scale", u(f"l{i}.ms", d, 0.05, 0.15)),
                 wq=put(p + "self_attn.q_proj.weight", w(f"l{i}.q", (qw, d), d)),
                 wk=put(p + "self_attn.k_proj.weight", w(f"l{i}.k", (kvw, d), d)),
                 wv=put(p + "self_attn.v_proj.weight", w(f"l{i}.v", (kvw, d), d)),
                 wo=put(p + "self_attn.o_proj.weight", w(f"l{i}.o", (d, qw), qw)),
                 gate=put(p + "mlp.gate_proj.weight", w(f"l{i}.g", (fg.tf_ffn, d), d)),
                 up=put(p + "mlp.up_proj.weight", w(f"l{i}.u", (fg.tf_ffn, d), d)),
                 down=put(p + "mlp.down_proj.weight", w(f"l{i}.d", (d, fg.tf_ffn), fg.tf_ffn)))
        fw.layers.append(L)
    fw.tf_norm = put(t + "norm.weight", u("tfn", d))
    fw.out_w = put(t + "output_proj.weight", w("out", (fg.latent_dim, d), d))
    fw.out_b = put(t + "output_proj.bias", b("outb", fg.latent_dim))
    c = fg.latent_dim
    for i, r in enumerate(fg.up_ratios):
        p = f"decoder.upsample.{i}."
        fw.up.append(dict(
            up_w=put(p + "0.conv.weight", w(f"up{i}", (c, c, r), c)), up_b=put(p + "0.conv.bias", b(f"up{i}b", c)),
            dw_w=put(p + "1.dwconv.conv.weight", w(f"dw{i}", (c, 1, fg.dw_kernel), fg.dw_kernel)),
            dw_b=put(p + "1.dwconv.conv.bias", b(f"dw{i}b", c)),
            ln_w=put(p + "1.norm.weight", u(f"ln{i}", c)), ln_b=put(p + "1.norm.bias", b(f"ln{i}b", c)),
            pw1_w=put(p + "1.pwconv1.weight", w(f"pw1{i}", (4 * c, c), c)), pw1_b=put(p + "1.pwconv1.bias", b(f"pw1{i}b", 4 * c)),
            pw2_w=put(p + "1.pwconv2.weight", w(f"pw2{i}", (c, 4 * c), 4 * c)), pw2_b=put(p + "1.pwconv2.bias", b(f"pw2{i}b", c)),
            gamma=put(p + "1.gamma", u(f"g{i}", c, 0.05, 0.15))))
    # ---- waveform stack
    dd = "decoder.decoder."
    ww = codec.HostWeights(head_w=put(dd + "0.conv.weight", w("head", (wg.channels[0], wg.latent_dim, wg.head_kernel),
                                                             wg.latent_dim * wg.head_kernel)),
                           head_b=put(dd + "0.conv.bias", b("headb", wg.channels[0])))

    def snake(prefix, n):
        a, bb = logs(prefix, n)
        return _snake_fold(put(prefix + ".alpha", a), put(prefix + ".beta", bb))

    for i, rate in enumerate(wg.rates):
        cin, co = wg.channels[i], wg.channels[i + 1]
        p = f"{dd}{i + 1}.block."
        blk = dict(act=snake(p + "0", cin),
                   up_w=put(p + "1.conv.weight", w(f"b{i}.up", (cin, co, 2 * rate), co * 2 * rate)),
                   up_b=put(p + "1.conv.bias", b(f"b{i}.upb", co)), units=[])
        for j in range(3):
            pu = f"{p}{j + 2}."
            un = dict(act1=snake(pu + "act1", co),
                      w1=put(pu + "conv1.conv.weight", w(f"b{i}u{j}.1", (co, co, wg.ru_kernel), co * wg.ru_kernel)),
                      b1=put(pu + "conv1.conv.bias", b(f"b{i}u{j}.1b", co)),
                      act2=snake(pu + "act2", co),
                      w2=put(pu + "conv2.conv.weight", w(f"b{i}u{j}.2", (co, co, 1), co)),
                      b2=put(pu + "conv2.conv.bias", b(f"b{i}u{j}.2b", co)))
            blk["units"].append(un)
        ww.blocks.append(blk)
    n = len(wg.rates)
    ww.out_act = snake(f"{dd}{n + 1}", wg.channels[-1])
    ww.out_w = put(f"{dd}{n + 2}.conv.weight", 0.05 * w("outc", (1, wg.channels[-1], wg.out_kernel),
                                                         wg.channels[-1] * wg.out_kernel))
    ww.out_b = put(f"{dd}{n + 2}.conv.bias", b("outcb", 1))
    return T, fw, ww


def write(path, tensors, dtype="F32"):
    """The tensors in `dtype` (F32, F16 or BF16), with a metadata entry, as a safetensors file."""
    if dtype == "BF16":
        import torch
        from safetensors.torch import save_file
        save_file({k: torch.from_numpy(np.ascontiguousarray(v)).to(torch.bfloat16) for k, v in tensors.items()},
                  str(path), metadata={"format": "pt"})
    else:
        from safetensors.numpy import save_file
        np_dtype = np.float16 if dtype == "F16" else np.float32
        save_file({k: np.ascontiguousarray(v, np_dtype) for k, v in tensors.items()}, str(path),
                  metadata={"format": "np"})


TINY_CKPT_FRONT = replace(TINY, max_frames=64)


def stack_tensors(geo, layers, final_norm, prefix):
    """A decoder stack's checkpoint-layout weights (stack.random_weights' form) under Layer::load's
    names (crates/qwen3tts/src/qwen3.rs:61-119) and Stack::load's final norm."""
    T = {}
    for i, L in enumerate(layers):
        p = f"{prefix}layers.{i}."
        T[p + "input_layernorm.weight"] = L["attn_norm"]
        T[p + "post_attention_layernorm.weight"] = L["ffn_norm"]
        for n, k in (("q", "wq"), ("k", "wk"), ("v", "wv"), ("o", "wo")):
            T[p + f"self_attn.{n}_proj.weight"] = L[k]
        for n in ("gate", "up", "down"):
            T[p + f"mlp.{n}_proj.weight"] = L[n]
        if geo.qk_norm:
            T[p + "self_attn.q_norm.weight"] = L["q_norm"]
            T[p + "self_attn.k_norm.weight"] = L["k_norm"]
        if geo.layer_scale:
            T[p + "self_attn_layer_scale.scale"] = L["attn_scale"]
            T[p + "mlp_layer_scale.scale"] = L["mlp_scale"]
    T[prefix + "norm.weight"] = final_norm
    return T
