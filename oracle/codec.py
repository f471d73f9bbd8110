"""CPU oracle of the codec waveform stack -- TEST INFRASTRUCTURE ONLY.

Restates Codec::forward's tail (drmhse/dream-tts crates/qwen3tts/src/codec.rs:426-436: head
conv, DecoderBlocks codec.rs:252-258 with TransConv codec.rs:153-158 and ResidualUnits
codec.rs:215-229, output SnakeBeta and conv) op by op, in two forms:

* ``decode_f16``: the f16 storage points the GPU stack keeps -- every activation stored in f16,
  every SnakeBeta and conv computed in f32 and rounded once (the parity oracle for the GPU decode).
* ``decode_f32_reference``: the reference's own CPU route in f32, one lane at a time: SnakeBeta
  passes, and every conv as pad + cat + GEMM + bias (crates/tts-nn/src/nlc.rs:102-131), the
  transposed conv through its tap-reversed polyphase weight (nlc.rs:158-183). This is what
  bench.py times as the CPU baseline.

The output conv ends in tanh (the benchmark's form of the stack); the reference clamps.
"""
from __future__ import annotations

import numpy as np

from . import (conv1d_nlc_cat_gemm_f32, conv1d_nlc_f16, snake_nlc_f16, snake_nlc_f32,
               tap_weight_f32, transpose_bias_f32, transpose_tap_weight_f32)


def _f16(a):
    return np.ascontiguousarray(np.asarray(a, np.float32).astype(np.float16).view(np.uint16))


def prepare(geo, w):
    """Tap-layout weights for both forms: f32 [k, cin, cout] and their f16 bit patterns."""
    def conv(wt, b):
        t = tap_weight_f32(wt)
        return dict(w32=t, b32=np.asarray(b, np.float32), w16=_f16(t), b16=_f16(b))

    p = dict(head=conv(w.head_w, w.head_b), blocks=[], out=conv(w.out_w, w.out_b), out_act=w.out_act)
    for i, blk in enumerate(w.blocks):
        r = geo.rates[i]
        t = transpose_tap_weight_f32(blk["up_w"], r)
        bb = transpose_bias_f32(blk["up_b"], r)
        up = dict(w32=t, b32=bb, w16=_f16(t), b16=_f16(bb))
        units = [dict(act1=u["act1"], act2=u["act2"], c1=conv(u["w1"], u["b1"]), c2=conv(u["w2"], u["b2"]))
                 for u in blk["units"]]
        p["blocks"].append(dict(act=blk["act"], up=up, units=units))
    return p


def decode_f16(geo, prep, latent_bits):
    """latent [lanes, frames, latent_dim] f16 bits -> audio [lanes, frames*hop] f16 bits."""
    x = conv1d_nlc_f16(latent_bits, prep["head"]["w16"], prep["head"]["b16"], 1)
    length = x.shape[1]
    lanes = x.shape[0]
    for i, blk in enumerate(prep["blocks"]):
        r, cout = geo.rates[i], geo.channels[i + 1]
        s = snake_nlc_f16(x, *blk["act"])
        u = conv1d_nlc_f16(s, blk["up"]["w16"], blk["up"]["b16"], 1)
        length *= r
        u = u.reshape(lanes, length, cout)
        for j, un in enumerate(blk["units"]):
            a = snake_nlc_f16(u, *un["act1"])
            h = conv1d_nlc_f16(a, un["c1"]["w16"], un["c1"]["b16"], geo.ru_dilations[j])
            h2 = snake_nlc_f16(h, *un["act2"])
            u = conv1d_nlc_f16(h2, un["c2"]["w16"], un["c2"]["b16"], 1, res_bits=u)
        x = u
    s = snake_nlc_f16(x, *prep["out_act"])
    # tanh (the benchmark's form) or Codec::forward's clamp to [-1, 1] (codec.rs:433-436)
    act = "clamp" if getattr(geo, "out_clamp", False) else "tanh"
    y = conv1d_nlc_f16(s, prep["out"]["w16"], prep["out"]["b16"], 1, act=act)
    return y.reshape(lanes, length)


def decode_f32_reference(geo, prep, latent):
    """One lane, f32: latent [frames, latent_dim] -> audio [frames*hop]."""
    x = conv1d_nlc_cat_gemm_f32(latent, prep["head"]["w32"], prep["head"]["b32"], 1)
    length = x.shape[0]
    for i, blk in enumerate(prep["blocks"]):
        r, cout = geo.rates[i], geo.channels[i + 1]
        s = snake_nlc_f32(x, *blk["act"])
        u = conv1d_nlc_cat_gemm_f32(s, blk["up"]["w32"], blk["up"]["b32"], 1)
        length *= r
        u = u.reshape(length, cout)
        for j, un in enumerate(blk["units"]):
            a = snake_nlc_f32(u, *un["act1"])
            h = conv1d_nlc_cat_gemm_f32(a, un["c1"]["w32"], un["c1"]["b32"], geo.ru_dilations[j])
            h2 = snake_nlc_f32(h, *un["act2"])
            u = u + conv1d_nlc_cat_gemm_f32(h2, un["c2"]["w32"], un["c2"]["b32"], 1)
        x = u
    s = snake_nlc_f32(x, *prep["out_act"])
    y = conv1d_nlc_cat_gemm_f32(s, prep["out"]["w32"], prep["out"]["b32"], 1)
    # tanh (the benchmark's form) or Codec::forward's clamp to [-1, 1] (codec.rs:433-436)
    if getattr(geo, "out_clamp", False):
        return np.clip(y.reshape(length), -1.0, 1.0)
    return np.tanh(y.reshape(length))
