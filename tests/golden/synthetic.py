"""The benchmark's synthetic tensors, by name, exactly as bench.py draws them (the seeded
counter-based generator of dream-tts_amd/dtts/synth.py: tag, shape and distribution fixed in
code), for their SHA-256 digests in synthetic_sha256.json. Each entry returns an ndarray; a
weight set returns a dict of them, hashed in sorted-key order."""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "dream-tts_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from dtts import codec, codec_front, synth  # noqa: E402


def _codec_weights():
    w = codec.random_weights(codec.CONFIG5, seed=0)
    out = {"head_w": w.head_w, "head_b": w.head_b, "out_a": w.out_act[0], "out_r": w.out_act[1],
           "out_w": w.out_w, "out_b": w.out_b}
    for i, b in enumerate(w.blocks):
        out[f"b{i}.act_a"], out[f"b{i}.act_r"] = b["act"]
        out[f"b{i}.up_w"], out[f"b{i}.up_b"] = b["up_w"], b["up_b"]
        for j, u in enumerate(b["units"]):
            for k in ("w1", "b1", "w2", "b2"):
                out[f"b{i}.u{j}.{k}"] = u[k]
            out[f"b{i}.u{j}.a1"], out[f"b{i}.u{j}.r1"] = u["act1"]
            out[f"b{i}.u{j}.a2"], out[f"b{i}.u{j}.r2"] = u["act2"]
    return out


def _front_weights():
    hw = codec_front.random_weights(codec_front.CODEC, 0)
    out = {k: getattr(hw, k) for k in ("codebooks", "out_proj_sem", "out_proj_ac", "pre_w", "pre_b", "in_w", "in_b",
                                       "tf_norm", "out_w", "out_b")}
    for i, L in enumerate(hw.layers):
        for k, v in L.items():
            out[f"l{i}.{k}"] = v
    for i, U in enumerate(hw.up):
        for k, v in U.items():
            out[f"up{i}.{k}"] = v
    return out


# name -> (generator, fast): `fast` entries are re-derived by the CPU test suite
ENTRIES = {
    "config5.latent": (lambda: synth.normal(0, "latent", (48, 250, 1024)), True),
    "config5.weights": (_codec_weights, True),
    "config1.x": (lambda: synth.normal(0, "cfg1.x", (1, 512, 4800)), True),
    "config1.alpha1": (lambda: synth.uniform(0, "cfg1.alpha1", (512,), 0.5, 1.5), True),
    "config1.alpha2": (lambda: synth.uniform(0, "cfg1.alpha2", (512,), 0.5, 1.5), True),
    "config1.w1": (lambda: synth.kaiming_normal(0, "cfg1.w1", (512, 512, 7), 512 * 7), True),
    "config1.w2": (lambda: synth.kaiming_normal(0, "cfg1.w2", (512, 512, 1), 512), True),
    "config1.b1": (lambda: synth.normal(0, "cfg1.b1", (512,), 0, 0.01), True),
    "config1.b2": (lambda: synth.normal(0, "cfg1.b2", (512,), 0, 0.01), True),
    "config2.h": (lambda: synth.normal(0, "cfg2.h", (48, 1, 1024)), True),
    "config2.gamma": (lambda: synth.uniform(0, "cfg2.gamma", (1024,), 0.9, 1.1), True),
    "config2.q": (lambda: synth.normal(0, "cfg2.q", (48, 16, 128)), True),
    "config2.k": (lambda: synth.normal(0, "cfg2.k", (48, 8, 128)), True),
    "config2.v": (lambda: synth.normal(0, "cfg2.v", (48, 8, 128)), True),
    "config2.pos": (lambda: synth.randint(0, "cfg2.pos", (48,), 0, 2047).astype(np.int32), True),
    "config2.kc": (lambda: synth.normal(0, "cfg2.kc", (48, 8, 2048, 128)), False),
    "config2.vc": (lambda: synth.normal(0, "cfg2.vc", (48, 8, 2048, 128)), False),
    "config4.w1024": (lambda: synth.normal(0, "cfg4.w1024", (6144, 1024), 0, 0.02), True),
    "config4.w3072": (lambda: synth.normal(0, "cfg4.w3072", (1024, 3072), 0, 0.02), True),
    "front.codes": (lambda: synth.randint(0, "front.codes", (48, 325, 16), 0, 2047).astype(np.int32), True),
    "front.doc": (lambda: synth.randint(0, "front.doc", (3000, 16), 0, 2047).astype(np.int32), True),
    "front.weights": (_front_weights, False),
}


def digest(value) -> str:
    h = hashlib.sha256()
    if isinstance(value, dict):
        for k in sorted(value):
            a = np.ascontiguousarray(value[k])
            h.update(k.encode())
            h.update(str(a.dtype).encode() + str(a.shape).encode())
            h.update(a.tobytes())
    else:
        a = np.ascontiguousarray(value)
        h.update(str(a.dtype).encode() + str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()
