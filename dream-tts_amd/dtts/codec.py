"""The codec waveform stack (dtts_codec_*) from Python: geometry, random-init weights in the
checkpoint's own layouts, their device upload in the kernels' layouts, and decode.

Weights are drawn with the seeded generator in torch's parameter layouts (conv [out, in, k],
ConvTranspose [in, out, k]), exactly as a checkpoint would hold them; `to_device` applies the
same host-side rearrangements a loader does (crates/qwen3tts/src/codec.rs:99-151).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np
import torch

from . import nlc, synth
from ._lib import DttsError, call, lib, stream_handle

MAX_BLOCKS = 8


@dataclass
class Geometry:
    latent_dim: int = 1024
    head_kernel: int = 7
    channels: tuple = (1536, 768, 384, 192, 96)
    rates: tuple = (8, 5, 4, 3)
    ru_kernel: int = 7
    ru_dilations: tuple = (1, 3, 9)
    out_kernel: int = 7
    out_clamp: bool = False  # True: Codec::forward's clamp to [-1, 1]; False: tanh (config 5's form)

    @property
    def n_blocks(self):
        return len(self.rates)

    @property
    def hop(self):
        return int(np.prod(self.rates))

    def flops_per_frame(self):
        """Algorithmic FLOPs (2*MACs) of one latent frame through the stack, one lane."""
        g, f, length = self, 0, 1
        f += 2 * g.latent_dim * g.channels[0] * g.head_kernel
        for i, r in enumerate(g.rates):
            cin, cout = g.channels[i], g.channels[i + 1]
            f += 2 * cin * (r * cout) * 2 * length  # TransConv: 2 taps, r phases
            length *= r
            f += 3 * (2 * cout * cout * g.ru_kernel + 2 * cout * cout) * length
        f += 2 * g.channels[-1] * g.out_kernel * length
        return f


# config 5 of the benchmark: 48 lanes x 250 frames through this geometry
CONFIG5 = Geometry()


@dataclass
class HostWeights:
    """numpy f32 tensors in checkpoint layouts (SnakeBeta already folded to alpha, 1/beta)."""
    head_w: np.ndarray
    head_b: np.ndarray
    blocks: list = field(default_factory=list)  # dicts: act (a, r), up_w [in,out,2r], up_b, units
    out_act: tuple = None
    out_w: np.ndarray = None
    out_b: np.ndarray = None


def random_weights(geo: Geometry, seed: int = 0, gain: float = 1.0) -> HostWeights:
    """Kaiming-normal conv weights (std gain/sqrt(fan_in), torch's fan_in = dim1 * k), biases
    N(0, 0.01), SnakeBeta alpha ~ U(0.5, 1.5) with brecip = 1/alpha.

    gain defaults to 1 (nonlinearity='linear'): with the ReLU gain sqrt(2) every conv doubles
    the residual stream's second moment and the last block's activations pass f16's 65504
    within a few frames; with gain 1 the stack peaks near 100 and stays finite in f16."""
    def act(tag, c):
        a = synth.uniform(seed, tag + ".alpha", (c,), 0.5, 1.5)
        return a, (1.0 / a.astype(np.float64)).astype(np.float32)

    def conv(tag, cout, cin, k):
        return (synth.kaiming_normal(seed, tag + ".w", (cout, cin, k), cin * k, gain),
                synth.normal(seed, tag + ".b", (cout,), 0.0, 0.01))

    hw, hb = conv("head", geo.channels[0], geo.latent_dim, geo.head_kernel)
    w = HostWeights(head_w=hw, head_b=hb)
    for i, r in enumerate(geo.rates):
        cin, cout = geo.channels[i], geo.channels[i + 1]
        p = f"block{i}"
        up_w = synth.kaiming_normal(seed, p + ".up.w", (cin, cout, 2 * r), cout * 2 * r, gain)
        up_b = synth.normal(seed, p + ".up.b", (cout,), 0.0, 0.01)
        units = []
        for j, d in enumerate(geo.ru_dilations):
            q = f"{p}.unit{j}"
            w1, b1 = conv(q + ".conv1", cout, cout, geo.ru_kernel)
            w2, b2 = conv(q + ".conv2", cout, cout, 1)
            units.append(dict(act1=act(q + ".act1", cout), w1=w1, b1=b1, act2=act(q + ".act2", cout),
                              w2=w2, b2=b2))
        w.blocks.append(dict(act=act(p + ".act", cin), up_w=up_w, up_b=up_b, units=units))
    w.out_act = act("out.act", geo.channels[-1])
    w.out_w, w.out_b = conv("out", 1, geo.channels[-1], geo.out_kernel)
    return w


# ---------------------------------------------------------------- ctypes mirrors of dtts.h

class _Geometry(ctypes.Structure):
    _fields_ = [("latent_dim", ctypes.c_int64), ("head_kernel", ctypes.c_int64),
                ("n_blocks", ctypes.c_int64), ("channels", ctypes.c_int64 * (MAX_BLOCKS + 1)),
                ("rates", ctypes.c_int64 * MAX_BLOCKS), ("ru_kernel", ctypes.c_int64),
                ("ru_dilations", ctypes.c_int64 * 3), ("out_kernel", ctypes.c_int64),
                ("out_clamp", ctypes.c_int64)]


class _Unit(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("act1_alpha", "act1_brecip", "conv1_w", "conv1_b",
                                               "act2_alpha", "act2_brecip", "conv2_w", "conv2_b")]


class _Block(ctypes.Structure):
    _fields_ = [("act_alpha", ctypes.c_void_p), ("act_brecip", ctypes.c_void_p),
                ("up_w", ctypes.c_void_p), ("up_b", ctypes.c_void_p), ("units", _Unit * 3)]


class _Stage(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 32), ("kernel", ctypes.c_char * 96),
                ("lanes", ctypes.c_int64), ("len", ctypes.c_int64), ("cin", ctypes.c_int64),
                ("cout", ctypes.c_int64), ("k", ctypes.c_int64), ("dilation", ctypes.c_int64),
                ("flops", ctypes.c_double), ("bytes", ctypes.c_double), ("ms", ctypes.c_float)]


class _Weights(ctypes.Structure):
    _fields_ = [("head_w", ctypes.c_void_p), ("head_b", ctypes.c_void_p),
                ("blocks", _Block * MAX_BLOCKS), ("out_alpha", ctypes.c_void_p),
                ("out_brecip", ctypes.c_void_p), ("out_w", ctypes.c_void_p), ("out_b", ctypes.c_void_p)]


def _f16_dev(a, dev):
    bits = synth.f16_bits(a)
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.float16).to(dev)


def _f32_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def c_geometry(geo: Geometry) -> _Geometry:
    g = _Geometry()
    g.latent_dim, g.head_kernel, g.n_blocks = geo.latent_dim, geo.head_kernel, geo.n_blocks
    for i, c in enumerate(geo.channels):
        g.channels[i] = c
    for i, r in enumerate(geo.rates):
        g.rates[i] = r
    g.ru_kernel, g.out_kernel = geo.ru_kernel, geo.out_kernel
    g.out_clamp = int(geo.out_clamp)
    for j, d in enumerate(geo.ru_dilations):
        g.ru_dilations[j] = d
    return g


class Codec:
    """Device weights + a dtts_codec handle. Keeps every device tensor alive.

    dtype "f16" (the default): f16 storage with f32 arithmetic, the benchmark's form. "f32": every
    tensor f32, the reference's own precision for its waveform stack (WAV_DTYPE = F32,
    crates/qwen3tts/src/codec.rs:33-43), through dtts_codec_create_f32 / dtts_codec_decode_f32."""

    def __init__(self, geo: Geometry, w: HostWeights, dev, dtype: str = "f16"):
        if dtype not in ("f16", "f32"):
            raise DttsError(f"codec: dtype {dtype!r} is not f16 or f32")
        self.geo = geo
        self.dtype = dtype
        self.torch_dtype = torch.float16 if dtype == "f16" else torch.float32
        self._keep = []

        def cw(a):  # conv weights and biases, in the codec's element type
            t = _f16_dev(a, dev) if dtype == "f16" else _f32_dev(a, dev)
            self._keep.append(t)
            return ctypes.c_void_p(t.data_ptr())

        def f32(a):
            t = _f32_dev(a, dev)
            self._keep.append(t)
            return ctypes.c_void_p(t.data_ptr())

        g = c_geometry(geo)
        ws = _Weights()
        ws.head_w = cw(nlc.tap_major_weight(w.head_w))
        ws.head_b = cw(w.head_b)
        for i, blk in enumerate(w.blocks):
            b = ws.blocks[i]
            b.act_alpha, b.act_brecip = f32(blk["act"][0]), f32(blk["act"][1])
            r = geo.rates[i]
            b.up_w = cw(nlc.transpose_tap_major_weight(blk["up_w"], r))
            b.up_b = cw(nlc.transpose_bias(blk["up_b"], r))
            for j, un in enumerate(blk["units"]):
                u = b.units[j]
                u.act1_alpha, u.act1_brecip = f32(un["act1"][0]), f32(un["act1"][1])
                u.conv1_w, u.conv1_b = cw(nlc.tap_major_weight(un["w1"])), cw(un["b1"])
                u.act2_alpha, u.act2_brecip = f32(un["act2"][0]), f32(un["act2"][1])
                u.conv2_w, u.conv2_b = cw(nlc.tap_major_weight(un["w2"])), cw(un["b2"])
        ws.out_alpha, ws.out_brecip = f32(w.out_act[0]), f32(w.out_act[1])
        ws.out_w, ws.out_b = cw(nlc.tap_major_weight(w.out_w)), cw(w.out_b)
        self._geo_c, self._w_c = g, ws
        handle = ctypes.c_void_p()
        call("dtts_codec_create" if dtype == "f16" else "dtts_codec_create_f32", ctypes.byref(g), ctypes.byref(ws),
             ctypes.byref(handle))
        self.handle = handle
        self.dev = dev
        self._ws = None

    def weight_bytes(self):
        return sum(t.numel() * t.element_size() for t in self._keep)

    def workspace(self, lanes, frames):
        need = int(lib().dtts_codec_workspace_bytes(self.handle, lanes, frames))
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.dev)
        return self._ws, need

    def decode(self, latent, out=None):
        """latent [lanes, frames, latent_dim] (device, the codec's dtype) -> audio [lanes, frames*hop]."""
        if latent.dtype != self.torch_dtype or not latent.is_contiguous() or latent.dim() != 3:
            raise DttsError(f"codec.decode: latent must be a contiguous {self.dtype} [lanes, frames, dim]")
        lanes, frames, _ = latent.shape
        audio = out if out is not None else torch.empty((lanes, frames * self.geo.hop),
                                                        dtype=self.torch_dtype, device=latent.device)
        ws, need = self.workspace(lanes, frames)
        call("dtts_codec_decode" if self.dtype == "f16" else "dtts_codec_decode_f32", self.handle,
             ctypes.c_void_p(latent.data_ptr()),
             ctypes.c_void_p(audio.data_ptr()), lanes, frames, ctypes.c_void_p(ws.data_ptr()),
             ctypes.c_size_t(need), stream_handle())
        return audio

    def profile(self, latent, out=None):
        """One decode with a HIP event around every launch: a list of per-launch dicts (name,
        kernel, shape, algorithmic flops/bytes, ms). Synchronises the stream."""
        lanes, frames, _ = latent.shape
        audio = out if out is not None else torch.empty((lanes, frames * self.geo.hop),
                                                        dtype=self.torch_dtype, device=latent.device)
        ws, need = self.workspace(lanes, frames)
        table = (_Stage * 128)()
        n = ctypes.c_int(0)
        call("dtts_codec_profile", self.handle, ctypes.c_void_p(latent.data_ptr()),
             ctypes.c_void_p(audio.data_ptr()), lanes, frames, ctypes.c_void_p(ws.data_ptr()),
             ctypes.c_size_t(need), stream_handle(), table, 128, ctypes.byref(n))
        return [dict(name=t.name.decode(), kernel=t.kernel.decode(), lanes=t.lanes, len=t.len,
                     cin=t.cin, cout=t.cout, k=t.k, dilation=t.dilation, flops=t.flops,
                     bytes=t.bytes, ms=t.ms) for t in table[: n.value]]

    def close(self):
        if self.handle:
            lib().dtts_codec_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
