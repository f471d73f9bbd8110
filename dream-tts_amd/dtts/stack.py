"""A Qwen3 decoder stack's decode step (dtts_stack_*) from Python: geometry presets, random-init
weights in the checkpoint's layouts, their device upload as Layer::load arranges them, per-layer
KV caches, and the step.

Mirrors crates/qwen3tts/src/qwen3.rs: Geometry (16-28), Layer::load (61-119: q|k|v rows
concatenated, q_norm pre-multiplied by 1/sqrt(head_dim)), State (128-212) and Stack::forward
(294-467) on its decode path (t = 1), with one position per lane.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import synth
from ._lib import call, lib, stream_handle

GRAPH = 1  # DTTS_STACK_GRAPH
# Stack::load's weight kinds (DTTS_WEIGHT_*): every kind but f16 keeps f32 caches
WEIGHTS = {"f16": 0, "f32": 1, "q8_0": 2, "q8_0_a32": 3}


def cache_dtype(weight: str):
    return torch.float16 if weight == "f16" else torch.float32


@dataclass(frozen=True)
class Geometry:
    dim: int
    layers: int
    heads: int
    n_kv: int
    head_dim: int
    ffn: int
    eps: float = 1e-6
    rope_base: float = 1_000_000.0
    qk_norm: bool = True
    layer_scale: bool = False
    window: int = 0  # 0: none
    capacity: int = 2048

    @property
    def gqa(self):
        return self.heads // self.n_kv

    @property
    def q_width(self):
        return self.heads * self.head_dim

    @property
    def kv_width(self):
        return self.n_kv * self.head_dim

    def weight_bytes_per_layer(self):
        """f16 projection bytes of one layer (what a decode step streams per layer)."""
        qkv = (self.q_width + 2 * self.kv_width) * self.dim
        return 2 * (qkv + self.dim * self.q_width + 2 * self.ffn * self.dim + self.dim * self.ffn)

    def flops_per_lane_layer(self):
        """Projection FLOPs (2*MACs) of one lane through one layer."""
        return self.weight_bytes_per_layer()  # 2 FLOP per f16 weight (2 bytes)


# crates/qwen3tts/src/cfg.rs:26-43 (talker; capacity talker.rs:75), 153-164 (code predictor; 17
# positions, talker.rs:291), 243-255 (codec transformer)
TALKER = Geometry(dim=2048, layers=28, heads=16, n_kv=8, head_dim=128, ffn=6144, capacity=1536)
PREDICTOR = Geometry(dim=1024, layers=5, heads=16, n_kv=8, head_dim=128, ffn=3072, capacity=17)
CODEC_TF = Geometry(dim=512, layers=8, heads=16, n_kv=16, head_dim=64, ffn=1024, eps=1e-5,
                    rope_base=10_000.0, qk_norm=False, layer_scale=True, window=72, capacity=1024)


def random_weights(geo: Geometry, seed: int = 0):
    """Checkpoint-layout f32 weights: projections [out, in] ~ N(0, 0.02), norm weights
    U(0.9, 1.1), LayerScale factors U(0.05, 0.15). Returns (layers, final_norm); each layer a dict
    with wq, wk, wv, wo, gate, up, down, attn_norm, ffn_norm, q_norm, k_norm, attn_scale,
    mlp_scale (the last four None when the geometry has no such weights)."""
    layers = []
    for i in range(geo.layers):
        p = f"stack.l{i}."

        def w(name, shape):
            return synth.normal(seed, p + name, shape, 0.0, 0.02)

        def u(name, n, lo=0.9, hi=1.1):
            return synth.uniform(seed, p + name, (n,), lo, hi)

        layers.append(dict(
            wq=w("wq", (geo.q_width, geo.dim)), wk=w("wk", (geo.kv_width, geo.dim)),
            wv=w("wv", (geo.kv_width, geo.dim)), wo=w("wo", (geo.dim, geo.q_width)),
            gate=w("gate", (geo.ffn, geo.dim)), up=w("up", (geo.ffn, geo.dim)),
            down=w("down", (geo.dim, geo.ffn)),
            attn_norm=u("attn_norm", geo.dim), ffn_norm=u("ffn_norm", geo.dim),
            q_norm=u("q_norm", geo.head_dim) if geo.qk_norm else None,
            k_norm=u("k_norm", geo.head_dim) if geo.qk_norm else None,
            attn_scale=u("attn_scale", geo.dim, 0.05, 0.15) if geo.layer_scale else None,
            mlp_scale=u("mlp_scale", geo.dim, 0.05, 0.15) if geo.layer_scale else None))
    return layers, synth.uniform(seed, "stack.norm", (geo.dim,), 0.9, 1.1)


def qk_norms(geo: Geometry, layer) -> np.ndarray:
    """[q_norm * 1/sqrt(head_dim); k_norm] in f32, as Layer::load folds the scale (qwen3.rs:78-91;
    candle's tensor * f64 is an f32 multiply by the f32-rounded factor)."""
    s = np.float32(1.0 / np.sqrt(np.float64(geo.head_dim)))
    return np.stack([layer["q_norm"].astype(np.float32) * s, layer["k_norm"].astype(np.float32)])


def qkv_rows(layer) -> np.ndarray:
    """Layer::load's fused [q; k; v] projection (qwen3.rs:69-77)."""
    return np.concatenate([layer["wq"], layer["wk"], layer["wv"]], axis=0)


# ---------------------------------------------------------------- ctypes mirrors of dtts.h

class _Geometry(ctypes.Structure):
    _fields_ = [("dim", ctypes.c_int64), ("layers", ctypes.c_int64), ("heads", ctypes.c_int64),
                ("n_kv", ctypes.c_int64), ("head_dim", ctypes.c_int64), ("ffn", ctypes.c_int64),
                ("eps", ctypes.c_float), ("rope_base", ctypes.c_double), ("qk_norm", ctypes.c_int32),
                ("layer_scale", ctypes.c_int32), ("window", ctypes.c_int64), ("capacity", ctypes.c_int64)]


class _Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("attn_norm", "ffn_norm", "wqkv", "wo", "w_gateup", "wdown",
                                               "qk_norms", "attn_scale", "mlp_scale")]


class _Cache(ctypes.Structure):
    _fields_ = [("k", ctypes.c_void_p), ("v", ctypes.c_void_p)]


def _f16_dev(a, dev):
    return torch.from_numpy(synth.f16_bits(a).view(np.int16).copy()).view(torch.float16).to(dev)


def _f32_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


class State:
    """Per-layer caches [lanes, n_kv, cap, head_dim] (State::new_state_with, qwen3.rs:245-268),
    zero-filled: f16, or f32 for a stack of another weight kind."""

    def __init__(self, geo: Geometry, lanes: int, cap: int, dev, dtype=torch.float16):
        shape = (lanes, geo.n_kv, cap, geo.head_dim)
        self.k = [torch.zeros(shape, dtype=dtype, device=dev) for _ in range(geo.layers)]
        self.v = [torch.zeros(shape, dtype=dtype, device=dev) for _ in range(geo.layers)]
        self.lanes, self.cap = lanes, cap
        self._c = (_Cache * geo.layers)()
        for i in range(geo.layers):
            self._c[i].k, self._c[i].v = self.k[i].data_ptr(), self.v[i].data_ptr()


def _q8_packed_dev(a, dev):
    """QTensor::quantize_onto of an [out, in] f32 weight (the library's host quantizer, GGML
    blocks), uploaded and repacked for the matrix cores (dtts_q8_0_repack)."""
    from . import ops

    a = np.ascontiguousarray(a, np.float32)
    blocks = torch.from_numpy(ops.q8_0_quantize(a)).to(dev)
    return ops.q8_0_repack(blocks, a.shape[1])


def upload(geo: Geometry, layers, final_norm, dev, weight: str = "f16"):
    """Host checkpoint-layout weights -> the device tensors dtts_stack_create takes, arranged as
    Layer::load arranges them: q|k|v rows concatenated, gate|up rows concatenated, q_norm folded
    with 1/sqrt(head_dim), projections of the weight kind (f16; f32; Q8_0 blocks, repacked),
    norms and scales in f32."""
    def f16(a):
        if weight == "f32":
            return _f32_dev(a, dev)
        if weight in ("q8_0", "q8_0_a32"):
            return _q8_packed_dev(a, dev)
        return _f16_dev(a, dev)

    def f32(a):
        return None if a is None else _f32_dev(a, dev)

    out = []
    for L in layers:
        out.append(dict(attn_norm=f32(L["attn_norm"]), ffn_norm=f32(L["ffn_norm"]), wqkv=f16(qkv_rows(L)),
                        wo=f16(L["wo"]), w_gateup=f16(np.concatenate([L["gate"], L["up"]], axis=0)),
                        wdown=f16(L["down"]), qk_norms=f32(qk_norms(geo, L)) if geo.qk_norm else None,
                        attn_scale=f32(L["attn_scale"]), mlp_scale=f32(L["mlp_scale"])))
    return out, f32(final_norm)


def random_device_weights(geo: Geometry, dev, seed: int = 0, weight: str = "f16"):
    """Device weights drawn with torch's generator on the device (for full-size benchmarks, where
    the host generator would take minutes): projections N(0, 0.02) of the weight kind (f16; f32;
    Q8_0 quantized on the device by dtts_convert_q8_0 and repacked), norms U(0.9, 1.1),
    LayerScale U(0.05, 0.15), in dtts_stack_create's layouts."""
    from . import ops
    from ._lib import ptr

    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def w(rows, cols):
        v = torch.randn((rows, cols), generator=g, device=dev) * 0.02
        if weight == "f32":
            return v
        if weight in ("q8_0", "q8_0_a32"):
            blocks = torch.empty(rows * cols // 32 * 34, dtype=torch.uint8, device=dev)
            call("dtts_convert_q8_0", ptr(v), 0, ptr(blocks), rows, cols, stream_handle(dev))  # 0: DTTS_DT_F32
            return ops.q8_0_repack(blocks.view(rows, cols // 32, 34), cols)
        return v.half()

    def u(n, lo=0.9, hi=1.1):
        return torch.rand((n,), generator=g, device=dev) * (hi - lo) + lo

    qkvw = geo.q_width + 2 * geo.kv_width
    out = []
    for _ in range(geo.layers):
        qk = None
        if geo.qk_norm:
            qk = torch.stack([u(geo.head_dim) * np.float32(1.0 / np.sqrt(geo.head_dim)), u(geo.head_dim)])
        out.append(dict(attn_norm=u(geo.dim), ffn_norm=u(geo.dim), wqkv=w(qkvw, geo.dim), wo=w(geo.dim, geo.q_width),
                        w_gateup=w(2 * geo.ffn, geo.dim), wdown=w(geo.dim, geo.ffn), qk_norms=qk,
                        attn_scale=u(geo.dim, 0.05, 0.15) if geo.layer_scale else None,
                        mlp_scale=u(geo.dim, 0.05, 0.15) if geo.layer_scale else None))
    return out, u(geo.dim)


def c_geometry(geo: Geometry) -> _Geometry:
    return _Geometry(geo.dim, geo.layers, geo.heads, geo.n_kv, geo.head_dim, geo.ffn, geo.eps, geo.rope_base,
                     int(geo.qk_norm), int(geo.layer_scale), geo.window, geo.capacity)


class Stack:
    """Device weights + a dtts_stack handle (keeps every device tensor alive)."""

    def __init__(self, geo: Geometry, layers, final_norm, dev, weight: str = "f16"):
        """layers / final_norm: host checkpoint-layout weights (random_weights' form), uploaded
        here; or device tensors already in the library's layouts (upload's or
        random_device_weights' form, recognised by final_norm being a torch tensor). weight:
        Stack::load's `how` (a WEIGHTS key)."""
        self.geo, self.dev, self.weight = geo, dev, weight
        if not isinstance(final_norm, torch.Tensor):
            layers, final_norm = upload(geo, layers, final_norm, dev, weight)
        self._keep = [final_norm]

        def ptr(t):
            if t is None:
                return None
            assert t.is_contiguous() and t.device.type == "cuda"
            self._keep.append(t)
            return t.data_ptr()

        g = c_geometry(geo)
        ls = (_Layer * geo.layers)()
        for i, L in enumerate(layers):
            for name, _ in _Layer._fields_:
                setattr(ls[i], name, ptr(L[name]))
        self._g, self._l = g, ls
        handle = ctypes.c_void_p()
        call("dtts_stack_create_as", ctypes.byref(g), ctypes.cast(ls, ctypes.c_void_p),
             ctypes.c_void_p(final_norm.data_ptr()), WEIGHTS[weight], ctypes.byref(handle))
        self.handle = handle
        self._ws = None

    @classmethod
    def from_handle(cls, geo: Geometry, handle, dev, owner):
        """A stack created elsewhere (dtts_stack_model_load); `owner` keeps it alive and destroys it."""
        s = cls.__new__(cls)
        s.geo, s.dev, s.handle, s._keep, s._ws, s._owner = geo, dev, handle, [], None, owner
        s.weight = "f16"
        return s

    def close(self):
        if self.handle and getattr(self, "_owner", None) is None:
            lib().dtts_stack_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def weight_bytes(self):
        return sum(t.numel() * t.element_size() for t in self._keep)

    def new_state(self, lanes: int, cap: int | None = None) -> State:
        return State(self.geo, lanes, cap or self.geo.capacity, self.dev, cache_dtype(self.weight))

    def workspace_bytes(self, lanes: int, cap: int) -> int:
        return int(lib().dtts_stack_workspace_bytes(self.handle, lanes, cap))

    def workspace(self, lanes, cap):
        need = self.workspace_bytes(lanes, cap)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.dev)
        return self._ws

    def decode(self, x: torch.Tensor, state: State, pos, out: torch.Tensor | None = None,
               graph: bool = False, workspace: torch.Tensor | None = None) -> torch.Tensor:
        """x [lanes, dim] f32 -> the normed hidden state [lanes, dim] f32; each lane's k and v land
        in its cache at pos[lane]."""
        lanes = x.shape[0]
        assert x.dtype == torch.float32 and x.is_contiguous() and x.shape[1] == self.geo.dim
        if out is None:
            out = torch.empty_like(x)
        p = np.ascontiguousarray(np.broadcast_to(np.asarray(pos, np.int32), (lanes,)))
        ws = workspace if workspace is not None else self.workspace(lanes, state.cap)
        call("dtts_stack_decode", self.handle, ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
             ctypes.cast(state._c, ctypes.c_void_p), lanes, state.cap, p.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(ws.data_ptr()),
             ws.numel(), GRAPH if graph else 0, stream_handle(self.dev))
        return out

    def prefill_workspace_bytes(self, lanes: int, t: int) -> int:
        return int(lib().dtts_stack_prefill_workspace_bytes(self.handle, lanes, t))

    def prefill(self, x: torch.Tensor, state: State, start: int, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None) -> torch.Tensor:
        """Stack::forward at t >= 2 (the prefill branch) for lanes sharing `start`: x [lanes, t, dim]
        f32 -> the normed hidden states [lanes, t, dim] f32; the new positions' k and v land in the
        caches at start .. start + t - 1."""
        lanes, t, dim = x.shape
        assert x.dtype == torch.float32 and x.is_contiguous() and dim == self.geo.dim
        if out is None:
            out = torch.empty_like(x)
        if workspace is None:
            workspace = torch.empty(max(self.prefill_workspace_bytes(lanes, t), 256), dtype=torch.uint8,
                                    device=self.dev)
        call("dtts_stack_prefill", self.handle, ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
             ctypes.cast(state._c, ctypes.c_void_p), lanes, t, start, state.cap, ctypes.c_void_p(workspace.data_ptr()),
             workspace.numel(), stream_handle(self.dev))
        return out
