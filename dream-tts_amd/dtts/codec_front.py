"""The codec's front half (dtts_codec_front_*) from Python: geometry, random-init weights in the
checkpoint's own layouts, their upload in the kernels' layouts, and decode.

Mirrors crates/qwen3tts/src/codec.rs: Rvq::load / decode (263-317; codebooks folded as
embedding_sum / clamp(cluster_usage, 1e-5)), Codec::load's front modules (337-399) and
Codec::forward up to the waveform stack (401-424), with ConvNext (160-196) and TransConv
(124-159) per upsampling ratio.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np
import torch

from . import nlc, synth
from ._lib import call, lib, stream_handle

MAX_LAYERS = 16
MAX_UP = 4


@dataclass(frozen=True)
class Geometry:
    # crates/qwen3tts/src/cfg.rs:196-260 (the codec module)
    n_books: int = 16
    n_first: int = 1
    book_size: int = 2048
    book_dim: int = 256
    codebook_dim: int = 512
    latent_dim: int = 1024
    pre_kernel: int = 3
    tf_dim: int = 512
    tf_layers: int = 8
    tf_heads: int = 16
    tf_n_kv: int = 16
    tf_head_dim: int = 64
    tf_ffn: int = 1024
    tf_window: int = 72
    tf_eps: float = 1e-5
    tf_rope_base: float = 10_000.0
    up_ratios: tuple = (2, 2)
    dw_kernel: int = 7
    ln_eps: float = 1e-6
    max_frames: int = 1024

    @property
    def upsample(self):
        return int(np.prod(self.up_ratios))

    def flops_per_frame(self):
        """Algorithmic FLOPs (2*MACs) per code frame and lane (projections, convs, attention)."""
        g, f = self, 0
        f += 2 * (2 * g.book_dim) * g.codebook_dim
        f += 2 * g.codebook_dim * g.latent_dim * g.pre_kernel + 2 * g.latent_dim * g.tf_dim
        qkvw = (g.tf_heads + 2 * g.tf_n_kv) * g.tf_head_dim
        qw = g.tf_heads * g.tf_head_dim
        per_layer = 2 * g.tf_dim * qkvw + 2 * qw * g.tf_dim + 2 * g.tf_dim * 2 * g.tf_ffn + 2 * g.tf_ffn * g.tf_dim
        per_layer += 2 * 2 * g.tf_heads * g.tf_head_dim * g.tf_window  # scores and weighted v, full window
        f += g.tf_layers * per_layer + 2 * g.tf_dim * g.latent_dim
        length = 1
        for r in g.up_ratios:
            f += 2 * g.latent_dim * r * g.latent_dim * length
            length *= r
            f += (2 * g.latent_dim * 4 * g.latent_dim * 2 + 2 * g.latent_dim * g.dw_kernel) * length
        return f


CODEC = Geometry()


@dataclass
class HostWeights:
    """Checkpoint-layout f32 tensors (codebooks already folded)."""
    codebooks: np.ndarray = None       # [n_books, size, dim]
    out_proj_sem: np.ndarray = None    # [codebook_dim, book_dim, 1]
    out_proj_ac: np.ndarray = None
    pre_w: np.ndarray = None           # [latent, codebook_dim, pre_kernel]
    pre_b: np.ndarray = None
    in_w: np.ndarray = None            # [tf_dim, latent] (Linear [out, in])
    in_b: np.ndarray = None
    layers: list = field(default_factory=list)
    tf_norm: np.ndarray = None
    out_w: np.ndarray = None           # [latent, tf_dim]
    out_b: np.ndarray = None
    up: list = field(default_factory=list)  # dicts: up_w [C, C, r] (ConvTranspose [in, out, k]), up_b, dw_w [C, 1, k], ...


def fold_codebook(embedding_sum, cluster_usage, eps=1e-5):
    """Rvq::load's fold (codec.rs:275-282): embedding_sum / clamp(cluster_usage, eps)[:, None]."""
    usage = np.maximum(np.asarray(cluster_usage, np.float32), np.float32(eps))
    return (np.asarray(embedding_sum, np.float32) / usage[:, None]).astype(np.float32)


def random_weights(geo: Geometry, seed: int = 0) -> HostWeights:
    """Projections and convs N(0, 1/fan_in) (unit-gain, as the waveform stack's init), biases
    N(0, 0.01), norms U(0.9, 1.1), LayerScale and ConvNeXt gamma U(0.05, 0.15), codebooks folded
    from N(0, 1) sums and U(0.5, 2) usage counts."""
    g = geo

    def w(tag, shape, fan_in):
        return synth.normal(seed, "front." + tag, shape, 0.0, float(1.0 / np.sqrt(fan_in)))

    def b(tag, n):
        return synth.normal(seed, "front." + tag, (n,), 0.0, 0.01)

    def u(tag, n, lo=0.9, hi=1.1):
        return synth.uniform(seed, "front." + tag, (n,), lo, hi)

    hw = HostWeights()
    sums = synth.normal(seed, "front.books.sum", (g.n_books, g.book_size, g.book_dim))
    usage = synth.uniform(seed, "front.books.usage", (g.n_books, g.book_size), 0.5, 2.0)
    hw.codebooks = np.stack([fold_codebook(sums[i], usage[i]) for i in range(g.n_books)])
    hw.out_proj_sem = w("outproj.sem", (g.codebook_dim, g.book_dim, 1), g.book_dim)
    hw.out_proj_ac = w("outproj.ac", (g.codebook_dim, g.book_dim, 1), g.book_dim * 4)
    hw.pre_w = w("pre.w", (g.latent_dim, g.codebook_dim, g.pre_kernel), g.codebook_dim * g.pre_kernel)
    hw.pre_b = b("pre.b", g.latent_dim)
    hw.in_w, hw.in_b = w("in.w", (g.tf_dim, g.latent_dim), g.latent_dim), b("in.b", g.tf_dim)
    qw, kvw = g.tf_heads * g.tf_head_dim, g.tf_n_kv * g.tf_head_dim
    for i in range(g.tf_layers):
        p = f"l{i}."
        hw.layers.append(dict(
            wq=w(p + "wq", (qw, g.tf_dim), g.tf_dim), wk=w(p + "wk", (kvw, g.tf_dim), g.tf_dim),
            wv=w(p + "wv", (kvw, g.tf_dim), g.tf_dim), wo=w(p + "wo", (g.tf_dim, qw), qw),
            gate=w(p + "gate", (g.tf_ffn, g.tf_dim), g.tf_dim), up=w(p + "up", (g.tf_ffn, g.tf_dim), g.tf_dim),
            down=w(p + "down", (g.tf_dim, g.tf_ffn), g.tf_ffn),
            attn_norm=u(p + "attn_norm", g.tf_dim), ffn_norm=u(p + "ffn_norm", g.tf_dim),
            attn_scale=u(p + "attn_scale", g.tf_dim, 0.05, 0.15), mlp_scale=u(p + "mlp_scale", g.tf_dim, 0.05, 0.15)))
    hw.tf_norm = u("tf_norm", g.tf_dim)
    hw.out_w, hw.out_b = w("out.w", (g.latent_dim, g.tf_dim), g.tf_dim), b("out.b", g.latent_dim)
    c = g.latent_dim
    for i, r in enumerate(g.up_ratios):
        p = f"up{i}."
        hw.up.append(dict(
            up_w=w(p + "up.w", (c, c, r), c), up_b=b(p + "up.b", c),
            dw_w=w(p + "dw.w", (c, 1, g.dw_kernel), g.dw_kernel), dw_b=b(p + "dw.b", c),
            ln_w=u(p + "ln.w", c), ln_b=b(p + "ln.b", c),
            pw1_w=w(p + "pw1.w", (4 * c, c), c), pw1_b=b(p + "pw1.b", 4 * c),
            pw2_w=w(p + "pw2.w", (c, 4 * c), 4 * c), pw2_b=b(p + "pw2.b", c),
            gamma=u(p + "gamma", c, 0.05, 0.15)))
    return hw


def kernel_layouts(geo: Geometry, hw: HostWeights):
    """The f16/f32 arrays dtts_codec_front_create takes, from checkpoint layouts: the two output
    projections side by side along the input; pre_conv tap-major; q|k|v and gate|up rows
    concatenated; the transposed convs in the polyphase tap-major layout with the bias repeated
    per phase; the depthwise taps as [C, k]."""
    f16 = synth.f16_bits
    out = dict(codebooks=hw.codebooks.astype(np.float32),
               out_proj=f16(np.concatenate([hw.out_proj_sem[:, :, 0], hw.out_proj_ac[:, :, 0]], axis=1)),
               pre_w=f16(nlc.tap_major_weight(hw.pre_w)), pre_b=f16(hw.pre_b),
               in_w=f16(hw.in_w), in_b=f16(hw.in_b), tf_norm=hw.tf_norm.astype(np.float32),
               out_w=f16(hw.out_w), out_b=f16(hw.out_b), layers=[], up=[])
    for L in hw.layers:
        out["layers"].append(dict(
            attn_norm=L["attn_norm"], attn_scale=L["attn_scale"], ffn_norm=L["ffn_norm"], mlp_scale=L["mlp_scale"],
            wqkv=f16(np.concatenate([L["wq"], L["wk"], L["wv"]], 0)), wo=f16(L["wo"]),
            w_gateup=f16(np.concatenate([L["gate"], L["up"]], 0)), wdown=f16(L["down"])))
    for i, U in enumerate(hw.up):
        r = geo.up_ratios[i]
        out["up"].append(dict(
            up_w=f16(nlc.transpose_tap_major_weight(U["up_w"], r)), up_b=f16(nlc.transpose_bias(U["up_b"], r)),
            dw_taps=np.ascontiguousarray(U["dw_w"][:, 0, :], np.float32), dw_bias=U["dw_b"],
            ln_weight=U["ln_w"], ln_bias=U["ln_b"], pw1_w=f16(U["pw1_w"]), pw1_b=f16(U["pw1_b"]),
            pw2_w=f16(U["pw2_w"]), pw2_b=f16(U["pw2_b"]), gamma=U["gamma"]))
    return out


# ---------------------------------------------------------------- ctypes mirrors of dtts.h

class _Geometry(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ("n_books", "n_first", "book_size", "book_dim", "codebook_dim",
                                              "latent_dim", "pre_kernel", "tf_dim", "tf_layers", "tf_heads",
                                              "tf_n_kv", "tf_head_dim", "tf_ffn", "tf_window")] + [
        ("tf_eps", ctypes.c_float), ("tf_rope_base", ctypes.c_double), ("n_up", ctypes.c_int64),
        ("up_ratios", ctypes.c_int64 * MAX_UP), ("dw_kernel", ctypes.c_int64), ("ln_eps", ctypes.c_float),
        ("max_frames", ctypes.c_int64)]


class _Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("attn_norm", "attn_scale", "ffn_norm", "mlp_scale", "wqkv", "wo",
                                               "w_gateup", "wdown")]


class _Up(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("up_w", "up_b", "dw_taps", "dw_bias", "ln_weight", "ln_bias",
                                               "pw1_w", "pw1_b", "pw2_w", "pw2_b", "gamma")]


class _Weights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("codebooks", "out_proj", "pre_w", "pre_b", "in_w", "in_b")] + [
        ("layers", _Layer * MAX_LAYERS), ("tf_norm", ctypes.c_void_p), ("out_w", ctypes.c_void_p),
        ("out_b", ctypes.c_void_p), ("up", _Up * MAX_UP)]


def c_geometry(geo: Geometry) -> _Geometry:
    g = _Geometry(geo.n_books, geo.n_first, geo.book_size, geo.book_dim, geo.codebook_dim, geo.latent_dim,
                  geo.pre_kernel, geo.tf_dim, geo.tf_layers, geo.tf_heads, geo.tf_n_kv, geo.tf_head_dim,
                  geo.tf_ffn, geo.tf_window, geo.tf_eps, geo.tf_rope_base, len(geo.up_ratios))
    for i, r in enumerate(geo.up_ratios):
        g.up_ratios[i] = r
    g.dw_kernel, g.ln_eps, g.max_frames = geo.dw_kernel, geo.ln_eps, geo.max_frames
    return g


class CodecFront:
    """Device weights + a dtts_codec_front handle (keeps every device tensor alive)."""

    def __init__(self, geo: Geometry, hw: HostWeights, dev):
        self.geo, self.dev = geo, dev
        self._keep = []
        kl = kernel_layouts(geo, hw)

        def put(a):
            a = np.ascontiguousarray(a)
            t = torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a.astype(np.float32)).to(dev)
            if a.dtype == np.uint16:
                t = t.view(torch.float16)
            self._keep.append(t)
            return t.data_ptr()

        g = c_geometry(geo)
        ws = _Weights()
        for n in ("codebooks", "out_proj", "pre_w", "pre_b", "in_w", "in_b", "tf_norm", "out_w", "out_b"):
            setattr(ws, n, put(kl[n]))
        for i, L in enumerate(kl["layers"]):
            for n, _ in _Layer._fields_:
                setattr(ws.layers[i], n, put(L[n]))
        for i, U in enumerate(kl["up"]):
            for n, _ in _Up._fields_:
                setattr(ws.up[i], n, put(U[n]))
        self._g, self._w = g, ws
        handle = ctypes.c_void_p()
        call("dtts_codec_front_create", ctypes.byref(g), ctypes.byref(ws), ctypes.byref(handle))
        self.handle = handle
        self._ws = None

    def close(self):
        if self.handle:
            lib().dtts_codec_front_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def workspace(self, lanes, frames):
        need = int(lib().dtts_codec_front_workspace_bytes(self.handle, lanes, frames))
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.dev)
        return self._ws

    def decode(self, codes, out=None):
        """codes: host int32 [lanes, frames, n_books] -> latent [lanes, frames * upsample, latent] f16."""
        codes = np.ascontiguousarray(codes, np.int32)
        lanes, frames, nb = codes.shape
        assert nb == self.geo.n_books
        y = out if out is not None else torch.empty((lanes, frames * self.geo.upsample, self.geo.latent_dim),
                                                    dtype=torch.float16, device=self.dev)
        ws = self.workspace(lanes, frames)
        call("dtts_codec_front_decode", self.handle, codes.ctypes.data_as(ctypes.c_void_p),
             ctypes.c_void_p(y.data_ptr()), lanes, frames, ctypes.c_void_p(ws.data_ptr()), ws.numel(),
             stream_handle(self.dev))
        return y


CHUNK_FRAMES = 300  # crates/qwen3tts/src/cfg.rs:281
CHUNK_LEFT_CONTEXT = 25  # cfg.rs:282


def decode_document(front: CodecFront, wave, codes, chunk=CHUNK_FRAMES, context=CHUNK_LEFT_CONTEXT, out=None):
    """Codec::decode (crates/qwen3tts/src/codec.rs:562-604) through dtts_codec_decode_document:
    codes host int32 [n, n_books] -> audio [n * upsample * hop] f32 on the device. `wave` is a
    dtts.codec.Codec (the waveform stack); its workspace is not used."""
    codes = np.ascontiguousarray(codes, np.int32)
    n, nb = codes.shape
    assert nb == front.geo.n_books
    spf = front.geo.upsample * wave.geo.hop
    y = out if out is not None else torch.empty(n * spf, dtype=torch.float32, device=front.dev)
    need = int(lib().dtts_codec_document_workspace_bytes(front.handle, wave.handle, n, chunk, context))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=front.dev)
    call("dtts_codec_decode_document", front.handle, wave.handle, codes.ctypes.data_as(ctypes.c_void_p), n, chunk,
         context, ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
         stream_handle(front.dev))
    return y
