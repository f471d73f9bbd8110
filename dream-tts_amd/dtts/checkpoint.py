"""Checkpoints and weight formats from Python: the safetensors reader (dtts_checkpoint_*), the
device conversions into kernel layouts (dtts_convert_*), and Codec::load (dtts_codec_model_load).

Mirrors crates/tts-nn/src/lib.rs:143-360 (Weights: open, get, names, len, file_shape) and
crates/qwen3tts/src/codec.rs:347-399 (Codec::load), whose tensor names the model loader reads.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import codec, codec_front, stack
from ._lib import call, lib, stream_handle

DT_F32, DT_F16, DT_BF16, DT_F64, DT_I64, DT_I32, DT_I16, DT_I8, DT_U8, DT_BOOL, DT_OTHER = range(11)
# numpy views of the on-disk bytes (bf16 as its uint16 bit patterns)
_NUMPY = {DT_F32: np.float32, DT_F16: np.float16, DT_BF16: np.uint16, DT_F64: np.float64, DT_I64: np.int64,
          DT_I32: np.int32, DT_I16: np.int16, DT_I8: np.int8, DT_U8: np.uint8, DT_BOOL: np.bool_}
_TORCH = {DT_F32: torch.float32, DT_F16: torch.float16, DT_BF16: torch.bfloat16, DT_F64: torch.float64}


class TensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * 8), ("data", ctypes.c_void_p), ("bytes", ctypes.c_size_t)]

    @property
    def dims(self):
        return tuple(self.shape[i] for i in range(self.ndim))


class Checkpoint:
    """A memory-mapped safetensors file (Weights::load)."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        call("dtts_checkpoint_open", str(path).encode(), ctypes.byref(h))
        self.handle, self.path = h, str(path)

    def close(self):
        if self.handle:
            lib().dtts_checkpoint_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __len__(self):
        return int(lib().dtts_checkpoint_count(self.handle))

    def info(self, key) -> TensorInfo:
        t = TensorInfo()
        if isinstance(key, int):
            call("dtts_checkpoint_at", self.handle, key, ctypes.byref(t))
        else:
            call("dtts_checkpoint_get", self.handle, key.encode(), ctypes.byref(t))
        return t

    def names(self):
        """Every tensor name, sorted (Weights::names)."""
        return sorted(self.info(i).name.decode() for i in range(len(self)))

    def host(self, name: str) -> np.ndarray:
        """The tensor's bytes in its on-disk dtype, copied out of the mapping."""
        t = self.info(name)
        raw = ctypes.string_at(t.data, t.bytes)
        return np.frombuffer(raw, dtype=_NUMPY[t.dtype]).reshape(t.dims).copy()

    def device(self, name: str, dev) -> tuple[torch.Tensor, int]:
        """The raw tensor uploaded as is (for the dtts_convert_* entry points) and its dtype code."""
        t = self.info(name)
        a = self.host(name)
        if t.dtype == DT_BF16:
            return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev), t.dtype
        return torch.from_numpy(a).to(dev), t.dtype


class _Part:
    """A model-owned handle with the attributes the decode helpers read."""

    def __init__(self, handle, geo, dev):
        self.handle, self.geo, self.dev = handle, geo, dev


class CodecModel:
    """Codec::load: the front half and waveform stack converted from a checkpoint into one device
    arena owned by the model."""

    def __init__(self, ck: Checkpoint, front_geo: codec_front.Geometry, wave_geo: codec.Geometry, dev):
        self._fg, self._wg = codec_front.c_geometry(front_geo), codec.c_geometry(wave_geo)
        h = ctypes.c_void_p()
        # dev None: the null stream (a checkpoint refused by the shape checks never reaches it)
        args = (ck.handle, ctypes.byref(self._fg), ctypes.byref(self._wg))
        if dev is None:
            call("dtts_codec_model_load", *args, ctypes.c_void_p(), ctypes.byref(h))
        else:
            with torch.cuda.device(dev):
                call("dtts_codec_model_load", *args, stream_handle(dev), ctypes.byref(h))
        self.handle, self.dev = h, dev
        self.front = _Part(ctypes.c_void_p(lib().dtts_codec_model_front(h)), front_geo, dev)
        self.wave = _Part(ctypes.c_void_p(lib().dtts_codec_model_wave(h)), wave_geo, dev)

    @property
    def nbytes(self):
        return int(lib().dtts_codec_model_bytes(self.handle))

    def close(self):
        if self.handle:
            lib().dtts_codec_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def latent(self, codes):
        """codes host int32 [lanes, frames, n_books] -> latent [lanes, frames * upsample, latent] f16."""
        codes = np.ascontiguousarray(codes, np.int32)
        lanes, frames, _ = codes.shape
        g = self.front.geo
        y = torch.empty((lanes, frames * g.upsample, g.latent_dim), dtype=torch.float16, device=self.dev)
        need = int(lib().dtts_codec_front_workspace_bytes(self.front.handle, lanes, frames))
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=self.dev)
        call("dtts_codec_front_decode", self.front.handle, codes.ctypes.data_as(ctypes.c_void_p),
             ctypes.c_void_p(y.data_ptr()), lanes, frames, ctypes.c_void_p(ws.data_ptr()), ws.numel(),
             stream_handle(self.dev))
        return y

    def decode(self, codes, chunk=codec_front.CHUNK_FRAMES, context=codec_front.CHUNK_LEFT_CONTEXT):
        """Codec::decode: codes [n, n_books] -> f32 audio on the device."""
        return codec_front.decode_document(self.front, self.wave, codes, chunk, context)


class StackModel:
    """Stack::load: a decoder stack's weights converted from a checkpoint into one device arena;
    `.stack` decodes like a dtts.stack.Stack."""

    def __init__(self, ck: Checkpoint, prefix: str, geo: stack.Geometry, dev, weight: str = "f16"):
        self._g = stack.c_geometry(geo)
        h = ctypes.c_void_p()
        args = (ck.handle, prefix.encode(), ctypes.byref(self._g), stack.WEIGHTS[weight])
        if dev is None:
            call("dtts_stack_model_load_as", *args, ctypes.c_void_p(), ctypes.byref(h))
        else:
            with torch.cuda.device(dev):
                call("dtts_stack_model_load_as", *args, stream_handle(dev), ctypes.byref(h))
        self.handle, self.dev = h, dev
        self.stack = stack.Stack.from_handle(geo, ctypes.c_void_p(lib().dtts_stack_model_stack(h)), dev, self)
        self.stack.weight = weight

    @property
    def nbytes(self):
        return int(lib().dtts_stack_model_bytes(self.handle))

    def close(self):
        if self.handle:
            self.stack.handle = None
            lib().dtts_stack_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def convert(fn: str, *args, dev=None):
    """Calls dtts_convert_<fn> on torch's current stream."""
    call("dtts_convert_" + fn, *args, stream_handle(dev))
