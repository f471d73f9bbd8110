"""dtts: MI355X (gfx950) kernels for dream-tts's tts-nn fused-op hot path.

``dtts.ops`` mirrors tts-nn's functions on torch device tensors; ``dtts._lib`` is the ctypes
binding of ``include/dtts.h``; ``dtts.synth`` draws the seeded synthetic inputs.
"""
from ._lib import DttsError, LIB_PATH, lib  # noqa: F401

__all__ = ["DttsError", "LIB_PATH", "lib"]
