"""The C-ABI library loads on the CPU host and exports exactly what include/*.h declares.

No compute calls (no GPU here): only entry points that fail argument checks before touching the
device are invoked, which also pins the error behaviour (status + dtts_last_error message).
"""
import ctypes
import glob
import os
import re

import pytest

from dtts import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(dtts_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = _declared()
    assert declared, "no declarations found"
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    unbound = sorted(declared - set(_lib.SIGNATURES))
    assert not unbound, f"declared but not bound in dtts._lib.SIGNATURES: {unbound}"


def test_version_and_error_slot():
    lib = _lib.lib()
    assert lib.dtts_version() >> 16 == 1
    assert isinstance(lib.dtts_last_error(), bytes)


def test_invalid_shape_is_rejected_before_any_device_work():
    lib = _lib.lib()
    rc = lib.dtts_snake_nlc_f32(None, None, None, None, -1, 4, None)
    assert rc == -1
    assert b"negative shape" in lib.dtts_last_error()
    rc = lib.dtts_snake_nlc_f32(None, None, None, None, 4, 4, None)
    assert rc == -1 and b"null pointer" in lib.dtts_last_error()
    # an empty tensor is a no-op, not an error
    assert lib.dtts_snake_nlc_f32(None, None, None, None, 0, 4, None) == 0
    with pytest.raises(_lib.DttsError, match="negative shape"):
        _lib.call("dtts_snake_ncl_f32", None, None, None, None, 1, -2, 3, None)


def test_stack_create_and_decode_check_arguments_on_the_host():
    """Geometry and argument errors of the decoder-stack entry points come back before any HIP
    call (these run without a GPU)."""
    import numpy as np
    from dtts import stack

    lib = _lib.lib()
    geo = stack.Geometry(dim=256, layers=1, heads=3, n_kv=2, head_dim=128, ffn=512)
    g = stack._Geometry(geo.dim, geo.layers, geo.heads, geo.n_kv, geo.head_dim, geo.ffn, geo.eps,
                        geo.rope_base, 1, 0, 0, 64)
    layers = (stack._Layer * 1)()
    handle = ctypes.c_void_p()
    rc = lib.dtts_stack_create(ctypes.byref(g), ctypes.cast(layers, ctypes.c_void_p), ctypes.c_void_p(16),
                               ctypes.byref(handle))
    assert rc == -1 and b"3 heads over 2 kv heads" in lib.dtts_last_error()
    g.heads = 4
    rc = lib.dtts_stack_create(ctypes.byref(g), ctypes.cast(layers, ctypes.c_void_p), ctypes.c_void_p(16),
                               ctypes.byref(handle))
    assert rc == -1 and b"layer 0 incomplete" in lib.dtts_last_error()
    g.ffn = 500
    rc = lib.dtts_stack_create(ctypes.byref(g), ctypes.cast(layers, ctypes.c_void_p), ctypes.c_void_p(16),
                               ctypes.byref(handle))
    assert rc == -1 and b"multiples of 128" in lib.dtts_last_error()
    assert lib.dtts_stack_workspace_bytes(None, 4, 16) == 0
    pos = np.zeros(4, np.int32)
    rc = lib.dtts_stack_decode(None, None, None, None, 4, 16, pos.ctypes.data_as(ctypes.c_void_p), None, 0, 0, None)
    assert rc == -1 and b"null stack" in lib.dtts_last_error()
