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
