"""dtts_gemm_f16_nt_noalloc: the decode projection with its k-range partials in the library's own
device scratch instead of a caller's workspace, through the C ABI.

Held to dtts_gemm_f16_nt with a workspace bit for bit (the same kernels, split and summation
order), on two calls in a row, the second with a smaller input whose partial tiles cover less of
the shared scratch than the first left behind; and the oracle's f32-accumulated product within
the f16 GEMM bars (max-abs 2e-2, max-rel 1e-4). Shapes whose partials exceed the scratch are
refused on the host before anything is enqueued.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from dtts import DttsError, synth
from dtts._lib import call, lib, ptr, stream_handle

from _util import rel, to_dev

pytestmark = pytest.mark.gpu


def _case(seed, m, k, n):
    a = synth.f16_bits(synth.normal(seed, "a", (m, k)))
    w = synth.f16_bits(synth.normal(seed, "w", (n, k), 0, 0.02))
    return a, w


def _with_workspace(a_d, w_d, m, k, n):
    need = int(lib().dtts_gemm_f16_workspace_bytes(m, k, n, 0))
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=a_d.device)
    c = torch.empty((m, n), dtype=torch.float32, device=a_d.device)
    call("dtts_gemm_f16_nt", ptr(a_d), ptr(w_d), ptr(c), m, k, n, ptr(ws), ctypes.c_size_t(need), stream_handle())
    return c, need


def _noalloc(a_d, w_d, m, k, n):
    c = torch.full((m, n), float("nan"), dtype=torch.float32, device=a_d.device)
    call("dtts_gemm_f16_nt_noalloc", ptr(a_d), ptr(w_d), ptr(c), m, k, n, stream_handle())
    return c


def test_noalloc_projection_matches_workspace_form_twice(dev):
    results = []
    for seed, (m, k, n) in ((80, (48, 6144, 2048)), (81, (16, 4096, 1024))):  # the second one smaller
        a, w = _case(seed, m, k, n)
        a_d, w_d = to_dev(a, dev), to_dev(w, dev)
        want, need = _with_workspace(a_d, w_d, m, k, n)
        assert need > 0  # the shape splits k, so the scratch is in use
        got = _noalloc(a_d, w_d, m, k, n)
        torch.cuda.synchronize()
        g, wv = got.cpu().numpy(), want.cpu().numpy()
        assert np.array_equal(g, wv), f"({m}, {k}, {n}): differs from dtts_gemm_f16_nt"
        ref = oracle.gemm_f16_f32acc(a, np.ascontiguousarray(w.T))
        assert np.max(np.abs(g - ref)) <= 2e-2
        assert rel(g, ref)[1] < 1e-4
        results.append(need)
    assert results[1] < results[0]


def test_noalloc_projection_refuses_shapes_past_its_scratch(dev):
    m, k, n = 64, 8192, 8192
    assert lib().dtts_gemm_f16_workspace_bytes(m, k, n, 0) > (16 << 20)
    c = torch.zeros((1,), dtype=torch.float32, device=dev)
    with pytest.raises(DttsError, match="more than the 16777216"):
        call("dtts_gemm_f16_nt_noalloc", ptr(c), ptr(c), ptr(c), m, k, n, stream_handle())
