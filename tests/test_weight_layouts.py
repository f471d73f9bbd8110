"""The library's host-side weight layouts against the oracle's restatements of tts-nn's
(tap_weight, tap_major_weight, transpose_tap_weight, transpose_bias). Bit-exact: these are
permutations. Runs on the CPU (host code of libdtts, no device calls)."""
import numpy as np
import pytest

import oracle
from dtts import nlc, synth


def test_tap_major_matches_reference_layout():
    w = synth.normal(30, "w", (12, 8, 7))
    assert np.array_equal(nlc.tap_major_weight(w), oracle.tap_major_weight_f32(w))
    # from nlc::tap_weight's [k, cin, cout] layout to the same place
    assert np.array_equal(nlc.tap_weight_to_tap_major(oracle.tap_weight_f32(w)),
                          oracle.tap_major_weight_f32(w))
    # f16 (2-byte elements) permute identically
    h = synth.f16_bits(w)
    assert np.array_equal(nlc.tap_major_weight(h), synth.f16_bits(oracle.tap_major_weight_f32(w)))


@pytest.mark.parametrize("cin,cout,stride,mult", [(8, 6, 2, 1), (8, 6, 2, 2), (12, 8, 5, 2),
                                                  (10, 7, 3, 2), (9, 5, 4, 1), (16, 8, 8, 2)])
def test_transpose_tap_major_matches_reference(cin, cout, stride, mult):
    w = synth.normal(31, f"w{cin}{stride}", (cin, cout, mult * stride))
    ref_tap = oracle.transpose_tap_weight_f32(w, stride)  # [m, cin, stride*cout]
    want = nlc.tap_weight_to_tap_major(ref_tap)
    assert np.array_equal(nlc.transpose_tap_major_weight(w, stride), want)
    b = synth.normal(31, "b", (cout,))
    assert np.array_equal(nlc.transpose_bias(b, stride), oracle.transpose_bias_f32(b, stride))


def test_transpose_rejects_indivisible_kernel():
    from dtts import DttsError

    with pytest.raises(DttsError, match="divisible"):
        nlc.transpose_tap_major_weight(np.zeros((2, 3, 5), np.float32), 2)
