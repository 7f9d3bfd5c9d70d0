"""The parity figures of tests/workloads.py on hand-made f16 arrays (CPU):
each figure on a case with a known answer, so a slip in the metric (a wrong
floor, a swapped operand, the ulp of the wrong exponent) fails here rather
than loosening every GPU parity check."""
from __future__ import annotations

import numpy as np

from workloads import HD, error_report, f16_ulp


def _u16(x):
    return np.asarray(x, dtype=np.float16).view(np.uint16)


def test_f16_ulp_known_values():
    # 1.0 .. 2.0: spacing 2^-10; 2.0 .. 4.0: 2^-9; subnormals: 2^-24
    assert f16_ulp(1.0) == 2.0 ** -10
    assert f16_ulp(1.999) == 2.0 ** -10
    assert f16_ulp(-2.0) == 2.0 ** -9
    assert f16_ulp(3.5) == 2.0 ** -9
    assert f16_ulp(2.0 ** -20) == 2.0 ** -24
    assert f16_ulp(0.0) == 2.0 ** -24
    # every finite f16 and its successor differ by exactly one ulp of the smaller
    bits = np.arange(0, 0x7BFF, dtype=np.uint16)
    a = bits.view(np.float16).astype(np.float64)
    b = (bits + 1).view(np.float16).astype(np.float64)
    assert np.all((b - a) == f16_ulp(a))


def test_error_report_figures():
    ref = np.zeros((2, HD), np.float32)
    ref[0, 0], ref[0, 1], ref[1, 5] = 3.0, 0.5, -1e-4
    got = ref.copy()
    got[0, 0] = np.float16(3.0) + np.float16(2.0 ** -9)  # one ulp at [2, 4)
    got[1, 5] = -2e-4                                    # 1e-4 absolute near zero
    e = error_report(_u16(got), _u16(ref))
    d16 = float(np.float16(-2e-4)) - float(np.float16(-1e-4))
    assert e["max_abs"] == 2.0 ** -9
    assert abs(e["max_rel"] - 2.0 ** -9 / 3.0) < 1e-12          # |ref| above the 0.2 floor
    assert abs(e["max_rel_small"] - abs(d16) / 1e-3) < 1e-9     # near zero: the 1e-3 floor
    assert e["max_ulp"] >= 1.0 and abs(e["max_ulp"] - abs(d16) / f16_ulp(np.float16(-1e-4))) < 1e-9
    assert e["max_ulp_big"] == 1.0  # the one-ulp difference at 3.0; the near-zero one is excluded
    assert e["ref_at_max_abs"] == 3.0
    # per-head vector norm: row 0 differs by one ulp in one of its two nonzero entries
    r0 = np.sqrt(3.0 ** 2 + 0.5 ** 2)
    assert e["max_rel_vec"] >= 2.0 ** -9 / r0 - 1e-12
    same = error_report(_u16(ref), _u16(ref))
    assert all(v == 0.0 for k, v in same.items() if k != "ref_at_max_abs")
