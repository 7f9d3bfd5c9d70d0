"""The attention kernels' softmax exponent against the reference's libm expf.

The reference weights key t of a row by e_t = expf(s_t - best) with
s_t = dot_t * scale (cpu_decoder.rs:292-365; Rust's f32::exp is glibc expf).
The kernels work in the exp2 domain: the scale is folded with log2(e) once
on the host (sl2), and v_exp_f32 exponentiates either f32(s*sl2) - f32(m*sl2)
(decode) or fma(s, sl2, -f32(m*sl2)) (prefill).  qasr_softmax_weights runs
those exact device expressions (common.hpp) over arrays; the oracle's
qo_softmax_weights runs the reference expression with glibc expf.

Bound: both sides round their products and difference once, so the exponent
arguments differ by at most (|s*scale| + |m*scale| + |d|) * 2^-24 in the
natural-log domain (d = (s - m) * scale), plus one-ulp-level errors of
v_exp_f32 and expf: relative error <= (|s*scale| + |m*scale| + |d|) * 2^-22 +
2^-21.  The sweep covers the weights a softmax row can produce
(d in [-80, 0], results stay normal f32) over raw dot products far beyond
what normed heads give.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SCALE = np.float32(1.0 / np.sqrt(np.float32(128.0)))


def _sweep(seed: int, n: int):
    rng = np.random.default_rng(seed)
    m = rng.uniform(-400.0, 400.0, n).astype(np.float32)
    d = rng.uniform(0.0, 80.0, n)  # natural-log distance below the max
    s = (m.astype(np.float64) - d / float(SCALE)).astype(np.float32)
    s = np.minimum(s, m)
    # special cases: s == m (weight 1), tiny distances, integer-valued dots
    k = 4096
    s[:k] = m[:k]
    s[k:2 * k] = np.nextafter(m[k:2 * k], np.float32(-np.inf))
    ints = rng.integers(-300, 300, 2 * k).astype(np.float32)
    m[2 * k:4 * k] = np.maximum(ints, ints[::-1])
    s[2 * k:4 * k] = np.minimum(ints, ints[::-1])
    return s, m


def test_softmax_exponent_matches_glibc_expf(O, gpu):
    import torch

    from gpu_helpers import say

    ctx = gpu.Context(16, 8, 128, 1, 1e-6, 16384, 0)
    s, m = _sweep(0x51A5E, 1 << 21)
    say(f"softmax weights: {s.size} (score, max) pairs")
    dec, pre = gpu.softmax_weights(ctx, torch.from_numpy(s).cuda(), torch.from_numpy(m).cuda())
    torch.cuda.synchronize()
    dec, pre = dec.cpu().numpy().astype(np.float64), pre.cpu().numpy().astype(np.float64)
    ref = O.softmax_weights(s, m, float(SCALE)).astype(np.float64)
    ctx.close()

    assert np.all(ref > 0) and np.all(np.isfinite(ref))
    ss = np.abs(s.astype(np.float64) * float(SCALE))
    mm = np.abs(m.astype(np.float64) * float(SCALE))
    dd = np.abs((s.astype(np.float64) - m) * float(SCALE))
    bound = (ss + mm + dd) * 2.0 ** -22 + 2.0 ** -21
    eq = s == m
    for name, got in (("decode", dec), ("prefill", pre)):
        rel = np.abs(got - ref) / ref
        ulps = np.abs(got - ref) / np.spacing(ref.astype(np.float32)).astype(np.float64)
        say(f"{name}: max rel {rel.max():.3e}, max {ulps.max():.1f} ulp, "
            f"median {np.median(ulps):.2f} ulp, worst rel/bound {(rel / bound).max():.3f}")
        assert np.all(rel <= bound), f"{name}: relative error beyond the rounding bound"
    # equal score and max: the reference's weight is exactly 1, and so is
    # the decode form's (its argument is exactly 0)
    assert np.all(ref[eq] == 1.0)
    assert np.all(dec[eq] == 1.0)


def test_softmax_weights_refuses_bad_arguments(gpu):
    import torch

    ctx = gpu.Context(16, 8, 128, 1, 1e-6, 16384, 0)
    s = torch.zeros(8, device="cuda")
    with pytest.raises(gpu.QasrError) as e:
        gpu.softmax_weights(ctx, s, torch.zeros(7, device="cuda"))
    assert e.value.code == gpu.QASR_EINVAL
    ctx.close()
