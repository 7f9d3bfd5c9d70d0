"""qasr_dequant_i8 -- the f16 values of a resident-int8 weight, f16(f32(q) *
scale[row]) with RNE (dequant_i8, src/weights.rs:366-385) -- on the GPU,
against the reference's own dequantisation tests (transcribed in
tests/golden/reference_known_answers.json) and, for every int8 value times
scales over the whole f16 range (subnormal results included), bitwise
against numpy's f32 product rounded to f16."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "reference_known_answers.json")


@pytest.fixture(scope="module")
def ctx(gpu):
    import qasr_attn

    c = qasr_attn.Context()
    yield c
    c.close()


def _run(ctx, q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    import torch

    import qasr_attn

    out = qasr_attn.dequant_i8(ctx, torch.from_numpy(q).cuda(), torch.from_numpy(scale).cuda())
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("case", range(2))
def test_reference_known_answers(ctx, case):
    c = json.load(open(GOLDEN))["int8_dequant"][case]
    rows, cols = c["rows"], c["cols"]
    q = np.zeros((rows, 8), np.int8)  # columns padded to the kernel's multiple of 8
    q[:, :cols] = np.array(c["q"], np.int8).reshape(rows, cols)
    got = _run(ctx, q, np.array(c["scale"], np.float32))
    assert got[:, :cols].reshape(-1).tolist() == c["expect"], c["source"]
    assert not got[:, cols:].any()


def test_every_int8_value_against_f32_then_f16_rounding(ctx):
    rng = np.random.default_rng(17)
    rows = 4096
    q = np.tile(np.arange(-128, 128, dtype=np.int16), (rows, 1)).astype(np.int8)
    # scales from 2^-30 (products in and below the f16 subnormal range) to 2^8
    scale = (rng.random(rows, dtype=np.float32) + 0.5) * np.exp2(
        rng.integers(-30, 9, size=rows)).astype(np.float32)
    scale[::7] *= -1
    want = (q.astype(np.float32) * scale[:, None]).astype(np.float16)
    got = _run(ctx, q, scale)
    bad = np.nonzero(got.view(np.uint16) != want.view(np.uint16))
    assert bad[0].size == 0, (f"{bad[0].size} values differ, e.g. q={q[bad][0]} "
                              f"scale={scale[bad[0][0]]!r}: {got[bad][0]} vs {want[bad][0]}")


def test_bad_shapes_are_refused(ctx):
    import torch

    import qasr_attn

    q = torch.zeros((4, 6), dtype=torch.int8, device="cuda")
    s = torch.ones(4, dtype=torch.float32, device="cuda")
    with pytest.raises(qasr_attn.QasrError, match="multiple of 8"):
        qasr_attn.dequant_i8(ctx, q, s)
