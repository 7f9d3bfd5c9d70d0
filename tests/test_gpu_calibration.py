"""The calibration entry points bench.py reads the rooflines against:
qasr_stream_read (a bare HBM stream) and qasr_mfma_probe (the matrix core's
rate, the shader clock, MFMA/VALU overlap).  They must run every mode, keep
their results live (finite sinks), time with the shader and 100 MHz clocks,
and refuse bad arguments."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_mfma_probe_runs_every_mode_and_kind(gpu):
    import torch

    import qasr_attn

    ctx = qasr_attn.Context()
    sink = torch.full((16 * 8,), float("nan"), dtype=torch.float32, device="cuda")
    clk = torch.zeros(4, dtype=torch.int64, device="cuda")
    for kind in range(8):
        for base in range(4):
            mode = base + 4 * kind
            waves = 8 if base == 2 else 4
            sink.fill_(float("nan"))
            qasr_attn.mfma_probe(ctx, mode, 16, waves, 50, 20, sink, clk)
            torch.cuda.synchronize()
            got = sink[:16 * waves].cpu().numpy()
            assert np.all(np.isfinite(got)), f"mode {mode}"
            c = clk.cpu().numpy()
            assert c[2] > c[0] and c[3] > c[1], f"mode {mode}: clocks {c}"
    ctx.close()


def test_mfma_probe_refuses_bad_arguments(gpu):
    import torch

    import qasr_attn

    ctx = qasr_attn.Context()
    sink = torch.zeros(64 * 8, dtype=torch.float32, device="cuda")
    clk = torch.zeros(4, dtype=torch.int64, device="cuda")
    with pytest.raises(qasr_attn.QasrError, match="VALU kind"):
        qasr_attn.mfma_probe(ctx, 4 * 8, 1, 4, 1, 1, sink, clk)
    with pytest.raises(qasr_attn.QasrError, match="negative mode"):
        qasr_attn.mfma_probe(ctx, -1, 1, 4, 1, 1, sink, clk)
    with pytest.raises(qasr_attn.QasrError, match="iterations"):
        qasr_attn.mfma_probe(ctx, 0, 1, 4, -1, 1, sink, clk)
    ctx.close()


def test_stream_read_runs_and_refuses_ragged_bytes(gpu):
    import torch

    import qasr_attn

    ctx = qasr_attn.Context()
    src = torch.ones(256 * 1024, dtype=torch.float16, device="cuda")
    sink = torch.zeros(64 * 4, dtype=torch.int32, device="cuda")
    qasr_attn.stream_read(ctx, src, 64, 4, sink)
    torch.cuda.synchronize()
    # every word of src is 0x3C00 twice: the per-wave xor-folds are equal
    got = sink.cpu().numpy()
    assert np.all(got == got[0])
    with pytest.raises(qasr_attn.QasrError, match="multiple of 16"):
        qasr_attn.stream_read(ctx, src[:1000], 64, 4, sink)
    ctx.close()
