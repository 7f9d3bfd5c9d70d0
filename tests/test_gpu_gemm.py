"""The prefill projections' GEMM (qasr_gemm_f16, csrc/gemm.hip) against a
plain PyTorch fp32 reference of the same product, and its refusals.

The kernel accumulates in f32 and rounds once (the residual, when
accumulating, is added in f32 before that rounding: batch_dot_acc,
cpu_decoder.rs:45-62).  An f32 sum of K terms taken in any order is within
(K - 1) 2^-24 sum|a_i b_i| of the exact sum, so each output is within half
an f16 spacing of the reference plus that bound; and since the bound is far
below an f16 spacing almost everywhere, nearly every output is the f16
rounding of the fp32 reference itself.  (A dropped term or a wrong index
breaks the bound by orders of magnitude.)"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _f16_spacing(x):
    """Spacing of f16 at |x| (x f32), the subnormal spacing below 2^-14."""
    ax = np.abs(x).astype(np.float32)
    e = np.floor(np.log2(np.maximum(ax, 2.0 ** -14)))
    return np.exp2(e - 10).astype(np.float64)


# (m, n, k): the 1.7B and 0.6B projections at a batched-prefill row count
# (qkv, o_proj, gate|up, down), ragged row counts around the 128/256-row
# blocks, and the smallest shapes the kernel takes.
SHAPES = [(4269, 4096, 2048), (4269, 2048, 2048), (4269, 12288, 2048), (4269, 2048, 6144),
          (1000, 4096, 1024), (420, 1024, 2048), (420, 6144, 1024), (420, 1024, 3072),
          (130, 256, 64), (129, 512, 128), (256, 256, 192), (1, 256, 64)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("accumulate", [False, True])
def test_gemm_matches_fp32_reference(gpu, m, n, k, accumulate):
    import torch

    import qasr_attn
    from gpu_helpers import say

    g = torch.Generator(device="cuda").manual_seed(7000 + m + n + k + int(accumulate))
    a = torch.randn((m, k), generator=g, device="cuda").to(torch.float16)
    b = (torch.randn((n, k), generator=g, device="cuda") * 0.05).to(torch.float16)
    c0 = torch.randn((m, n), generator=g, device="cuda").to(torch.float16)
    c = c0.clone()
    say(f"gemm {m}x{n}x{k} accumulate={accumulate}")
    qasr_attn.gemm_f16(g_ctx(), a, b, c, accumulate=accumulate)
    bt = b.float().t().contiguous()
    ref = torch.mm(a.float(), bt)
    mag = torch.mm(a.float().abs(), bt.abs())
    if accumulate:
        ref = ref + c0.float()
        mag = mag + c0.float().abs()
    got = c.float().cpu().numpy().astype(np.float64)
    ref = ref.cpu().numpy().astype(np.float64)
    mag = mag.cpu().numpy().astype(np.float64)
    want16 = ref.astype(np.float32).astype(np.float16).astype(np.float64)
    assert np.all(np.isfinite(got))
    # the kernel's and the reference's own f32 sums each within (k+1) 2^-24 mag
    bound = 0.5 * _f16_spacing(ref) + 2 * (k + 1) * 2.0 ** -24 * mag
    err = np.abs(got - ref)
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert np.all(err <= bound), (f"error {err[worst]:.3e} above bound {bound[worst]:.3e} at {worst}, "
                                  f"ref {ref[worst]:.6e}")
    assert (got == want16).mean() > 0.99


def test_gemm_refuses_bad_shapes(gpu):
    import torch

    import qasr_attn

    a = torch.zeros((64, 100), dtype=torch.float16, device="cuda")
    b = torch.zeros((256, 100), dtype=torch.float16, device="cuda")
    with pytest.raises(qasr_attn.QasrError, match="multiple of 64"):
        qasr_attn.gemm_f16(g_ctx(), a, b)
    a = torch.zeros((64, 128), dtype=torch.float16, device="cuda")
    b = torch.zeros((200, 128), dtype=torch.float16, device="cuda")
    with pytest.raises(qasr_attn.QasrError, match="multiple of 64, n of 256"):
        qasr_attn.gemm_f16(g_ctx(), a, b)


_CTX = None


def g_ctx():
    """One context for the module (the GEMM only needs a device)."""
    global _CTX
    if _CTX is None:
        import qasr_attn
        _CTX = qasr_attn.Context()
    return _CTX


# Block tiles the launcher chooses from (QASR_GEMM_TILE = 1..6): 256x256,
# 192x256 and 128x128 (eight waves), 64x128, 128x64, 64x64 (four).
TILES = [1, 2, 3, 4, 5, 6]


@pytest.mark.parametrize("m,n,k,accumulate", [(300, 512, 256, False), (4269, 2048, 2048, True),
                                              (65, 1024, 3072, True), (520, 768, 64, True),
                                              (257, 512, 128, False)])
def test_gemm_tile_choice_keeps_bits(gpu, m, n, k, accumulate, monkeypatch):
    """Every block tile gives the same bits, so the per-shape tile choice
    (a function of the row count) cannot make a row's result depend on how
    many rows the call carries; the default choice is one of them, and the
    shared result meets the fp32 reference's bound.  K = 64 and 128 run the
    large tiles' ping-pong loop over one and two K steps (its copies and
    waits at their boundaries)."""
    import torch

    import qasr_attn
    from gpu_helpers import say

    g = torch.Generator(device="cuda").manual_seed(7100 + m + n + k)
    a = torch.randn((m, k), generator=g, device="cuda").to(torch.float16)
    b = (torch.randn((n, k), generator=g, device="cuda") * 0.05).to(torch.float16)
    c0 = torch.randn((m, n), generator=g, device="cuda").to(torch.float16)
    outs = {}
    for tile in [0] + TILES:
        if tile:
            monkeypatch.setenv("QASR_GEMM_TILE", str(tile))
        else:
            monkeypatch.delenv("QASR_GEMM_TILE", raising=False)
        c = c0.clone()
        say(f"gemm {m}x{n}x{k} tile {tile}")
        qasr_attn.gemm_f16(g_ctx(), a, b, c, accumulate=accumulate)
        outs[tile] = c.cpu().numpy()
    monkeypatch.delenv("QASR_GEMM_TILE", raising=False)
    for tile in TILES:
        assert np.array_equal(outs[tile].view(np.uint16), outs[0].view(np.uint16)), tile
    ref = torch.mm(a.float(), b.float().t().contiguous())
    mag = torch.mm(a.float().abs(), b.float().abs().t().contiguous())
    if accumulate:
        ref, mag = ref + c0.float(), mag + c0.float().abs()
    ref = ref.cpu().numpy().astype(np.float64)
    bound = 0.5 * _f16_spacing(ref) + 2 * (k + 1) * 2.0 ** -24 * mag.cpu().numpy()
    assert np.all(np.abs(outs[0].astype(np.float64) - ref) <= bound)
