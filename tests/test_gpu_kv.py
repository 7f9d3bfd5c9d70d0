"""KV pool behaviour and error handling on the GPU: grow-with-copy keeps the
written rows bit for bit (decoder.rs:1617-1650), growth is grow-only and
KV_STEP granular, and every bounds violation the reference rejects
(cpu_decoder.rs:489-495, 520; decoder.rs:4500-4530) comes back as a status
code before any kernel runs."""
from __future__ import annotations

import numpy as np
import pytest

from workloads import QDIM, SEED_BASE, TOT, Layer

pytestmark = pytest.mark.gpu


def test_ensure_capacity_keeps_rows(O, gpu):
    from gpu_helpers import Gpu, say

    from oracle import Rng

    rng = Rng(SEED_BASE + 700)
    lay = Layer(rng)
    g = Gpu(slots=3, cap=1024, layers=2)
    rows = rng.normal_f16((3 * 700, TOT))
    say("fill before growth")
    g.append(1, lay, [(0, 0, 700), (1, 0, 700), (2, 0, 700)], rows)
    before = [g.cache(sl, 1, 700) for sl in range(3)]
    assert g.kv.ensure_capacity(1000, 700) == 1024  # fits: unchanged
    say("grow 1024 -> 2560")
    assert g.kv.ensure_capacity(2400, 700) == 2560
    assert g.kv.cap == 2560
    for sl in range(3):
        k, v = g.cache(sl, 1, 2560)
        assert np.array_equal(k[:, :700], before[sl][0]) and np.array_equal(v[:, :700], before[sl][1])
        assert not k[:, 700:].any() and not v[:, 700:].any()
    assert g.kv.ensure_capacity(100, 700) == 2560  # grow-only
    assert g.kv.ensure_capacity(10 ** 6, 700) == 16384  # clamped to max_seq
    g.close()


def test_errors_before_launch(O, gpu):
    import qasr_attn
    from gpu_helpers import Gpu, dev, empty

    from oracle import Rng

    rng = Rng(SEED_BASE + 701)
    lay = Layer(rng)
    g = Gpu(slots=2, cap=1024, max_seq=2000)
    qg, kg = g.gains(lay)
    q = empty(2, QDIM)
    out = empty(2, QDIM)
    row = dev(rng.normal_f16((2, TOT)))
    # buffers sized for the refused calls' rows: the binding refuses an
    # undersized tensor itself (EINVAL), and these checks are about the
    # library's own range checks
    q40, out40 = empty(40, QDIM), empty(40, QDIM)
    row40 = dev(rng.normal_f16((40, TOT)))
    E = qasr_attn.QasrError

    def code(fn):
        with pytest.raises(E) as e:
            fn()
        return e.value.code

    assert code(lambda: qasr_attn.decode_attn(g.ctx, g.kv, 0, [1025, 3], q, out)) == qasr_attn.QASR_ERANGE
    assert code(lambda: qasr_attn.decode_attn(g.ctx, g.kv, 0, [0, 3], q, out)) == qasr_attn.QASR_EINVAL
    assert code(lambda: qasr_attn.decode_attn(g.ctx, g.kv, 0, [4, 3], q, out, slots=[0, 2])) == qasr_attn.QASR_EINVAL
    assert code(lambda: qasr_attn.decode_attn(g.ctx, g.kv, 1, [4, 3], q, out)) == qasr_attn.QASR_EINVAL
    assert code(lambda: qasr_attn.decode_step(g.ctx, g.kv, 0, [1024, 3], row, qg, kg, out)) == qasr_attn.QASR_ERANGE
    assert code(lambda: qasr_attn.decode_step(g.ctx, g.kv, 0, [4, 3], row, qg, kg, out, slots=[1, 1])) == qasr_attn.QASR_EINVAL
    assert code(lambda: qasr_attn.prefill_attn(g.ctx, g.kv, 0, 0, 1000, 30, q40, out40)) == qasr_attn.QASR_ERANGE
    assert code(lambda: qasr_attn.prefill_attn(g.ctx, g.kv, 0, 5, 0, 1, q, out)) == qasr_attn.QASR_EINVAL
    assert code(lambda: qasr_attn.qk_norm_rope_append(g.ctx, g.kv, 0, [(0, 1020, 10)], row40, qg, kg, q40)) == qasr_attn.QASR_ERANGE
    # beyond max_seq after growth
    assert g.kv.ensure_capacity(5000, 0) == 2000
    assert code(lambda: qasr_attn.decode_step(g.ctx, g.kv, 0, [2000, 3], row, qg, kg, out)) == qasr_attn.QASR_ERANGE
    assert code(lambda: qasr_attn.prefill_attn(g.ctx, g.kv, 0, 0, 1990, 11, q40, out40)) == qasr_attn.QASR_ERANGE
    # undersized, wrong dtype or host tensors never reach the library
    import torch

    assert code(lambda: qasr_attn.prefill_attn(g.ctx, g.kv, 0, 0, 0, 30, q, out)) == qasr_attn.QASR_EINVAL

    with pytest.raises(ValueError):
        qasr_attn.decode_attn(g.ctx, g.kv, 0, [4, 3], q.float(), out)
    with pytest.raises(ValueError):
        qasr_attn.decode_attn(g.ctx, g.kv, 0, [4, 3], q.cpu(), out)
    # tables missing -> ESTATE
    ctx2 = qasr_attn.Context(layers=1)
    kv2 = qasr_attn.KVPool(ctx2, 1, 256)
    assert code(lambda: qasr_attn.decode_step(ctx2, kv2, 0, [3], row[:1], qg, kg, out[:1])) == qasr_attn.QASR_ESTATE
    # a pool used with the wrong context
    assert code(lambda: qasr_attn.decode_attn(ctx2, g.kv, 0, [4], q[:1], out[:1])) == qasr_attn.QASR_EINVAL
    torch.cuda.synchronize()
    kv2.close()
    ctx2.close()
    g.close()


def test_backend_mirror_prefill_then_steps(O, gpu):
    """AttnBackend keeps the reference's TextBackend call sequence:
    set_rope_tables -> ensure_capacity -> prefill -> step -> step."""
    import qasr_attn
    from gpu_helpers import dev, host, rope_tables

    from oracle import Rng
    from workloads import OracleSeq, assert_parity, tables

    rng = Rng(SEED_BASE + 702)
    lay = Layer(rng)
    be = qasr_attn.AttnBackend(layers=1, slots=2, cap=1024)
    be.set_rope_tables(*rope_tables())
    assert be.ensure_capacity(1500) == 1536
    prompt = rng.normal_f16((900, TOT))
    qg, kg = dev(lay.q_gain), dev(lay.k_gain)
    out = host(be.prefill(0, dev(prompt), 900, 0, qg, kg, slot=1))
    ref = OracleSeq(O, 1536, lay, tables(O))
    _, want = ref.step(prompt, 0)
    assert_parity(out, want, "backend prefill", p_f16=True)
    for _ in range(2):
        row = rng.normal_f16((1, TOT))
        p = be.pos[1]
        got = host(be.step(0, dev(row), qg, kg, slots=[1]))
        _, want = ref.step(row, p)
        assert_parity(got, want, "backend step")
    assert be.pos == [0, 902]


def test_growth_during_pipelined_steps_on_a_side_stream(O, gpu):
    """The pool grows (1024 -> 1280 rows) from step_async while the previous
    step, queued on a non-default torch stream, may still be appending row
    pos-1: every row written before and after the growth equals, bit for
    bit, the same steps run on a pool that never grows."""
    import torch

    import qasr_attn
    from decoder_model import CFG_0P6B, synth_weights
    from gpu_helpers import say

    cfg = dict(CFG_0P6B, layers=2, vocab=4096)
    W = synth_weights(cfg, SEED_BASE + 710, device="cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(SEED_BASE + 711)
    prompt = torch.randn((1016, cfg["hs"]), device="cuda", generator=g).half()
    steps = 20  # positions 1016 .. 1035: crosses the 1024-row capacity
    runs = []
    for cap in (1024, 2048):
        dec = qasr_attn.TextDecoder(W, cfg["nqh"], cfg["nkvh"], cfg["hd"], cfg["layers"],
                                    cfg["eps"], cfg["max_seq"], slots=1, max_rows=1024, cap=cap)
        dec.prefill(prompt, 0)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        toks = []
        say(f"pipelined steps from cap {cap}")
        with torch.cuda.stream(side):
            h = dec.step_async([0])
            for _ in range(steps - 1):
                h_next = dec.step_async([0])  # may grow the pool: h is in flight
                toks += dec.step_result(h)
                h = h_next
            toks += dec.step_result(h)
        torch.cuda.synchronize()
        end = 1016 + steps
        kv = dec.kv.tensor()[0, :, :, :, :end].clone()
        runs.append((dec.kv.cap, toks, kv))
        dec.close()
    (cap_a, toks_a, kv_a), (cap_b, toks_b, kv_b) = runs
    assert cap_a == 1280 and cap_b == 2048
    assert toks_a == toks_b
    assert torch.equal(kv_a, kv_b), "rows differ after growth during a pipelined step"
