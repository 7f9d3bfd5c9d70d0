"""qasr_prefill_attn_noalloc against qasr_prefill_attn.

The no-allocation entry point keeps its split-K partials in the library's
static per-GPU scratch array instead of the KV pool's workspace.  Up to its
row limit every default plan fits that array, so it runs exactly the
allocating entry point's work items and its output must equal that entry
point's bit for bit.  The calls run on a fresh pool (one that never grew a
prefill workspace), twice: the first pass lets the runtime load the
kernels' code, and the device's free memory must not move over the second.
Five calls in a row (later ones smaller or elsewhere, so stale scratch
contents from an earlier one would show), among them 192 rows at kv_start
8000 (a plan with more work items than the row blocks times kv heads
suggest), the row limit itself and an unsplit 16-row plan; the refusal of a
call beyond the limit; and the regular entry point still working afterwards.
"""
from __future__ import annotations

import numpy as np
import pytest

from workloads import QDIM, SEED_BASE, TOT, Layer, OracleSeq, assert_parity, tables

pytestmark = pytest.mark.gpu


def test_noalloc_prefill_equals_allocating_prefill(O, gpu):
    import torch

    import qasr_attn
    from gpu_helpers import Gpu, dev, empty, host, say

    from oracle import Rng

    rng = Rng(SEED_BASE + 1400)
    lay = Layer(rng)
    cap = 8448
    g = Gpu(slots=5, cap=cap)
    # slot 0: config 4's last chunk (512 rows at kv_start 7680, 4-way key
    # splits); slot 1: 300 rows at kv_start 1000 (smaller, other splits);
    # slot 2: 192 rows at 8000; slot 3: 2048 rows from 0 (the row limit);
    # slot 4: 300 rows from 0 (unsplit 16-row blocks on four waves)
    cases = [(0, 7680, 512), (1, 1000, 300), (2, 8000, 192), (3, 0, 2048), (4, 0, 300)]
    assert qasr_attn.plan_prefill(300, 0, 8)["rows_per_block"] == 16
    qs = {}
    for slot, kv_start, s in cases:
        pre = rng.normal_f16((kv_start + s, TOT))
        say(f"fill slot {slot}: {kv_start + s} rows")
        q_all = g.append(0, lay, [(slot, 0, kv_start + s)], pre)
        qs[slot] = (dev(q_all[kv_start:]), pre)
    outs_n = {slot: empty(s, QDIM) for slot, _, s in cases}
    # A first pass: the HIP runtime loads a kernel's code on its first launch
    # in the process (device memory of its own, once per process, not the
    # entry point's), so free memory is compared across a second pass.
    for slot, kv_start, s in cases:
        say(f"noalloc prefill (first pass) slot {slot} kv_start {kv_start} s {s}")
        qasr_attn.prefill_attn_noalloc(g.ctx, g.kv, 0, slot, kv_start, s, qs[slot][0], outs_n[slot])
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for slot, kv_start, s in cases:
        say(f"noalloc prefill slot {slot} kv_start {kv_start} s {s}")
        qasr_attn.prefill_attn_noalloc(g.ctx, g.kv, 0, slot, kv_start, s, qs[slot][0], outs_n[slot])
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0, "the no-allocation calls allocated device memory"
    for slot, kv_start, s in cases:
        out_a = empty(s, QDIM)
        say(f"allocating prefill slot {slot}")
        qasr_attn.prefill_attn(g.ctx, g.kv, 0, slot, kv_start, s, qs[slot][0], out_a)
        got_n, got_a = host(outs_n[slot]), host(out_a)
        assert np.array_equal(got_n, got_a), f"slot {slot}: no-alloc output differs"
    # the 192-row call also meets the oracle bound
    ref = OracleSeq(O, cap, lay, tables(O))
    q2, pre2 = qs[2]
    ref.append(pre2, 0)
    want = ref.attend(host(q2), 8000)
    assert_parity(host(outs_n[2]), want, "noalloc slot 2", p_f16=True)
    # beyond the scratch's row limit: refused before any launch
    big = empty(2049, QDIM)
    with pytest.raises(qasr_attn.QasrError) as e:
        qasr_attn.prefill_attn_noalloc(g.ctx, g.kv, 0, 0, 0, 2049, big, big)
    assert e.value.code == qasr_attn.QASR_EINVAL
    g.close()
