"""qasr_prefill_attn_noalloc against qasr_prefill_attn.

The no-allocation entry point keeps its split-K partials in the library's
static per-GPU scratch array instead of the KV pool's workspace; with the
same launch plan its output must equal the allocating entry point's bit for
bit.  Two calls in a row (the second smaller, on another slot and position,
so stale scratch contents from the first would show), the refusal of a call
beyond the scratch's row limit, and the regular entry point still working
afterwards.
"""
from __future__ import annotations

import numpy as np
import pytest

from workloads import QDIM, SEED_BASE, TOT, Layer, OracleSeq, assert_parity, tables

pytestmark = pytest.mark.gpu


def test_noalloc_prefill_equals_allocating_prefill(O, gpu):
    import qasr_attn
    from gpu_helpers import Gpu, dev, empty, host, say

    from oracle import Rng

    rng = Rng(SEED_BASE + 1400)
    lay = Layer(rng)
    cap = 8448
    g = Gpu(slots=2, cap=cap)
    # slot 0: config 4's last chunk (512 rows at kv_start 7680, 4-way key
    # splits); slot 1: 300 rows at kv_start 1000 (smaller, other splits)
    cases = [(0, 7680, 512), (1, 1000, 300)]
    qs = {}
    for slot, kv_start, s in cases:
        pre = rng.normal_f16((kv_start + s, TOT))
        say(f"fill slot {slot}: {kv_start + s} rows")
        q_all = g.append(0, lay, [(slot, 0, kv_start + s)], pre)
        qs[slot] = (q_all[kv_start:], pre)
    for slot, kv_start, s in cases:
        q = dev(qs[slot][0])
        out_a, out_n = empty(s, QDIM), empty(s, QDIM)
        say(f"noalloc prefill slot {slot} kv_start {kv_start} s {s}")
        qasr_attn.prefill_attn_noalloc(g.ctx, g.kv, 0, slot, kv_start, s, q, out_n)
        say(f"allocating prefill slot {slot}")
        qasr_attn.prefill_attn(g.ctx, g.kv, 0, slot, kv_start, s, q, out_a)
        got_n, got_a = host(out_n), host(out_a)
        assert np.array_equal(got_n, got_a), f"slot {slot}: no-alloc output differs"
    # the second call's output also meets the oracle bound
    ref = OracleSeq(O, cap, lay, tables(O))
    q1, pre1 = qs[1]
    ref.append(pre1, 0)
    want = ref.attend(q1, 1000)
    assert_parity(got_n, want, "noalloc slot 1", p_f16=True)
    # beyond the scratch's row limit: refused before any launch
    big = empty(2049, QDIM)
    with pytest.raises(qasr_attn.QasrError) as e:
        qasr_attn.prefill_attn_noalloc(g.ctx, g.kv, 0, 0, 0, 2049, big, big)
    assert e.value.code == qasr_attn.QASR_EINVAL
    g.close()
