"""Stage (a) on the GPU -- fused q/k RMSNorm + MRoPE + f16 KV append -- is
bit-identical to the oracle (cpu_decoder.rs:274-290, 398-423): roped Q, the
K rows written to the cache and the V rows copied, for prefill segments,
decode batches (one row per slot) and chunked segments at kv_start > 0."""
from __future__ import annotations

import numpy as np
import pytest

from workloads import HD, NKVH, SEED_BASE, TOT, Layer, OracleSeq, tables

pytestmark = pytest.mark.gpu


def test_stage_a_prefill_config2_bitexact(O, gpu):
    from gpu_helpers import Gpu, say

    from oracle import Rng

    rng = Rng(SEED_BASE + 2)
    lay = Layer(rng)
    s = 420
    qkv = rng.normal_f16((s, TOT))
    say(f"stage_a prefill s={s}")
    g = Gpu(slots=1, cap=1024)
    q_gpu = g.append(0, lay, [(0, 0, s)], qkv)
    ref = OracleSeq(O, 1024, lay, tables(O))
    q_ref = ref.append(qkv, 0)
    assert np.array_equal(q_gpu, q_ref)
    k_gpu, v_gpu = g.cache(0, 0, s)
    k_ref, v_ref = ref.cache_f16()
    assert np.array_equal(k_gpu, k_ref[:, :s])
    assert np.array_equal(v_gpu, v_ref[:, :s])
    g.close()


def test_stage_a_decode_batch_and_chunks_bitexact(O, gpu):
    from gpu_helpers import Gpu, say

    from oracle import Rng

    rng = Rng(SEED_BASE + 100)
    lay = Layer(rng)
    slots, cap, layers = 5, 4352, 3
    g = Gpu(slots=slots, cap=cap, layers=layers)
    refs = [OracleSeq(O, cap, lay, tables(O)) for _ in range(slots)]
    # chunked prefill per slot at growing offsets, into layer 2
    pos = [0] * slots
    for rnd, size in enumerate((37, 1, 300, 129)):
        segs, rows = [], []
        for sl in range(slots):
            n = size + sl
            segs.append((sl, pos[sl], n))
            rows.append(rng.normal_f16((n, TOT), 0.0, 1.0 + 0.5 * sl))
        qkv = np.concatenate(rows)
        say(f"stage_a segments round {rnd} rows={qkv.shape[0]}")
        q_gpu = g.append(2, lay, segs, qkv)
        q_ref = np.concatenate([refs[sl].append(rows[sl], pos[sl]) for sl in range(slots)])
        assert np.array_equal(q_gpu, q_ref)
        for sl in range(slots):
            pos[sl] += size + sl
    # a decode batch at the end: one row per slot, slots in scrambled order
    order = [3, 0, 4, 1, 2]
    rows = rng.normal_f16((slots, TOT))
    say("stage_a decode batch")
    q_gpu = g.append(2, lay, [(sl, pos[sl], 1) for sl in order], rows)
    q_ref = np.concatenate([refs[sl].append(rows[i:i + 1], pos[sl]) for i, sl in enumerate(order)])
    assert np.array_equal(q_gpu, q_ref)
    for sl in range(slots):
        n = pos[sl] + 1
        k_gpu, v_gpu = g.cache(sl, 2, n)
        k_ref, v_ref = refs[sl].cache_f16()
        assert np.array_equal(k_gpu, k_ref[:, :n]), sl
        assert np.array_equal(v_gpu, v_ref[:, :n]), sl
        # the other layers were not touched
        k0, v0 = g.cache(sl, 0, n)
        assert not k0.any() and not v0.any()
    g.close()


def test_stage_a_extreme_inputs_bitexact(O, gpu):
    """Large, tiny and subnormal-producing rows round exactly like the oracle."""
    from gpu_helpers import Gpu, say

    from oracle import Rng

    rng = Rng(SEED_BASE + 101)
    lay = Layer(rng)
    rows = []
    for scale in (1e-4, 1e-2, 1.0, 30.0, 3000.0):
        rows.append(rng.normal_f16((4, TOT), 0.0, scale))
    z = np.zeros((1, TOT), np.uint16)  # all-zero heads: inv = 1/sqrt(eps)
    qkv = np.concatenate(rows + [z])
    n = qkv.shape[0]
    say(f"stage_a extremes rows={n}")
    g = Gpu(slots=1, cap=1024)
    q_gpu = g.append(0, lay, [(0, 5000 - 1024 * 4, n)], qkv)
    ref = OracleSeq(O, 1024, lay, tables(O))
    q_ref = ref.append(qkv, 5000 - 1024 * 4)
    assert np.array_equal(q_gpu, q_ref)
    k_gpu, _ = g.cache(0, 0, 1024)
    k_ref, _ = ref.cache_f16()
    assert np.array_equal(k_gpu, k_ref)
    g.close()
