"""Stage (b) decode attention on the GPU against the oracle
(cpu_decoder.rs:292-365 with one row; stage (a) per 398-423), at the BASELINE
decode configs and at edge lengths, plus invariants: fused step == stage (a)
then attention (bitwise), every granule and run plan within the bound, an
entry's output bits independent of its batch mates, slot order and the
workgroup budget (--batch N == --batch 1), appended rows bit-exact."""
from __future__ import annotations

import os

import numpy as np
import pytest

from workloads import (NKVH, QDIM, SEED_BASE, TOT, Layer, OracleSeq, assert_parity, cap_for,
                       decode_lengths, tables)

pytestmark = pytest.mark.gpu


def _setup(O, rng, lay, lengths, cap, g, layer=0):
    """Fill each slot's cache with positions 0..L-1 (GPU by stage (a), oracle by
    its restatement) from the same raw rows; returns the oracle sequences."""
    from gpu_helpers import say

    refs = []
    for sl, L in enumerate(lengths):
        ref = OracleSeq(O, cap, lay, tables(O))
        if L > 0:
            rows = rng.normal_f16((L, TOT))
            ref.append(rows, 0)
            say(f"fill slot {sl} L={L}")
            g.append(layer, lay, [(sl, 0, L)], rows)
        refs.append(ref)
    return refs


def _decode_step_check(O, rng, lay, g, refs, lengths, layer=0, slots=None):
    """One fused step at pos = L per slot; compares with the oracle step."""
    import qasr_attn
    from gpu_helpers import dev, empty, host, say

    b = len(lengths)
    slots = list(range(b)) if slots is None else slots
    rows = rng.normal_f16((b, TOT))
    out = empty(b, QDIM)
    qg, kg = g.gains(lay)
    say(f"decode_step batch={b} lengths[:4]={lengths[:4]}")
    qasr_attn.decode_step(g.ctx, g.kv, layer, [lengths[i] for i in range(b)], dev(rows), qg, kg,
                          out, slots=slots)
    got = host(out)
    worst = (0.0, 0.0)
    for i in range(b):
        sl = slots[i]
        _, want = refs[sl].step(rows[i:i + 1], lengths[i])
        ma, mr = assert_parity(got[i:i + 1], want, f"entry {i} slot {sl} L={lengths[i] + 1}")
        worst = (max(worst[0], ma), max(worst[1], mr))
        # the appended row is bit-exact
        k_gpu, v_gpu = g.cache_row(sl, layer, lengths[i])
        k_ref, v_ref = refs[sl].row_f16(lengths[i])
        assert np.array_equal(k_gpu, k_ref)
        assert np.array_equal(v_gpu, v_ref)
    return got, rows, worst


def test_config1_single_slot_decode(O, gpu):
    from gpu_helpers import Gpu

    from oracle import Rng

    rng = Rng(SEED_BASE + 1)
    lay = Layer(rng)
    g = Gpu(slots=1, cap=1024)
    refs = _setup(O, rng, lay, [511], 1024, g)
    _, _, worst = _decode_step_check(O, rng, lay, g, refs, [511])
    print("config1 max_abs/max_rel", worst)
    g.close()


def test_config3_batch16_ragged_decode(O, gpu):
    from gpu_helpers import Gpu

    from oracle import Rng

    rng = Rng(SEED_BASE + 3)
    lengths = decode_lengths(rng, 16, 400, 2400)  # drawn first, as bench.py does
    lay = Layer(rng)
    cap = cap_for(max(lengths) + 1)
    g = Gpu(slots=16, cap=cap)
    refs = _setup(O, rng, lay, lengths, cap, g)
    _, _, worst = _decode_step_check(O, rng, lay, g, refs, lengths)
    print("config3 max_abs/max_rel", worst)
    g.close()


# (minimum granule keys, workgroup budget, granules per entry at most): from
# the finest granules (256 keys, one workgroup each) through the default plan
# to one granule per entry (no merge), runs of many granules whose partials
# are published for another workgroup's merge, and the greedy plan of a small
# budget where most (entry, kv head) pairs run whole in one workgroup and
# merge in LDS.
GRANULE_PLANS = [("256", "4096", "32"), ("512", "256", "32"), ("256", "64", "32"),
                 ("100000", "512", "32"), ("256", "8", "32"), ("256", "40", "6")]


@pytest.mark.parametrize("gran,wgs,gmax", GRANULE_PLANS)
def test_decode_plans_and_unfused_equal_fused(O, gpu, gran, wgs, gmax, monkeypatch):
    """Every granule and run plan matches the oracle; the unfused path
    (qasr_decode_attn on stage-(a) output) equals the fused step bitwise."""
    import qasr_attn
    from gpu_helpers import Gpu, dev, empty, host, say

    from oracle import Rng

    monkeypatch.setenv("QASR_DECODE_GRANULE", gran)
    monkeypatch.setenv("QASR_DECODE_WGS", wgs)
    monkeypatch.setenv("QASR_DECODE_MAX_GRANULES", gmax)
    plan = f"{gran}/{wgs}/{gmax}"
    rng = Rng(SEED_BASE + 200 + int(gran) % 1000 + int(wgs) % 97)
    lay = Layer(rng)
    # 8000 keys: 32 granules of 256 (the merge's largest batch)
    lengths = [1, 2, 127, 128, 129, 255, 256, 1023, 1024, 1500, 2047, 2048, 4095, 8000]
    cap = cap_for(max(lengths) + 1)
    n = len(lengths)
    g = Gpu(slots=n, cap=cap)
    refs = _setup(O, rng, lay, [L - 1 for L in lengths], cap, g)
    say(f"decode plan {plan}: {qasr_attn.plan_decode(lengths, NKVH, 256)}")
    got_fused, rows, _ = _decode_step_check(O, rng, lay, g, refs, [L - 1 for L in lengths])
    # unfused: q from stage (a) (re-appending the same rows rewrites the same bits)
    q = g.append(0, lay, [(i, lengths[i] - 1, 1) for i in range(n)], rows)
    out = empty(n, QDIM)
    say(f"decode_attn unfused plan={plan}")
    qasr_attn.decode_attn(g.ctx, g.kv, 0, lengths, dev(q), out)
    assert np.array_equal(host(out), got_fused)
    g.close()


def test_decode_output_independent_of_batch_mates(O, gpu, monkeypatch):
    """--batch N == --batch 1 for attention: each entry decoded alone, inside
    two different batches (other slots, other order), under other workgroup
    budgets and with the split off gives the same bits, on the unfused and
    the fused path.
    The granule plan depends on an entry's own length only; the batch and the
    device change only which workgroup runs which granules."""
    import qasr_attn
    from gpu_helpers import Gpu, dev, empty, host, say

    from oracle import Rng

    rng = Rng(SEED_BASE + 960)
    lay = Layer(rng)
    lengths = [5, 300, 700, 1500, 2047, 2600, 3333, 7000, 129, 1024, 256, 3900]
    n = len(lengths)
    cap = cap_for(max(lengths) + 1)
    g = Gpu(slots=n, cap=cap)
    refs = _setup(O, rng, lay, [L - 1 for L in lengths], cap, g)
    rows = rng.normal_f16((n, TOT))
    q = g.append(0, lay, [(i, lengths[i] - 1, 1) for i in range(n)], rows)
    qg, kg = g.gains(lay)

    def attn(slots, wgs=None):
        if wgs is None:
            monkeypatch.delenv("QASR_DECODE_WGS", raising=False)
        else:
            monkeypatch.setenv("QASR_DECODE_WGS", str(wgs))
        out = empty(len(slots), QDIM)
        qasr_attn.decode_attn(g.ctx, g.kv, 0, [lengths[s] for s in slots], dev(q[slots]), out,
                              slots=slots)
        return host(out)

    def step(slots, wgs=None):
        if wgs is None:
            monkeypatch.delenv("QASR_DECODE_WGS", raising=False)
        else:
            monkeypatch.setenv("QASR_DECODE_WGS", str(wgs))
        out = empty(len(slots), QDIM)
        qasr_attn.decode_step(g.ctx, g.kv, 0, [lengths[s] - 1 for s in slots], dev(rows[slots]),
                              qg, kg, out, slots=slots)
        return host(out)

    batch_a = [3, 0, 7, 5]
    batch_b = [11, 6, 2, 9, 4, 1, 10, 8, 3, 7, 0, 5]
    say("decode batch invariance: alone, two batches, three budgets")
    alone = {s: attn([s]) for s in range(n)}
    for i in range(n):
        _, want = refs[i].step(rows[i:i + 1], lengths[i] - 1)
        assert_parity(alone[i], want, f"slot {i} alone")
    for slots, wgs in [(batch_a, None), (batch_b, None), (batch_b, 64), (batch_a, 1000)]:
        got = attn(slots, wgs)
        for k, s in enumerate(slots):
            assert np.array_equal(got[k:k + 1], alone[s]), (slots, wgs, s)
    monkeypatch.setenv("QASR_DECODE_SPLIT", "0")  # every (entry, kv head) on one workgroup
    got = attn(batch_b)
    monkeypatch.delenv("QASR_DECODE_SPLIT")
    for k, s in enumerate(batch_b):
        assert np.array_equal(got[k:k + 1], alone[s]), ("unsplit", s)
    step_alone = {s: step([s]) for s in (3, 7, 11)}
    for slots in (batch_a, batch_b):
        got = step(slots, 100)
        for k, s in enumerate(slots):
            if s in step_alone:
                assert np.array_equal(got[k:k + 1], step_alone[s]), (slots, s)
            assert np.array_equal(got[k:k + 1], alone[s]), (slots, s)
    g.close()


def test_decode_partials_do_not_leak_between_launches(O, gpu, monkeypatch):
    """Split-K partial slots are shared by every launch on a pool and the
    arrival counters are handed back at zero by each launch's merger.  Steps
    that alternate planner settings (so a slot serves a different entry, kv
    head and granule each time, or no split at all) each match the oracle,
    and a step repeated after them reproduces its first output bitwise."""
    import qasr_attn
    from gpu_helpers import Gpu, dev, empty, host, say

    from oracle import Rng

    rng = Rng(SEED_BASE + 940)
    lay = Layer(rng)
    lengths = [1500, 700, 2047, 129, 3000, 900, 2, 1024]
    n = len(lengths)
    cap = cap_for(max(lengths) + 1)
    g = Gpu(slots=n, cap=cap)
    pos = [L - 1 for L in lengths]
    refs = _setup(O, rng, lay, pos, cap, g)
    qg, kg = g.gains(lay)

    def step_rows(rows):
        out = empty(n, QDIM)
        qasr_attn.decode_step(g.ctx, g.kv, 0, pos, dev(rows), qg, kg, out)
        return host(out)

    rows0 = rng.normal_f16((n, TOT))
    say("decode leak check: first step, default plan")
    first = step_rows(rows0)
    for i in range(n):
        _, want = refs[i].step(rows0[i:i + 1], pos[i])
        assert_parity(first[i:i + 1], want, f"first step entry {i}")
    for gran, wgs, gmax in [("256", "4096", "32"), ("100000", "512", "32"),
                            ("256", "97", "32"), ("768", "256", "5"), ("256", "20", "32")]:
        monkeypatch.setenv("QASR_DECODE_GRANULE", gran)
        monkeypatch.setenv("QASR_DECODE_WGS", wgs)
        monkeypatch.setenv("QASR_DECODE_MAX_GRANULES", gmax)
        say(f"decode leak check: plan {gran}/{wgs}/{gmax}")
        _decode_step_check(O, rng, lay, g, refs, pos)
    for var in ("QASR_DECODE_GRANULE", "QASR_DECODE_WGS", "QASR_DECODE_MAX_GRANULES"):
        monkeypatch.delenv(var)
    say("decode leak check: repeated first step")
    again = step_rows(rows0)
    assert np.array_equal(again, first)
    g.close()


def test_decode_cap_length_and_permuted_slots(O, gpu):
    """cur_len == cap; slot order in the batch does not change any slot's output."""
    import qasr_attn
    from gpu_helpers import Gpu, dev, empty, host, say

    from oracle import Rng

    rng = Rng(SEED_BASE + 300)
    lay = Layer(rng)
    cap = 1280
    lengths = [cap - 1, 5, 700, 1000]
    g = Gpu(slots=4, cap=cap)
    refs = _setup(O, rng, lay, lengths, cap, g)
    got, rows, _ = _decode_step_check(O, rng, lay, g, refs, lengths)
    q = g.append(0, lay, [(i, lengths[i], 1) for i in range(4)], rows)
    perm = [2, 0, 3, 1]
    out = empty(4, QDIM)
    say("decode_attn permuted slots")
    qasr_attn.decode_attn(g.ctx, g.kv, 0, [lengths[p] + 1 for p in perm], dev(q[perm]), out,
                          slots=perm)
    assert np.array_equal(host(out), got[perm])
    g.close()


def test_config5_64_slots_all_layers(O, gpu):
    """Config 5: 64 slots, ragged [64, 4096], the fused step of all 28 layers.
    Layer 0's caches are filled through stage (a) on both sides; every other
    layer's caches are device copies of them (the oracle reuses its arrays),
    and each layer then steps with its own gains and raw qkv rows, so each of
    the 28 launches reads its own cache region and appends its own row."""
    from gpu_helpers import Gpu, say

    from oracle import Rng

    rng = Rng(SEED_BASE + 5)
    lengths = decode_lengths(rng, 64, 64, 4096)
    cap = cap_for(max(lengths) + 1)
    layers = 28
    g = Gpu(slots=64, cap=cap, layers=layers)
    lay0 = Layer(rng)
    refs = _setup(O, rng, lay0, lengths, cap, g, layer=0)
    pool = g.kv.tensor()
    for layer in range(1, layers):
        pool[:, layer].copy_(pool[:, 0])
    worst = (0.0, 0.0)
    for layer in range(layers):
        lay = lay0 if layer == 0 else Layer(rng)
        for ref in refs:
            ref.layer = lay
        say(f"config5 layer {layer}")
        _, _, w = _decode_step_check(O, rng, lay, g, refs, lengths, layer=layer)
        worst = (max(worst[0], w[0]), max(worst[1], w[1]))
    print("config5 max_abs/max_rel", worst)
    g.close()


def test_decode_long_context_split(O, gpu):
    """Config 4's decode side: one slot at 8192 cached keys, the workload's
    64 consecutive steps (positions 8192..8255)."""
    from gpu_helpers import Gpu

    from oracle import Rng

    rng = Rng(SEED_BASE + 4)
    lay = Layer(rng)
    L0 = 8192
    cap = cap_for(L0 + 64)
    g = Gpu(slots=1, cap=cap)
    refs = _setup(O, rng, lay, [L0], cap, g)
    for step in range(64):
        _decode_step_check(O, rng, lay, g, refs, [L0 + step])
    g.close()
