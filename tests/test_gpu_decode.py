"""Stage (b) decode attention on the GPU against the oracle
(cpu_decoder.rs:292-365 with one row; stage (a) per 398-423), at the BASELINE
decode configs and at edge lengths, plus invariants: fused step == stage (a)
then attention (bitwise), chunk-size independence, slot-permutation
invariance, appended rows bit-exact."""
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


# (minimum chunk keys, workgroup target): from the finest split the planner
# allows (32-key chunks, up to 256 per entry) through the default plan to one
# chunk per entry (no split-K, no merge), plus 8-wave workgroups.
CHUNK_PLANS = [("32", "4096", "4"), ("64", "512", "4"), ("256", "512", "4"),
               ("100000", "512", "4"), ("64", "512", "8")]


@pytest.mark.parametrize("min_chunk,wgs,waves", CHUNK_PLANS)
def test_decode_chunk_sizes_and_unfused_equal_fused(O, gpu, min_chunk, wgs, waves, monkeypatch):
    """Every split-K chunking matches the oracle; the unfused path
    (qasr_decode_attn on stage-(a) output) equals the fused step bitwise."""
    import qasr_attn
    from gpu_helpers import Gpu, dev, empty, host, say

    from oracle import Rng

    monkeypatch.setenv("QASR_DECODE_MIN_CHUNK", min_chunk)
    monkeypatch.setenv("QASR_DECODE_WGS", wgs)
    monkeypatch.setenv("QASR_DECODE_WAVES", waves)
    chunk = f"{min_chunk}/{wgs}/w{waves}"
    rng = Rng(SEED_BASE + 200 + int(min_chunk) % 1000 + int(waves))
    lay = Layer(rng)
    lengths = [1, 2, 127, 128, 129, 255, 256, 1023, 1024, 1500, 2047, 2048, 4095]
    cap = cap_for(max(lengths) + 1)
    n = len(lengths)
    g = Gpu(slots=n, cap=cap)
    refs = _setup(O, rng, lay, [L - 1 for L in lengths], cap, g)
    got_fused, rows, _ = _decode_step_check(O, rng, lay, g, refs, [L - 1 for L in lengths])
    # unfused: q from stage (a) (re-appending the same rows rewrites the same bits)
    q = g.append(0, lay, [(i, lengths[i] - 1, 1) for i in range(n)], rows)
    out = empty(n, QDIM)
    say(f"decode_attn unfused chunk={chunk}")
    qasr_attn.decode_attn(g.ctx, g.kv, 0, lengths, dev(q), out)
    assert np.array_equal(host(out), got_fused)
    g.close()


def test_decode_merge_past_16_chunks(O, gpu, monkeypatch):
    """Up to 64 chunks per entry (QASR_DECODE_MAX_SPLIT=64, 32-key chunks):
    the last arrival merges the partials in batches of 32, one round trip
    each, in chunk order -- the same oracle bound and fused/unfused equality."""
    monkeypatch.setenv("QASR_DECODE_MAX_SPLIT", "64")
    test_decode_chunk_sizes_and_unfused_equal_fused(O, gpu, "32", "4096", "4", monkeypatch)


def test_decode_partials_do_not_leak_between_launches(O, gpu, monkeypatch):
    """Split-K partial slots are shared by every launch on a pool and handed
    back unset by each launch's merger.  Steps that alternate planner settings
    (so a slot serves a different entry, kv head and chunk each time, or no
    split at all) each match the oracle, and a step repeated after them
    reproduces its first output bitwise."""
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
    for min_chunk, wgs, split in [("32", "4096", "64"), ("100000", "512", "32"),
                                  ("64", "97", "32"), ("128", "256", "5")]:
        monkeypatch.setenv("QASR_DECODE_MIN_CHUNK", min_chunk)
        monkeypatch.setenv("QASR_DECODE_WGS", wgs)
        monkeypatch.setenv("QASR_DECODE_MAX_SPLIT", split)
        say(f"decode leak check: plan {min_chunk}/{wgs}/{split}")
        _decode_step_check(O, rng, lay, g, refs, pos)
    for var in ("QASR_DECODE_MIN_CHUNK", "QASR_DECODE_WGS", "QASR_DECODE_MAX_SPLIT"):
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
