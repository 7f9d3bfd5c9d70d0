"""The library's launch planners on the host (qasr_plan_decode,
qasr_plan_prefill; no device needed): every key of every entry falls in
exactly one decode granule and one workgroup's run, granule sizes depend on
an entry's own length only (so its output bits do not depend on its batch
mates), the workgroup bases add up, and every prefill row block's key tiles
are covered by its splits -- over random batches, the knobs the GPU tests
drive, the bench configurations the documentation cites, and the refusals."""
from __future__ import annotations

import numpy as np
import pytest

import qasr_attn

NKVH = 8
SPLITMIX_SEED_CONFIG3 = 0x51A50000 + 3


def splitmix_lengths(seed: int, n: int, lo: int, hi: int):
    """bench.py's config-3 lengths (SplitMix64, U[lo, hi])."""
    state = seed & 0xFFFFFFFFFFFFFFFF
    out = []
    for _ in range(n):
        state = (state + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        z ^= z >> 31
        out.append(lo + z % (hi - lo + 1))
    return out


def granule(L: int, gmin: int = 0, gmax: int = 32) -> int:
    """The granule rule, restated: a multiple of 256 keys (two workgroup
    passes); by default 256 keys up to 1024 keys, 1024 up to 8192 and
    len / 32 beyond; with a forced gmin, the smallest multiple that is at
    least gmin and leaves at most gmax granules."""
    if gmin:
        want = max(gmin, -(-L // gmax))
    else:
        want = 256 if L <= 1024 else 1024 if L <= 8192 else -(-L // gmax)
    return -(-want // 256) * 256


def check_decode_plan(lens, plan, nkvh=NKVH, gmin=0, gmax=32):
    gran, run, base = plan
    assert base[0] == 0
    parts = 0
    for b, L in enumerate(lens):
        g, r = gran[b], run[b]
        assert g == granule(L, gmin, gmax), (b, L, g)
        ngr = -(-L // g)
        # granules [i g, min((i+1) g, L)) for i < ngr: none empty, none past L
        assert (ngr - 1) * g < L <= ngr * g and ngr <= 32
        assert 1 <= r <= min(ngr, 8)  # a run's wave partials fit the workgroup's LDS
        assert base[b + 1] - base[b] == nkvh * -(-ngr // r), (b, L, g, r)
        parts += nkvh * ngr
    assert parts <= 64 * nkvh * 32  # the workspace's partial records


@pytest.fixture(autouse=True)
def _no_knobs(monkeypatch):
    for v in ("QASR_DECODE_WGS", "QASR_DECODE_GRANULE", "QASR_DECODE_MAX_GRANULES",
              "QASR_DECODE_SPLIT", "QASR_PREFILL_TPS"):
        monkeypatch.delenv(v, raising=False)


def test_decode_plan_covers_every_key_random_batches():
    rng = np.random.default_rng(5)
    for _ in range(300):
        n = int(rng.integers(1, 65))
        lens = [int(x) for x in rng.integers(1, 16385, size=n)]
        plan = qasr_attn.plan_decode(lens, NKVH, 256)
        check_decode_plan(lens, plan)
        base = plan[2]
        assert base[-1] >= NKVH * n
        # the budget is one workgroup per CU unless the batch alone exceeds it
        # (or its runs would pass 8 granules)
        floor = sum(NKVH * -(-(-(-L // granule(L))) // 8) for L in lens)
        if NKVH * n < 256:
            assert base[-1] <= max(256, floor)


def test_decode_granules_do_not_depend_on_the_batch():
    """An entry's granules alone equal its granules in any batch and on any
    device: the property that makes --batch N byte-identical to --batch 1."""
    rng = np.random.default_rng(11)
    for _ in range(100):
        n = int(rng.integers(2, 65))
        lens = [int(x) for x in rng.integers(1, 16385, size=n)]
        gran, _, _ = qasr_attn.plan_decode(lens, NKVH, int(rng.integers(1, 512)))
        for b in range(0, n, 7):
            alone, _, _ = qasr_attn.plan_decode([lens[b]], NKVH, 256)
            assert alone[0] == gran[b]


def test_decode_plan_bench_configs():
    lens3 = [L + 1 for L in splitmix_lengths(SPLITMIX_SEED_CONFIG3, 16, 400, 2400)]
    gran, run, base = plan = qasr_attn.plan_decode(lens3, NKVH, 256)
    check_decode_plan(lens3, plan)
    assert gran == [1024 if L > 1024 else 256 for L in lens3]
    assert 240 <= base[-1] <= 256  # config 3: about one workgroup per CU
    gran, run, base = plan = qasr_attn.plan_decode([8193], NKVH, 256)
    assert gran == [512] and run == [1] and base == [0, 8 * 17]  # config 4: 17 granules
    gran, run, base = qasr_attn.plan_decode([512], NKVH, 256)
    assert gran == [256] and run == [1] and base == [0, 16]  # config 1: two granules
    lens = [1, 2, 255, 256, 257, 4096, 8192]
    gran, run, base = plan = qasr_attn.plan_decode(lens, NKVH, 256)
    check_decode_plan(lens, plan)
    assert gran == [256] * 5 + [1024] * 2 and base[-1] <= 256
    assert run[:4] == [1, 1, 1, 1]  # one granule each
    # a batch past the budget (64 entries x 8 kv heads) splits only its longest entries
    lens = [100] * 63 + [4000]
    gran, run, base = plan = qasr_attn.plan_decode(lens, NKVH, 256)
    check_decode_plan(lens, plan)
    assert base[:64] == [8 * i for i in range(64)] and base[-1] > 512


def test_decode_plan_knobs(monkeypatch):
    monkeypatch.setenv("QASR_DECODE_GRANULE", "768")
    lens = [8193, 130, 1000]
    plan = qasr_attn.plan_decode(lens, NKVH, 256)
    check_decode_plan(lens, plan, gmin=768)
    monkeypatch.setenv("QASR_DECODE_MAX_GRANULES", "4")
    plan = qasr_attn.plan_decode(lens, NKVH, 256)
    check_decode_plan(lens, plan, gmin=768, gmax=4)
    monkeypatch.setenv("QASR_DECODE_WGS", "8")  # past the budget: the greedy plan
    plan = qasr_attn.plan_decode(lens, NKVH, 256)
    check_decode_plan(lens, plan, gmin=768, gmax=4)
    plan = qasr_attn.plan_decode([3000, 3000], NKVH, 256)
    assert plan[1] == [4, 4]  # equal entries stay whole: one workgroup per (entry, kv head)
    monkeypatch.setenv("QASR_DECODE_GRANULE", "256")
    monkeypatch.delenv("QASR_DECODE_MAX_GRANULES")
    plan = qasr_attn.plan_decode([8000, 8000], NKVH, 256)
    assert plan[1] == [8, 8]  # whole entries, but a run holds at most 8 granules
    monkeypatch.setenv("QASR_DECODE_WGS", "4096")
    plan = qasr_attn.plan_decode(lens, NKVH, 256)
    assert plan[1] == [1, 1, 1]


def test_decode_plan_unsplit(monkeypatch):
    """QASR_DECODE_SPLIT=0: every (entry, kv head) on one workgroup (runs of
    up to 8 granules, the LDS limit), same granules as the split plan."""
    monkeypatch.setenv("QASR_DECODE_SPLIT", "0")
    rng = np.random.default_rng(13)
    for _ in range(50):
        n = int(rng.integers(1, 65))
        lens = [int(x) for x in rng.integers(1, 16385, size=n)]
        gran, run, base = plan = qasr_attn.plan_decode(lens, NKVH, 256)
        check_decode_plan(lens, plan)
        for b, L in enumerate(lens):
            assert run[b] == min(-(-L // gran[b]), 8)
        monkeypatch.delenv("QASR_DECODE_SPLIT")
        assert qasr_attn.plan_decode(lens, NKVH, 256)[0] == gran  # granules unchanged
        monkeypatch.setenv("QASR_DECODE_SPLIT", "0")


def test_decode_plan_refusals():
    for lens in ([], [0], [5, -1], [1] * 65):
        with pytest.raises(qasr_attn.QasrError):
            qasr_attn.plan_decode(lens, NKVH, 256)


def check_prefill_plan(rows, kv_start, p):
    rpb, nrb, tps, sp = p["rows_per_block"], p["nrb"], p["tiles_per_split"], p["sp_base"]
    assert rpb in (16, 32, 64) and tps >= 1
    assert nrb == -(-rows // rpb)
    assert sp[0] == 0 and len(sp) == nrb + 1
    for rb in range(nrb):
        kend = kv_start + min((rb + 1) * rpb, rows)
        tiles = -(-kend // 128)
        assert sp[rb + 1] - sp[rb] == -(-tiles // tps), (rows, kv_start, rb)
    if rpb < 64:  # 32- and 16-row blocks only for unsplit key ranges
        assert all(sp[rb + 1] - sp[rb] == 1 for rb in range(nrb))


def test_prefill_plan_covers_every_tile_random_launches():
    rng = np.random.default_rng(6)
    for _ in range(300):
        rows = int(rng.integers(1, 4097))
        kv_start = int(rng.integers(0, 12289))
        check_prefill_plan(rows, kv_start, qasr_attn.plan_prefill(rows, kv_start, NKVH))


def test_prefill_plan_fewest_tiles_per_split_within_256_items():
    """A split plan has at most 256 items over the kv heads, and one tile per
    split fewer would exceed that (the rounding of every row block counted);
    a plan past 256 items splits nothing."""
    rng = np.random.default_rng(7)
    for _ in range(400):
        rows = int(rng.integers(1, 4097))
        kv_start = int(rng.integers(0, 12289))
        p = qasr_attn.plan_prefill(rows, kv_start, NKVH)
        check_prefill_plan(rows, kv_start, p)
        if p["rows_per_block"] < 64:
            continue
        nrb, tps, items = p["nrb"], p["tiles_per_split"], p["sp_base"][-1]
        tiles = [-(-(kv_start + min((rb + 1) * 64, rows)) // 128) for rb in range(nrb)]
        if items > nrb:  # some row block split
            assert items * NKVH <= 256, (rows, kv_start, tps, items)
            if tps > 2:
                fewer = sum(-(-t // (tps - 1)) for t in tiles)
                assert fewer * NKVH > 256, (rows, kv_start, tps)
        else:
            assert tps >= max(tiles)
    p = qasr_attn.plan_prefill(1500, 2000, NKVH)  # 21 tiles per split would make 304 items
    assert (p["tiles_per_split"], p["sp_base"][-1] * NKVH) == (24, 256)


def test_prefill_plan_fits_the_noalloc_scratch_up_to_its_row_limit():
    """qasr_prefill_attn_noalloc runs qasr_prefill_attn's own plan out of a
    512-item scratch; its header's limit, s <= 64 * min(64, 256 / nkvh) rows,
    must keep every default plan within it, for every kv-head count."""
    rng = np.random.default_rng(8)
    for nkvh in (1, 2, 4, 8, 16):
        limit = 64 * min(64, 256 // nkvh)
        for rows in [1, 64, 65, 1024, limit] + [int(x) for x in rng.integers(1, limit + 1, 60)]:
            for kv_start in [0, 500, 7680, int(rng.integers(0, 12289))]:
                p = qasr_attn.plan_prefill(rows, kv_start, nkvh)
                assert p["sp_base"][-1] * nkvh <= 512, (nkvh, rows, kv_start, p["tiles_per_split"])


def test_prefill_plan_bench_configs(monkeypatch):
    p = qasr_attn.plan_prefill(420, 0, NKVH)  # config 2: 16-row blocks, 216 items
    assert (p["rows_per_block"], p["nrb"], p["tiles_per_split"]) == (16, 27, 4)
    assert p["sp_base"] == list(range(28))
    p = qasr_attn.plan_prefill(512, 7680, NKVH)  # config 4's last chunk: 4 splits of 16 tiles
    assert (p["rows_per_block"], p["nrb"], p["tiles_per_split"]) == (64, 8, 16)
    assert p["sp_base"][-1] * NKVH == 256
    p = qasr_attn.plan_prefill(512, 0, NKVH)  # 4 tiles: never split; 32 x 8 16-row items fit 256
    assert p["rows_per_block"] == 16 and p["sp_base"][-1] == 32
    p = qasr_attn.plan_prefill(520, 0, NKVH)  # 33 x 8 16-row items would not: 32-row blocks
    assert p["rows_per_block"] == 32 and p["sp_base"][-1] == 17
    p = qasr_attn.plan_prefill(1024, 0, NKVH)  # 8 tiles: never split
    assert p["rows_per_block"] == 32 and p["sp_base"][-1] == 32
    p = qasr_attn.plan_prefill(300, 724, NKVH)  # 8 tiles at kv_start 724: never split
    assert p["rows_per_block"] == 16 and p["sp_base"][-1] == 19
    p = qasr_attn.plan_prefill(1025, 0, NKVH)  # 9 tiles: 64-row blocks, split
    assert p["rows_per_block"] == 64 and p["sp_base"][-1] > p["nrb"]
    check_prefill_plan(1025, 0, p)
    monkeypatch.setenv("QASR_PREFILL_TPS", "3")
    p = qasr_attn.plan_prefill(420, 0, NKVH)
    assert (p["rows_per_block"], p["tiles_per_split"]) == (64, 3)
    check_prefill_plan(420, 0, p)


def test_prefill_plan_refusals():
    for rows, ks in ((0, 0), (4097, 0), (10, -1)):
        with pytest.raises(qasr_attn.QasrError):
            qasr_attn.plan_prefill(rows, ks, NKVH)
