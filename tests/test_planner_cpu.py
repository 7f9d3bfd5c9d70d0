"""The library's launch planners on the host (qasr_plan_decode,
qasr_plan_prefill; no device needed): every key of every entry falls in
exactly one decode workgroup's chunk, chunks are whole 32-key passes, the
workgroup bases add up, and every prefill row block's key tiles are covered
by its splits -- over random batches, the knobs the GPU tests drive, the
bench configurations the documentation cites, and the refusals."""
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


def check_decode_plan(lens, chunk, base, max_split=32, nkvh=NKVH):
    assert base[0] == 0
    for b, L in enumerate(lens):
        c = chunk[b]
        assert c >= 32 and c % 32 == 0, (b, c)
        nch = -(-L // c)
        # chunks [j c, min((j+1) c, L)) for j < nch: none empty, none past L
        assert (nch - 1) * c < L <= nch * c
        assert nch <= max_split
        assert base[b + 1] - base[b] == nkvh * nch, (b, L, c)
    assert base[-1] <= 8192


@pytest.fixture(autouse=True)
def _no_knobs(monkeypatch):
    for v in ("QASR_DECODE_WGS", "QASR_DECODE_MIN_CHUNK", "QASR_DECODE_MAX_SPLIT", "QASR_PREFILL_TPS"):
        monkeypatch.delenv(v, raising=False)


def test_decode_plan_covers_every_key_random_batches():
    rng = np.random.default_rng(5)
    for _ in range(300):
        n = int(rng.integers(1, 65))
        lens = [int(x) for x in rng.integers(1, 16385, size=n)]
        chunk, base = qasr_attn.plan_decode(lens, NKVH, 256)
        check_decode_plan(lens, chunk, base)
        # the budget is one workgroup per CU unless the batch alone exceeds it
        assert base[-1] >= NKVH * n
        if NKVH * n < 256:
            assert base[-1] <= 256


def test_decode_plan_bench_configs():
    lens3 = splitmix_lengths(SPLITMIX_SEED_CONFIG3, 16, 400, 2400)
    chunk, base = qasr_attn.plan_decode([L + 1 for L in lens3], NKVH, 256)
    check_decode_plan([L + 1 for L in lens3], chunk, base)
    assert base[-1] == 256 and max(chunk) == 960  # config 3: one workgroup per CU
    # one common chunk size; only entries shorter than it stay whole
    lens3p = [L + 1 for L in lens3]
    assert all(c == 960 or c >= L for c, L in zip(chunk, lens3p))
    full = sum(NKVH * (L // 960) for L in lens3p if L > 960)
    assert full >= 128  # most workgroups stream a full chunk until the end
    chunk, base = qasr_attn.plan_decode([8193], NKVH, 256)
    assert chunk == [544] and base == [0, 8 * 16]  # config 4: 16 chunks of 544 keys
    chunk, base = qasr_attn.plan_decode([512], NKVH, 256)
    assert chunk == [64] and base == [0, 64]  # config 1: 64-key minimum chunk
    # below two minimum chunks an entry stays whole: one chunk of whole passes
    chunk, base = qasr_attn.plan_decode([1, 2, 31, 32, 33, 255, 256, 257], NKVH, 256)
    assert chunk == [32, 32, 32, 32, 64, 64, 64, 64]
    assert base == [0, 8, 16, 24, 32, 40, 72, 104, 144]
    # a batch at the budget (64 entries x 8 kv heads) splits only its longest entries
    lens = [100] * 63 + [4000]
    chunk, base = qasr_attn.plan_decode(lens, NKVH, 256)
    check_decode_plan(lens, chunk, base)
    assert chunk[:63] == [128] * 63 and base[-1] > 512


def test_decode_plan_knobs(monkeypatch):
    # the finest plan the merge tests force: past 32 chunks per entry
    monkeypatch.setenv("QASR_DECODE_MAX_SPLIT", "64")
    monkeypatch.setenv("QASR_DECODE_MIN_CHUNK", "32")
    monkeypatch.setenv("QASR_DECODE_WGS", "4096")
    chunk, base = qasr_attn.plan_decode([8193], NKVH, 256)
    check_decode_plan([8193], chunk, base, max_split=64)
    assert 32 < base[-1] // NKVH <= 64
    monkeypatch.delenv("QASR_DECODE_WGS")
    monkeypatch.setenv("QASR_DECODE_MAX_SPLIT", "32")
    monkeypatch.setenv("QASR_DECODE_MIN_CHUNK", "100000")
    lens = [1500, 700, 4095]
    chunk, base = qasr_attn.plan_decode(lens, NKVH, 256)
    check_decode_plan(lens, chunk, base)
    assert base == [0, 8, 16, 24]  # one chunk per entry: no split, no merge
    monkeypatch.delenv("QASR_DECODE_MIN_CHUNK")
    monkeypatch.setenv("QASR_DECODE_WGS", "512")
    lens3 = [L + 1 for L in splitmix_lengths(SPLITMIX_SEED_CONFIG3, 16, 400, 2400)]
    chunk, base = qasr_attn.plan_decode(lens3, NKVH, 256)
    check_decode_plan(lens3, chunk, base)
    assert 256 < base[-1] <= 512


def test_decode_plan_refusals():
    for lens in ([], [0], [5, -1], [1] * 65):
        with pytest.raises(qasr_attn.QasrError):
            qasr_attn.plan_decode(lens, NKVH, 256)


def check_prefill_plan(rows, kv_start, p):
    rpb, nrb, tps, sp = p["rows_per_block"], p["nrb"], p["tiles_per_split"], p["sp_base"]
    assert rpb in (32, 64) and tps >= 1
    assert nrb == -(-rows // rpb)
    assert sp[0] == 0 and len(sp) == nrb + 1
    for rb in range(nrb):
        kend = kv_start + min((rb + 1) * rpb, rows)
        tiles = -(-kend // 128)
        assert sp[rb + 1] - sp[rb] == -(-tiles // tps), (rows, kv_start, rb)
    if rpb == 32:  # 32-row blocks only for unsplit key ranges
        assert all(sp[rb + 1] - sp[rb] == 1 for rb in range(nrb))


def test_prefill_plan_covers_every_tile_random_launches():
    rng = np.random.default_rng(6)
    for _ in range(300):
        rows = int(rng.integers(1, 4097))
        kv_start = int(rng.integers(0, 12289))
        check_prefill_plan(rows, kv_start, qasr_attn.plan_prefill(rows, kv_start, NKVH))


def test_prefill_plan_bench_configs(monkeypatch):
    p = qasr_attn.plan_prefill(420, 0, NKVH)  # config 2
    assert (p["rows_per_block"], p["nrb"], p["tiles_per_split"]) == (32, 14, 4)
    assert p["sp_base"] == list(range(15))
    p = qasr_attn.plan_prefill(512, 7680, NKVH)  # config 4's last chunk: 4 splits of 16 tiles
    assert (p["rows_per_block"], p["nrb"], p["tiles_per_split"]) == (64, 8, 16)
    assert p["sp_base"][-1] * NKVH == 256
    p = qasr_attn.plan_prefill(512, 0, NKVH)  # 4 tiles: never split
    assert p["rows_per_block"] == 32 and p["sp_base"][-1] == 16
    p = qasr_attn.plan_prefill(513, 0, NKVH)  # 5 tiles: 64-row blocks, split
    assert p["rows_per_block"] == 64
    monkeypatch.setenv("QASR_PREFILL_TPS", "3")
    p = qasr_attn.plan_prefill(420, 0, NKVH)
    assert (p["rows_per_block"], p["tiles_per_split"]) == (64, 3)
    check_prefill_plan(420, 0, p)


def test_prefill_plan_refusals():
    for rows, ks in ((0, 0), (4097, 0), (10, -1)):
        with pytest.raises(qasr_attn.QasrError):
            qasr_attn.plan_prefill(rows, ks, NKVH)
