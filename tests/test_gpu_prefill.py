"""Stage (c) causal prefill attention on the GPU against the oracle
(cpu_decoder.rs:292-365 with rows = s, q0 = kv_start), at config 2's shape,
ragged row counts, chunked prefill against an existing cache (config 4), and
the invariants: chunked == full prefill (stream.rs:366-376 / stream_api.rs:
178-185) and prefill row r == a decode query at position kv_start + r."""
from __future__ import annotations

import numpy as np
import pytest

from workloads import QDIM, SEED_BASE, TOT, Layer, OracleSeq, assert_parity, cap_for, tables

pytestmark = pytest.mark.gpu


def _prefill_gpu(g, layer, lay, slot, kv_start, qkv):
    import qasr_attn
    from gpu_helpers import dev, empty, host, say

    s = qkv.shape[0]
    q = empty(s, QDIM)
    out = empty(s, QDIM)
    qg, kg = g.gains(lay)
    say(f"prefill slot={slot} kv_start={kv_start} s={s}")
    qasr_attn.prefill_layer(g.ctx, g.kv, layer, slot, kv_start, s, dev(qkv), qg, kg, q, out)
    return host(q), host(out)


def test_config2_prefill_420(O, gpu):
    from gpu_helpers import Gpu

    from oracle import Rng

    rng = Rng(SEED_BASE + 2)
    lay = Layer(rng)
    s = 420
    qkv = rng.normal_f16((s, TOT))
    g = Gpu(slots=1, cap=1024)
    q_gpu, out_gpu = _prefill_gpu(g, 0, lay, 0, 0, qkv)
    ref = OracleSeq(O, 1024, lay, tables(O))
    q_ref, out_ref = ref.step(qkv, 0)
    assert np.array_equal(q_gpu, q_ref)
    ma, mr = assert_parity(out_gpu, out_ref, "config2", p_f16=True)
    print("config2 max_abs/max_rel", ma, mr)
    g.close()


@pytest.mark.parametrize("kv_start,s", [(0, 1), (0, 31), (0, 64), (0, 65), (0, 200), (5, 1),
                                        (100, 3), (640, 129), (724, 300), (1000, 600), (3000, 64)])
def test_prefill_ragged_against_oracle(O, gpu, kv_start, s):
    from gpu_helpers import Gpu

    from oracle import Rng

    rng = Rng(SEED_BASE + 400 + kv_start + s)
    lay = Layer(rng)
    cap = cap_for(kv_start + s)
    g = Gpu(slots=2, cap=cap)
    ref = OracleSeq(O, cap, lay, tables(O))
    if kv_start:
        pre = rng.normal_f16((kv_start, TOT))
        ref.append(pre, 0)
        g.append(0, lay, [(1, 0, kv_start)], pre)
    qkv = rng.normal_f16((s, TOT))
    _, out_gpu = _prefill_gpu(g, 0, lay, 1, kv_start, qkv)
    _, out_ref = ref.step(qkv, kv_start)
    assert_parity(out_gpu, out_ref, f"kv_start={kv_start} s={s}", p_f16=True)
    g.close()


@pytest.mark.parametrize("tps", ["1", "3", "1000"])
def test_prefill_split_choices(O, gpu, tps, monkeypatch):
    """Any split of the key range (1 tile per item .. no split) matches."""
    from gpu_helpers import Gpu

    from oracle import Rng

    monkeypatch.setenv("QASR_PREFILL_TPS", tps)
    rng = Rng(SEED_BASE + 500)
    lay = Layer(rng)
    s = 700
    qkv = rng.normal_f16((s, TOT))
    g = Gpu(slots=1, cap=1024)
    _, out_gpu = _prefill_gpu(g, 0, lay, 0, 0, qkv)
    ref = OracleSeq(O, 1024, lay, tables(O))
    _, out_ref = ref.step(qkv, 0)
    assert_parity(out_gpu, out_ref, f"tps={tps}", p_f16=True)
    g.close()


def test_config4_chunked_prefill_long_context(O, gpu):
    """Config 4: 16 chunks of 512 rows at kv_start = 0..7680.  Every row of
    every chunk matches the oracle; the chunked result equals a single
    8192-row prefill within tolerance, and re-running a chunk is
    deterministic."""
    from gpu_helpers import Gpu

    from oracle import Rng

    rng = Rng(SEED_BASE + 4)
    lay = Layer(rng)
    total, chunk = 8192, 512
    cap = cap_for(total + 64)
    qkv = rng.normal_f16((total, TOT))
    g = Gpu(slots=2, cap=cap)
    outs = []
    for c in range(total // chunk):
        _, o = _prefill_gpu(g, 0, lay, 0, c * chunk, qkv[c * chunk:(c + 1) * chunk])
        outs.append(o)
    chunked = np.concatenate(outs)
    _, full = _prefill_gpu(g, 0, lay, 1, 0, qkv)
    assert_parity(chunked, full, "chunked vs full", p_f16=True)
    _, again = _prefill_gpu(g, 0, lay, 0, total - chunk, qkv[total - chunk:])
    assert np.array_equal(again, outs[-1])
    # oracle: cache from stage (a) over all rows, then every chunk's rows
    from gpu_helpers import say

    ref = OracleSeq(O, cap, lay, tables(O))
    q_ref = ref.append(qkv, 0)
    for c in range(total // chunk):
        r0 = c * chunk
        say(f"oracle chunk {c}")
        want = ref.attend(q_ref[r0:r0 + chunk], r0)
        assert_parity(chunked[r0:r0 + chunk], want, f"config4 chunk {c} (kv_start {r0})",
                      p_f16=True)
    g.close()


def test_prefill_row_equals_decode_query(O, gpu):
    """Prefill row r attends exactly what a decode query at kv_start + r does."""
    import qasr_attn
    from gpu_helpers import Gpu, dev, empty, host

    from oracle import Rng

    rng = Rng(SEED_BASE + 600)
    lay = Layer(rng)
    kv_start, s = 300, 250
    g = Gpu(slots=1, cap=1024)
    pre = rng.normal_f16((kv_start, TOT))
    g.append(0, lay, [(0, 0, kv_start)], pre)
    qkv = rng.normal_f16((s, TOT))
    q, out = _prefill_gpu(g, 0, lay, 0, kv_start, qkv)
    rows = [0, 1, 63, 64, 127, 200, 249]
    dq = empty(len(rows), QDIM)
    dq.copy_(dev(q[rows]))
    dout = empty(len(rows), QDIM)
    qasr_attn.decode_attn(g.ctx, g.kv, 0, [kv_start + r + 1 for r in rows], dq, dout,
                          slots=[0] * len(rows))
    assert_parity(host(dout), out[rows], "prefill vs decode", p_f16=True)
    g.close()


def _segments_setup(O, rng, lay, segments, cap):
    """Pool with every segment's earlier keys appended; returns (Gpu, per-slot
    oracles, the segments' qkv rows concatenated, roped q rows)."""
    from gpu_helpers import Gpu

    g = Gpu(slots=len(segments), cap=cap)
    refs = []
    for slot, kv_start, _ in segments:
        ref = OracleSeq(O, cap, lay, tables(O))
        if kv_start:
            pre = rng.normal_f16((kv_start, TOT))
            ref.append(pre, 0)
            g.append(0, lay, [(slot, 0, kv_start)], pre)
        refs.append(ref)
    qkv = rng.normal_f16((sum(r for _, _, r in segments), TOT))
    q = g.append(0, lay, list(segments), qkv)
    return g, refs, qkv, q


@pytest.mark.parametrize("tps", [None, "3"])
def test_prefill_attn_batch_equals_single_segment_calls(O, gpu, tps, monkeypatch):
    """--batch N == --batch 1 for prefill attention: one batched call over
    segments whose plans differ (32-row unsplit blocks, 64-row blocks with
    key splits, config 4's last chunk, a segment longer than one 4096-row
    piece) gives every segment the bits of its own qasr_prefill_attn call,
    under the default plans and under a forced split count."""
    import qasr_attn
    from gpu_helpers import dev, empty, host, say

    from oracle import Rng

    if tps is None:
        monkeypatch.delenv("QASR_PREFILL_TPS", raising=False)
    else:
        monkeypatch.setenv("QASR_PREFILL_TPS", tps)
    rng = Rng(SEED_BASE + 480)
    lay = Layer(rng)
    segments = [(0, 0, 37), (1, 0, 200), (2, 100, 120), (3, 0, 1), (4, 190, 66),
                (5, 7680, 512), (6, 900, 4200)]
    g, _, _, q = _segments_setup(O, rng, lay, segments, cap_for(7680 + 512))
    total = q.shape[0]
    say(f"prefill_attn_batch over {segments} tps={tps}")
    out_b = empty(total, QDIM)
    qasr_attn.prefill_attn_batch(g.ctx, g.kv, 0, segments, dev(q), out_b)
    got = host(out_b)
    r0 = 0
    for slot, kv_start, rows in segments:
        out_s = empty(rows, QDIM)
        qasr_attn.prefill_attn(g.ctx, g.kv, 0, slot, kv_start, rows, dev(q[r0:r0 + rows]), out_s)
        assert np.array_equal(got[r0:r0 + rows], host(out_s)), f"segment {slot}"
        r0 += rows
    g.close()


def test_prefill_attn_batch_of_many_short_segments_equals_single_calls(O, gpu):
    """Short segments alone run 16-row blocks (four waves, both q heads in
    one wave's MFMA columns); twelve of them in one batched call run 32-row
    blocks (eight waves, one q head per wave).  Every segment must still get
    its lone call's bits."""
    import qasr_attn
    from gpu_helpers import dev, empty, host, say

    from oracle import Rng

    rng = Rng(SEED_BASE + 482)
    lay = Layer(rng)
    segments = [(i, ks, rows) for i, (ks, rows) in enumerate(
        [(0, 420), (0, 150), (100, 300), (0, 512), (37, 1), (0, 33), (200, 250), (0, 400),
         (5, 90), (0, 320), (64, 448), (0, 17)])]
    for _, ks, rows in segments:  # each alone plans 16-row blocks
        assert qasr_attn.plan_prefill(rows, ks, 8)["rows_per_block"] == 16, (ks, rows)
    g, _, _, q = _segments_setup(O, rng, lay, segments, cap_for(1024))
    say(f"prefill_attn_batch over {len(segments)} short segments")
    out_b = empty(q.shape[0], QDIM)
    qasr_attn.prefill_attn_batch(g.ctx, g.kv, 0, segments, dev(q), out_b)
    got = host(out_b)
    r0 = 0
    for slot, kv_start, rows in segments:
        out_s = empty(rows, QDIM)
        qasr_attn.prefill_attn(g.ctx, g.kv, 0, slot, kv_start, rows, dev(q[r0:r0 + rows]), out_s)
        assert np.array_equal(got[r0:r0 + rows], host(out_s)), f"segment {slot}"
        r0 += rows
    g.close()


def test_prefill_attn_batch_long_segments_against_oracle(O, gpu):
    """Key ranges up to 2048 in one batched call (each segment on its own
    plan, some with key splits) against the oracle, segment by segment."""
    import qasr_attn
    from gpu_helpers import dev, empty, host, say

    from oracle import Rng

    rng = Rng(SEED_BASE + 481)
    lay = Layer(rng)
    segments = [(0, 0, 300), (1, 500, 700), (2, 0, 1500), (3, 1200, 64), (4, 2000, 48)]
    g, refs, qkv, q = _segments_setup(O, rng, lay, segments, cap_for(2048))
    say(f"prefill_attn_batch over {segments}")
    out_b = empty(q.shape[0], QDIM)
    qasr_attn.prefill_attn_batch(g.ctx, g.kv, 0, segments, dev(q), out_b)
    got = host(out_b)
    r0 = 0
    for (slot, kv_start, rows), ref in zip(segments, refs):
        _, want = ref.step(qkv[r0:r0 + rows], kv_start)
        assert_parity(got[r0:r0 + rows], want, f"segment {slot} kv_start={kv_start} rows={rows}", p_f16=True)
        r0 += rows
    g.close()


def test_prefill_attn_batch_refuses_bad_segments(gpu):
    """Every segment is checked before any launch: a slot outside the pool,
    positions past the pool's capacity or max_seq are refused with the
    reference's error kinds, and nothing is written."""
    import torch

    import qasr_attn
    from gpu_helpers import Gpu, empty

    g = Gpu(slots=2, cap=512)
    q = torch.zeros((40, QDIM), dtype=torch.float16, device="cuda")
    out = empty(40, QDIM)
    out.fill_(7.0)
    cases = [([(0, 0, 20), (2, 0, 20)], qasr_attn.QASR_EINVAL),   # slot 2 of 2
             ([(0, 0, 20), (1, 500, 20)], qasr_attn.QASR_ERANGE),  # past capacity 512
             ([(0, -1, 20), (1, 0, 20)], qasr_attn.QASR_EINVAL)]   # negative kv_start
    for segs, code in cases:
        with pytest.raises(qasr_attn.QasrError) as e:
            qasr_attn.prefill_attn_batch(g.ctx, g.kv, 0, segs, q, out)
        assert e.value.code == code, (segs, e.value)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()), "a refused call wrote output"
    g.close()
