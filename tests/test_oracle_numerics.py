"""Pins the CPU oracle (oracle/oracle.cpp) without the reference running.

The reference (Rust) cannot be compiled here and ships no golden vectors for
this path; its only unit tests on it are the MRoPE dim-map tests
(src/mrope.rs:86-107), restated first.  Everything else is pinned by what the
mathematics fixes -- independent implementations (numpy float64, complex
rotations), closed forms, invariants and special cases -- each chosen so that a
plausible mistake (dropped term, wrong sign or index, transposed operand)
fails it.  Planted-mistake tests show that the checks do catch such errors.
"""
from __future__ import annotations

import numpy as np
import pytest

from workloads import HD, NKVH, NQH, TOT, tables


# ---------------------------------------------------------------------------
# IEEE binary16 conversions (half 2.7.1 semantics)
# ---------------------------------------------------------------------------
def test_f16_to_f32_exhaustive(O):
    h = np.arange(65536, dtype=np.uint16)
    got = O.f32_from_f16(h)
    want = h.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_f32_to_f16_rne_against_numpy(O):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(300_000) * 10.0 ** rng.integers(-9, 6, 300_000)).astype(np.float32)
    edge = np.array([0.0, -0.0, 65504, 65519.996, 65520, 1e9, -1e9, np.inf, -np.inf, 2 ** -25,
                     2 ** -25 * 1.0001, 2 ** -24, 3 * 2 ** -26, 2 ** -14,
                     2 ** -14 * (1 - 2 ** -11), 1 + 2 ** -11, 1 + 3 * 2 ** -11], dtype=np.float32)
    # every f16 midpoint (ties must go to even)
    h = np.arange(0, 0x7BFF, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)
    x = np.concatenate([x, edge, mids, -mids])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f16_from_f32(x), want)


# ---------------------------------------------------------------------------
# MRoPE tables: src/mrope.rs:86-107 (the reference's own tests), then closed forms
# ---------------------------------------------------------------------------
def test_reference_interleaved_map_respects_quotas(O):  # mrope.rs:86-94
    m = O.build_dim_map([24, 20, 20], 64, True)
    assert len(m) == 64
    assert m.count(0) == 24 and m.count(1) == 20 and m.count(2) == 20
    assert m[:6] == [0, 1, 2, 0, 1, 2]


def test_reference_blocked_map_is_grouped(O):  # mrope.rs:96-100
    assert O.build_dim_map([2, 1], 4, False) == [0, 0, 1, 1]


def test_reference_text_positions_duplicate_halves(O):  # mrope.rs:102-107
    pos3 = np.tile(np.arange(3, dtype=np.int64), (3, 1))
    c, _ = O.mrope_cos_sin(pos3, 8, 1e6, [2, 1, 1], True)
    assert c.shape == (3, 8)
    assert np.array_equal(c[:, :4], c[:, 4:])


def test_interleaved_map_tail_after_quota_exhaustion(O):
    # After axes 1 and 2 run out (20 each) the remaining 4 slots go to axis 0.
    m = O.build_dim_map([24, 20, 20], 64, True)
    assert m[60:] == [0, 0, 0, 0]
    assert m[:60] == [0, 1, 2] * 20


def test_text_tables_closed_form(O):
    """cos/sin[t][j] = f16(f32(cos(t * theta^(-2(j%64)/128)))), numpy float64."""
    tab = tables(O)
    t = np.arange(16384, dtype=np.float64)[:, None]
    inv = 1.0 / (1e6 ** (2.0 * np.arange(64, dtype=np.float64) / 128))[None, :]
    with np.errstate(over="ignore"):
        cn = np.cos(t * inv).astype(np.float32).astype(np.float16).view(np.uint16)
        sn = np.sin(t * inv).astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(tab.cos_u16[:, :64], cn) and np.array_equal(tab.cos_u16[:, 64:], cn)
    assert np.array_equal(tab.sin_u16[:, :64], sn) and np.array_equal(tab.sin_u16[:, 64:], sn)
    # position 0 is the identity rotation; frequency 0 is angle = t.
    assert np.all(tab.cos[0] == 1.0) and np.all(tab.sin[0] == 0.0)
    assert np.allclose(tab.cos[:, 0], np.cos(np.arange(16384)), atol=5e-4)
    assert np.allclose(tab.cos ** 2 + tab.sin ** 2, 1.0, atol=2e-3)


def test_text_tables_independent_of_section_map(O):
    """All three axes carry the same text position, so any map gives one table."""
    a = O.text_rope_tables_f16(300, section=(24, 20, 20), interleaved=True)
    b = O.text_rope_tables_f16(300, section=(24, 20, 20), interleaved=False)
    c = O.text_rope_tables_f16(300, section=(64, 0, 0), interleaved=False)
    for x, y in ((a, b), (a, c)):
        assert np.array_equal(x[0], y[0]) and np.array_equal(x[1], y[1])


def test_mrope_three_axis_positions_follow_map(O):
    """With distinct per-axis positions, column j uses axis dm[j] (brute force)."""
    rng = np.random.default_rng(5)
    pos3 = rng.integers(0, 4000, size=(3, 17)).astype(np.int64)
    for inter in (True, False):
        dm = O.build_dim_map([24, 20, 20], 64, inter)
        c, s = O.mrope_cos_sin(pos3, 128, 1e6, [24, 20, 20], inter)
        inv = 1.0 / (1e6 ** (2.0 * np.arange(64) / 128))
        ang = np.stack([pos3[dm[j]] * inv[j] for j in range(64)], axis=1)
        assert np.array_equal(c[:, :64], np.cos(ang).astype(np.float32))
        assert np.array_equal(s[:, 64:], np.sin(ang).astype(np.float32))


# ---------------------------------------------------------------------------
# norm_rope_head (cpu_decoder.rs:274-290)
# ---------------------------------------------------------------------------
def _norm_rope_f64(raw_u16, gain_f32, cos_row, sin_row, eps=1e-6, sign=1.0):
    """Independent formulation: RMSNorm, then multiply (y_j + i y_{j+64}) by
    e^{i*angle} -- rotate-half RoPE as a complex rotation, in float64."""
    x = raw_u16.view(np.float16).astype(np.float64)
    y = x / np.sqrt(np.mean(x * x) + eps) * gain_f32.astype(np.float64)
    z = (y[:64] + 1j * y[64:]) * (cos_row[:64].astype(np.float64) + 1j * sign * sin_row[:64])
    return np.concatenate([z.real, z.imag])


def test_norm_rope_matches_complex_rotation(O):
    from oracle import Rng

    tab = tables(O)
    rng = Rng(11)
    worst = 0.0
    for p in (0, 1, 7, 511, 2400, 8191, 16383):
        for _ in range(8):
            raw = rng.normal_f16((HD,))
            g = O.f32_from_f16(rng.normal_f16((HD,), 1.0, 0.1))
            got = O.f32_from_f16(O.norm_rope_head(raw, g, tab.cos[p], tab.sin[p])).astype(np.float64)
            want = _norm_rope_f64(raw, g, tab.cos[p], tab.sin[p])
            # f16 output: half an f16 ulp plus the f32 path's few ulps.
            tol = np.maximum(np.abs(want), 2 ** -14) * 2 ** -10 + 1e-6
            assert np.all(np.abs(got - want) <= tol), p
            worst = max(worst, float(np.max(np.abs(got - want))))
    assert worst > 0.0  # the comparison is live (f16 rounding shows up)


def test_norm_rope_planted_sign_mistake_is_caught(O):
    """A rotation with the wrong sign (sin negated) must fail the check above."""
    from oracle import Rng

    tab = tables(O)
    rng = Rng(12)
    raw = rng.normal_f16((HD,))
    g = O.f32_from_f16(rng.normal_f16((HD,), 1.0, 0.1))
    p = 1000
    got = O.f32_from_f16(O.norm_rope_head(raw, g, tab.cos[p], tab.sin[p])).astype(np.float64)
    wrong = _norm_rope_f64(raw, g, tab.cos[p], tab.sin[p], sign=-1.0)
    assert np.max(np.abs(got - wrong)) > 0.1


def test_norm_rope_invariants(O):
    from oracle import Rng

    tab = tables(O)
    rng = Rng(13)
    ones = np.ones(HD, dtype=np.float32)
    for _ in range(20):
        raw = rng.normal_f16((HD,), 0.0, 3.0)
        out0 = O.f32_from_f16(O.norm_rope_head(raw, ones, tab.cos[0], tab.sin[0])).astype(np.float64)
        # position 0 + unit gains: a pure RMSNorm, RMS 1
        assert abs(np.sqrt(np.mean(out0 ** 2)) - 1.0) < 2e-3
        # any position: each (j, j+64) pair keeps its norm (rotation)
        p = int(rng.uniform_int(1, 16383))
        outp = O.f32_from_f16(O.norm_rope_head(raw, ones, tab.cos[p], tab.sin[p])).astype(np.float64)
        n0 = out0[:64] ** 2 + out0[64:] ** 2
        npp = outp[:64] ** 2 + outp[64:] ** 2
        assert np.allclose(n0, npp, rtol=4e-3, atol=1e-5)


def test_rope_relative_position_property(O):
    """q(p).k(p') depends only on p - p' (up to f16 table/output rounding)."""
    from oracle import Rng

    tab = tables(O)
    rng = Rng(14)
    ones = np.ones(HD, dtype=np.float32)
    qr, kr = rng.normal_f16((HD,)), rng.normal_f16((HD,))

    def dot(pq, pk):
        q = O.f32_from_f16(O.norm_rope_head(qr, ones, tab.cos[pq], tab.sin[pq])).astype(np.float64)
        k = O.f32_from_f16(O.norm_rope_head(kr, ones, tab.cos[pk], tab.sin[pk])).astype(np.float64)
        return float(q @ k)

    for d in (0, 1, 5, 37):
        vals = [dot(p + d, p) for p in (0, 3, 100, 1234)]
        assert max(vals) - min(vals) < 0.3, (d, vals)  # |q.k| ~ 128 scale


# ---------------------------------------------------------------------------
# attention (cpu_decoder.rs:292-365)
# ---------------------------------------------------------------------------
def _attn_f64(q_u16, k_f32, v_f32, q0):
    """Causal GQA softmax attention in float64; q [rows][nqh*hd]."""
    rows = q_u16.shape[0]
    q = q_u16.view(np.float16).astype(np.float64).reshape(rows, NQH, HD)
    k = k_f32.astype(np.float64)
    v = v_f32.astype(np.float64)
    out = np.zeros((rows, NQH, HD))
    scale = 1.0 / np.sqrt(HD)
    for r in range(rows):
        L = q0 + r + 1
        for h in range(NQH):
            kh = h // (NQH // NKVH)
            s = k[kh, :L] @ q[r, h] * scale
            w = np.exp(s - s.max())
            w /= w.sum()
            out[r, h] = w @ v[kh, :L]
    return out.reshape(rows, NQH * HD)


def _random_caches(rng, L, cap):
    k = np.zeros((NKVH, cap, HD), np.float32)
    v = np.zeros((NKVH, cap, HD), np.float32)
    from oracle import f32_from_f16

    k[:, :L] = f32_from_f16(rng.normal_f16((NKVH, L, HD)))
    v[:, :L] = f32_from_f16(rng.normal_f16((NKVH, L, HD)))
    return k, v


@pytest.mark.parametrize("L,rows", [(1, 1), (7, 1), (300, 1), (64, 64), (200, 24)])
def test_attention_matches_float64(O, L, rows):
    from oracle import Rng

    rng = Rng(20 + L + rows)
    cap = 1024
    k, v = _random_caches(rng, L, cap)
    q = rng.normal_f16((rows, NQH * HD), 0.0, 0.3)
    q0 = L - rows
    sh = O.make_shape()
    got = O.f32_from_f16(O.attention(sh, cap, q, q0, k, v)).astype(np.float64)
    want = _attn_f64(q, k, v, q0)
    assert np.max(np.abs(got - want)) <= 2 ** -11 * np.maximum(np.abs(want), 2 ** -14).max() + 2e-6


def test_attention_special_cases(O):
    from oracle import Rng

    rng = Rng(30)
    cap, sh = 1024, O.make_shape()
    k, v = _random_caches(rng, 50, cap)
    vf16 = O.f16_from_f32(v)
    # L = 1: output is exactly v_0 of the head's kv head.
    q = rng.normal_f16((1, NQH * HD))
    out = O.attention(sh, cap, q, 0, k, v).reshape(NQH, HD)
    for h in range(NQH):
        assert np.array_equal(out[h], vf16[h // 2, 0])
    # q = 0: uniform weights, the mean of the V rows.
    L = 50
    q0 = np.zeros((1, NQH * HD), np.uint16)
    out = O.f32_from_f16(O.attention(sh, cap, q0, L - 1, k, v)).reshape(NQH, HD)
    for h in range(NQH):
        assert np.allclose(out[h], v[h // 2, :L].mean(0), atol=1e-3)
    # a key that dominates by far picks its V row.
    k2 = k.copy()
    hot = 17
    qv = rng.normal_f16((1, NQH * HD))
    qf = O.f32_from_f16(qv).reshape(NQH, HD)
    for kh in range(NKVH):
        k2[kh, hot] = qf[2 * kh] * 40.0
    out = O.f32_from_f16(O.attention(sh, cap, qv, L - 1, k2, v)).reshape(NQH, HD)
    for kh in range(NKVH):
        assert np.allclose(out[2 * kh], v[kh, hot], atol=2e-3)


def test_attention_causal_and_gqa_mapping(O):
    from oracle import Rng

    rng = Rng(31)
    cap, sh = 1024, O.make_shape()
    L = 80
    k, v = _random_caches(rng, 120, cap)
    q = rng.normal_f16((1, NQH * HD))
    base = O.attention(sh, cap, q, L - 1, k, v)
    # keys beyond the row's position never matter
    k2, v2 = k.copy(), v.copy()
    k2[:, L:] += 5.0
    v2[:, L:] -= 3.0
    assert np.array_equal(O.attention(sh, cap, q, L - 1, k2, v2), base)
    # perturbing kv head 3 changes q heads 6 and 7 only
    k3 = k.copy()
    k3[3, :L] *= -1.0
    pert = O.attention(sh, cap, q, L - 1, k3, v).reshape(NQH, HD)
    b = base.reshape(NQH, HD)
    changed = [h for h in range(NQH) if not np.array_equal(pert[h], b[h])]
    assert changed == [6, 7]


def test_attention_threads_do_not_change_results(O):
    from oracle import Rng

    rng = Rng(32)
    cap, sh = 1024, O.make_shape()
    k, v = _random_caches(rng, 333, cap)
    q = rng.normal_f16((9, NQH * HD))
    a = O.attention(sh, cap, q, 324, k, v, nthreads=1)
    b = O.attention(sh, cap, q, 324, k, v, nthreads=5)
    assert np.array_equal(a, b)


def test_layer_attn_equals_stage_a_then_attention(O):
    from oracle import Rng

    from workloads import Layer, OracleSeq

    tab = tables(O)
    rng = Rng(33)
    lay = Layer(rng)
    a = OracleSeq(O, 1024, lay, tab)
    b = OracleSeq(O, 1024, lay, tab)
    qkv = rng.normal_f16((40, TOT))
    qa, oa = a.step(qkv, 0)
    qb = b.append(qkv, 0)
    ob = b.attend(qb, 0)
    assert np.array_equal(qa, qb) and np.array_equal(oa, ob)
    assert np.array_equal(a.k, b.k) and np.array_equal(a.v, b.v)
    # V is copied untouched; K rows are the roped k heads
    vraw = O.f32_from_f16(qkv[:, (NQH + NKVH) * HD:]).reshape(40, NKVH, HD)
    assert np.array_equal(a.v[:, :40].transpose(1, 0, 2), vraw)


def test_chunked_equals_full(O):
    """Prefill in pieces (kv_start > 0) equals one prefill (stream.rs:366-376)."""
    from oracle import Rng

    from workloads import Layer, OracleSeq

    tab = tables(O)
    rng = Rng(34)
    lay = Layer(rng)
    qkv = rng.normal_f16((90, TOT))
    full = OracleSeq(O, 1024, lay, tab)
    _, of = full.step(qkv, 0)
    part = OracleSeq(O, 1024, lay, tab)
    _, o1 = part.step(qkv[:33], 0)
    _, o2 = part.step(qkv[33:], 33)
    assert np.array_equal(np.concatenate([o1, o2]), of)


def test_kv_target_cap(O):
    # grow-only, KV_STEP (256) granular, clamped to max_seq (cpu_decoder.rs:228)
    assert O.kv_target_cap(1000, 1024, 16384) == 1024
    assert O.kv_target_cap(1025, 1024, 16384) == 1280
    assert O.kv_target_cap(1280, 1024, 16384) == 1280
    assert O.kv_target_cap(20000, 1024, 16384) == 16384
    assert O.kv_target_cap(100, 2048, 16384) == 2048
    assert O.kv_target_cap(16385, 1024, 16000) == 16000


def test_softmax_weights_are_expf_of_the_rounded_difference(O):
    """qo_softmax_weights = expf(f32(s*scale) - f32(m*scale)): against float64
    exp of the same f32 argument (glibc expf is within one ulp), exactly 1 at
    s == m, and a planted mistake (the difference taken before scaling, a
    different rounding of the argument) is told apart on integer dots."""
    rng = np.random.default_rng(11)
    scale = np.float32(1.0 / np.sqrt(np.float32(128.0)))
    m = rng.uniform(-300, 300, 200000).astype(np.float32)
    s = (m - rng.uniform(0, 80 / float(scale), m.size)).astype(np.float32)
    got = O.softmax_weights(s, m, float(scale)).astype(np.float64)
    arg = (s * scale).astype(np.float32) - (m * scale).astype(np.float32)  # f32 ops
    want = np.exp(arg.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= ulp)
    assert np.all(O.softmax_weights(m, m, float(scale)) == 1.0)
    si = np.arange(-200, 0, dtype=np.float32)
    mi = np.zeros_like(si) + 7.0
    planted = np.exp(((si - mi) * scale).astype(np.float32).astype(np.float64))
    real = O.softmax_weights(si, mi, float(scale)).astype(np.float64)
    assert np.any(real != planted.astype(np.float32))
