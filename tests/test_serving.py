"""serving.py on the CPU: the batch scheduler (decode_batch_embeds /
run_batch_attempt / fill_slots, src/inference.rs:707-764, 1944-2227) over a
scripted decoder whose next token is a fixed function of (segment, position),
as a real decoder's greedy stream is.  The fake checks the pool invariants
itself (distinct live slots, steps only on occupied slots, no position past
the pool's capacity); the tests check that every segment gets exactly the
tokens the single-sequence loop (generate_from_embeds, inference.rs:
2300-2380) gives it, whatever the width, plus admission order, refill,
width halving after a failure, cancellation and the BATCH_SEQ_CAP split."""
from __future__ import annotations

import numpy as np
import pytest

import serving as S

EOS = S.ENDOFTEXT_TOKEN_ID


class FakeDecoder:
    """Segment g's hidden rows carry g in element [0, 0]; its token stream is
    script[g] (then a filler token)."""

    def __init__(self, scripts, max_seq=16384, fail_slots_above=None, fail_on_step=None):
        self.scripts = scripts
        self.max_seq = max_seq
        self.fail_slots_above = fail_slots_above
        self.fail_on_step = fail_on_step  # (pool width, step call index) that raises once
        self.slots_state = []
        self.cap = 0
        self.nslots = 0
        self.steps = 0
        self.pools = []
        self.prefill_calls = []
        self.step_rows = []

    def reset_pool(self, slots, cap):
        if self.fail_slots_above is not None and slots > self.fail_slots_above:
            raise MemoryError(f"{slots} slots do not fit")
        self.pools.append((slots, cap))
        self.nslots, self.cap = slots, cap
        self.slots_state = [None] * slots
        self.steps = 0

    def _admit(self, slot, hidden):
        assert 0 <= slot < self.nslots
        g = int(hidden[0, 0])
        s = hidden.shape[0]
        assert s <= self.cap
        self.slots_state[slot] = [g, s, 1]
        return self.scripts[g][0]

    def prefill(self, hidden, kv_start=0, slot=0):
        assert kv_start == 0
        self.prefill_calls.append([slot])
        return self._admit(slot, hidden)

    def prefill_batch(self, items):
        slots = [s for s, _ in items]
        assert len(set(slots)) == len(slots)
        self.prefill_calls.append(slots)
        return [self._admit(s, h) for s, h in items]

    def step(self, slots):
        assert len(set(slots)) == len(slots)
        self.steps += 1
        if self.fail_on_step == (self.nslots, self.steps):
            self.fail_on_step = None
            raise RuntimeError("device lost")
        self.step_rows.append(len(slots))
        out = []
        for s in slots:
            st = self.slots_state[s]
            assert st is not None, f"step of empty slot {s}"
            g, pos, k = st
            assert pos + 1 <= self.cap, "position past the pool capacity"
            script = self.scripts[g]
            out.append(script[k] if k < len(script) else 1000 + g)
            st[1], st[2] = pos + 1, k + 1
        return out


class PipeFakeDecoder(FakeDecoder):
    """The same scripted decoder with the pipelined interface: step_async
    launches a step (the tokens are fixed at launch, as the device feedback
    fixes them), step_result hands them over; at most two steps in flight."""

    def __init__(self, *a, **k):
        super().__init__(*a, **k)
        self.in_flight = 0
        self.max_in_flight = 0

    def reset_pool(self, slots, cap):
        super().reset_pool(slots, cap)
        self.in_flight = 0  # a new pool waits for every step in flight

    def step_async(self, slots):
        toks = self.step(slots)
        self.in_flight += 1
        self.max_in_flight = max(self.max_in_flight, self.in_flight)
        return (list(slots), toks)

    def step_result(self, handle):
        self.in_flight -= 1
        return handle[1]


def _hidden(g, rows):
    h = np.zeros((rows, 4), np.float32)
    h[0, 0] = g
    return h


def _case(seed, n, eos_rate=0.08, lens=(20, 400)):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lens[0], lens[1], size=n)
    scripts = []
    for g in range(n):
        sc = [int(t) for t in rng.integers(0, 5000, size=rng.integers(1, 60))]
        for k in range(len(sc)):
            if rng.random() < eos_rate:
                sc[k] = EOS if rng.random() < 0.5 else S.IM_END_TOKEN_ID
        scripts.append(sc)
    plans = [_hidden(g, int(lens[g])) for g in range(n)]
    max_news = [int(m) for m in rng.integers(0, 50, size=n)]
    return plans, max_news, scripts


def _single_expected(script, max_new):
    """generate_from_embeds: the first token counts; then max_new - 1 steps."""
    if script[0] in S.EOS_IDS:
        return [], S.StopReason.EOS
    ids = [script[0]]
    for k in range(1, max(max_new, 1)):
        tok = script[k] if k < len(script) else None
        if tok in S.EOS_IDS:
            return ids, S.StopReason.EOS
        ids.append(tok)
    return ids, S.StopReason.MAX_TOKENS


def _batch_stop(script, ids):
    """run_batch_attempt: the step after the last kept token decides the
    reason -- an EOS there is an EOS stop even at the token limit."""
    if not ids:
        return S.StopReason.EOS
    nxt = script[len(ids)] if len(ids) < len(script) else None
    return S.StopReason.EOS if nxt in S.EOS_IDS else S.StopReason.MAX_TOKENS


def _fill_filler(scripts, plans, max_news):
    return [sc + [1000 + g] * (max_news[g] + 2) for g, sc in enumerate(scripts)]


@pytest.mark.parametrize("pipe", [False, True])
@pytest.mark.parametrize("width", [1, 2, 3, 8, 16, 64])
def test_every_width_gives_the_single_path_tokens(width, pipe):
    plans, max_news, scripts = _case(1, 37)
    scripts = _fill_filler(scripts, plans, max_news)
    dec = PipeFakeDecoder(scripts) if pipe else FakeDecoder(scripts)
    res = S.decode_batch(dec, plans, max_news, width)
    if pipe:
        assert dec.max_in_flight == 2 and dec.in_flight <= 1
    for g, r in enumerate(res):
        ids, stop = _single_expected(scripts[g], max_news[g])
        assert r.ids == ids, g
        want_stop = stop if width < 2 else _batch_stop(scripts[g], ids)
        assert r.stop_reason == want_stop, g


@pytest.mark.parametrize("pipe", [False, True])
def test_single_path_generate_matches_reference_loop(pipe):
    plans, max_news, scripts = _case(2, 12)
    scripts = _fill_filler(scripts, plans, max_news)
    dec = PipeFakeDecoder(scripts) if pipe else FakeDecoder(scripts)
    for g in range(12):
        r = S.generate(dec, plans[g], max_news[g])
        assert (r.ids, r.stop_reason) == _single_expected(scripts[g], max_news[g])
        assert dec.pools[-1] == (1, S.kv_cap(plans[g].shape[0], max_news[g]))


def test_longest_prompt_first_admission_and_refill():
    plans, max_news, scripts = _case(3, 20, eos_rate=0.0)
    scripts = _fill_filler(scripts, plans, max_news)

    class Ev(S.BatchEvents):
        def __init__(self):
            self.admits = []
            self.items = []

        def on_admit(self, i, slot):
            self.admits.append((i, slot))

        def on_item(self, i, r):
            self.items.append(i)

    ev = Ev()
    dec = FakeDecoder(scripts)
    S.decode_batch(dec, plans, max_news, 4, events=ev)
    lens = [p.shape[0] for p in plans]
    order = sorted(range(20), key=lambda i: -lens[i])
    assert [i for i, _ in ev.admits] == order
    # the first four go to slots 0..3 in one prefill call
    assert ev.admits[:4] == [(order[k], k) for k in range(4)]
    assert dec.prefill_calls[0] == [0, 1, 2, 3]
    assert sorted(ev.items) == list(range(20))
    # a pool of min(width, n) slots sized for the longest segment
    assert dec.pools == [(4, max(S.kv_cap(lens[i], max_news[i]) for i in range(20)))]
    # never more rows than slots, and a refill lands in the slot just freed
    assert max(dec.step_rows) <= 4


def test_first_token_eos_is_an_empty_eos_result():
    scripts = [[EOS], [5, 6, EOS], [S.IM_END_TOKEN_ID, 3]]
    plans = [_hidden(g, 10 + g) for g in range(3)]
    res = S.decode_batch(FakeDecoder(scripts), plans, [8, 8, 8], 4)
    assert (res[0].ids, res[0].stop_reason) == ([], S.StopReason.EOS)
    assert (res[1].ids, res[1].stop_reason) == ([5, 6], S.StopReason.EOS)
    assert (res[2].ids, res[2].stop_reason) == ([], S.StopReason.EOS)


def test_width_halves_until_the_pool_fits():
    plans, max_news, scripts = _case(4, 30)
    scripts = _fill_filler(scripts, plans, max_news)
    dec = FakeDecoder(scripts, fail_slots_above=5)
    res = S.decode_batch(dec, plans, max_news, 16)
    assert [p[0] for p in dec.pools] == [4]
    for g, r in enumerate(res):
        assert r.ids == _single_expected(scripts[g], max_news[g])[0]


def test_pipelining_can_be_switched_off(monkeypatch):
    plans, max_news, scripts = _case(7, 9)
    scripts = _fill_filler(scripts, plans, max_news)
    monkeypatch.setenv("QASR_DEC_PIPE", "off")
    dec = PipeFakeDecoder(scripts)
    res = S.decode_batch(dec, plans, max_news, 4)
    assert dec.max_in_flight == 0
    for g, r in enumerate(res):
        assert r.ids == _single_expected(scripts[g], max_news[g])[0]


def test_failure_mid_run_keeps_finished_segments_and_reruns_the_rest():
    plans, max_news, scripts = _case(5, 24, eos_rate=0.2)
    scripts = _fill_filler(scripts, plans, max_news)
    done_order = []

    class Ev(S.BatchEvents):
        def on_item(self, i, r):
            done_order.append(i)

    dec = FakeDecoder(scripts, fail_on_step=(8, 6))
    res = S.decode_batch(dec, plans, max_news, 8, events=Ev())
    assert [p[0] for p in dec.pools][:2] == [8, 4]
    assert sorted(done_order) == list(range(24))  # each segment reported once
    for g, r in enumerate(res):
        assert r.ids == _single_expected(scripts[g], max_news[g])[0]


def test_cancellation_reports_the_rest_cancelled():
    plans, max_news, scripts = _case(6, 16, eos_rate=0.0)
    scripts = _fill_filler(scripts, plans, [40] * 16)

    class Ev(S.BatchEvents):
        polls = 0

        def should_stop(self):
            self.polls += 1
            return self.polls > 10

    res = S.decode_batch(FakeDecoder(scripts), plans, [40] * 16, 4, events=Ev())
    assert all(isinstance(r, S.Cancelled) for r in res)


def test_segments_past_batch_seq_cap_take_the_single_path_first():
    plans = [_hidden(0, 4000), _hidden(1, 100), _hidden(2, 200)]
    scripts = [[7] * 200, [8] * 200, [9] * 200]
    max_news = [120, 30, 30]  # 4000 + 120 + 8 -> 4352 > 4096
    dec = FakeDecoder(scripts)
    res = S.decode_batch(dec, plans, max_news, 8)
    assert dec.pools[0] == (1, S.kv_cap(4000, 120))
    assert dec.pools[1] == (2, S.kv_cap(200, 30))
    assert [len(r.ids) for r in res] == [120, 30, 30]


def test_max_seq_overflow_fails_only_that_segment():
    plans = [_hidden(0, 5000), _hidden(1, 50)]
    scripts = [[7] * 10, [8] * 10]
    res = S.decode_batch(FakeDecoder(scripts, max_seq=5004), plans, [10, 5], 4)
    assert isinstance(res[0], ValueError)
    assert res[1].ids == [8] * 5
