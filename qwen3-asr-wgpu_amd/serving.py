"""Batched greedy decoding of many segments over one text decoder's slots.

Host mirror of the reference's batch scheduler (src/inference.rs):

  * `decode_batch` -- `decode_batch_embeds` (inference.rs:1944-2102): segments
    whose KV would pass BATCH_SEQ_CAP are decoded alone first; the rest run in
    slot batches of `width`, and a batch-wide failure halves the width and
    re-runs only the segments not yet finished (width 1 is the single path).
  * `_attempt` -- `run_batch_attempt` (inference.rs:2117-2227): one pool of
    min(width, n) slots sized for the longest segment (`fork_capped`),
    longest prompt admitted first, every slot stepped together, a finished
    slot refilled at once.
  * `fill` in `_attempt` -- `fill_slots` (inference.rs:707-750): the free
    slots (ascending) take the next segments in admission order; their
    prompts are prefilled together (`prefill_batch`: one projection pass over
    all their rows).  A segment whose first token is an EOS id is reported at
    once as an empty EOS result, as the single path reports it (the
    reference's batch path leaves it unreported, so its `finish` calls it
    "not decoded").
  * `generate` -- the single-sequence greedy loop of `generate_from_embeds`
    (inference.rs:2229-2385, the non-pipelined arm).

A segment is its prompt's hidden rows ([s][hs] f16; building the prompt from
a tokenizer and audio embeddings happens before this layer); the result is
the generated token ids and the stop reason.  The decoder is duck-typed: a
`qasr_attn.TextDecoder`, or anything with `max_seq`, `reset_pool(slots, cap)`,
`prefill(hidden, kv_start, slot)`, `prefill_batch([(slot, hidden)])` and
`step(slots)`.
"""
from __future__ import annotations

import enum
import os
import sys
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

ENDOFTEXT_TOKEN_ID = 151643  # prompt.rs:25
IM_END_TOKEN_ID = 151645  # prompt.rs:24
EOS_IDS = (ENDOFTEXT_TOKEN_ID, IM_END_TOKEN_ID)
KV_STEP = 256  # decoder.rs KV_STEP
BATCH_SEQ_CAP = 4096  # decoder.rs:684


class StopReason(enum.Enum):
    MAX_TOKENS = "max_tokens"
    EOS = "eos"


@dataclass
class Generation:
    ids: List[int] = field(default_factory=list)
    stop_reason: StopReason = StopReason.MAX_TOKENS


class Cancelled(Exception):
    """`BatchEvents.should_stop` ended the job before this segment finished."""


class NotDecoded(Exception):
    """The job ended without a result for this segment."""


class BatchEvents:
    """Callbacks of a batch job (BatchEvents, inference.rs): `should_stop`
    is polled before every step; `on_item` receives each segment's final
    result (a Generation or an exception) once, as soon as it is final;
    `on_admit` says which slot a segment was admitted to."""

    def should_stop(self) -> bool:
        return False

    def on_item(self, index: int, result) -> None:
        pass

    def on_admit(self, index: int, slot: int) -> None:
        pass


def pipelined(decoder) -> bool:
    """One step in flight (QASR_DEC_PIPE, on unless "0", "off" or "false";
    pipelined_decode, inference.rs:2431-2439), when the decoder can launch a
    step without waiting for it (step_async / step_result)."""
    off = os.environ.get("QASR_DEC_PIPE", "") in ("0", "off", "false")
    return not off and hasattr(decoder, "step_async")


def kv_cap(seq_len: int, max_new: int) -> int:
    """Positions a segment may need: prompt + generation + 8, rounded up to
    KV_STEP (inference.rs:2036, 2127-2131)."""
    return -(-(seq_len + max_new + 8) // KV_STEP) * KV_STEP


class _Outcomes:
    """One entry per segment, emitted once (Outcomes, inference.rs:866-911)."""

    def __init__(self, n: int, events: BatchEvents):
        self.results = [None] * n
        self.emitted = [False] * n
        self.events = events

    def done(self, i: int, r) -> None:
        if self.emitted[i]:
            return
        self.emitted[i] = True
        self.events.on_item(i, r)
        self.results[i] = r

    def finish(self) -> list:
        for i in range(len(self.results)):
            if not self.emitted[i]:
                self.done(i, NotDecoded("item was not decoded"))
        return self.results


def generate(decoder, hidden, max_new: int, eos: Sequence[int] = EOS_IDS) -> Generation:
    """One segment alone on a fresh one-slot pool: prefill, then greedy steps
    until an EOS id or max_new tokens (the first token counts)."""
    seq_len = int(hidden.shape[0])
    if seq_len + max_new + 8 > decoder.max_seq:
        raise ValueError(f"seq {seq_len} + max_new {max_new} exceeds decoder max_seq "
                         f"{decoder.max_seq}")
    decoder.reset_pool(1, kv_cap(seq_len, max_new))
    first = decoder.prefill(hidden, 0, slot=0)
    gen = Generation()
    if first in eos:
        gen.stop_reason = StopReason.EOS
        return gen
    gen.ids.append(first)
    if not pipelined(decoder):
        for _ in range(1, max_new):
            tok = decoder.step([0])[0]
            if tok in eos:
                gen.stop_reason = StopReason.EOS
                break
            gen.ids.append(tok)
        return gen
    # The same max_new - 1 steps, the next one launched before this one's
    # token is read (inference.rs:2311-2347); a step launched past an EOS is
    # dropped.
    h = decoder.step_async([0]) if max_new > 1 else None
    for i in range(1, max_new):
        nh = decoder.step_async([0]) if i + 1 < max_new else None
        tok = decoder.step_result(h)[0]
        if tok in eos:
            gen.stop_reason = StopReason.EOS
            break
        gen.ids.append(tok)
        h = nh
    return gen


def _single(decoder, plans, max_news, idx, eos, events, out) -> None:
    for i in idx:
        if events.should_stop():
            r = Cancelled()
        else:
            try:
                r = generate(decoder, plans[i], max_news[i], eos)
            except Exception as e:  # charged to this segment alone
                r = e
        out.done(i, r)


def decode_batch(decoder, plans: Sequence, max_news: Sequence[int], width: int,
                 events: Optional[BatchEvents] = None,
                 eos: Sequence[int] = EOS_IDS) -> list:
    """Greedy decode of every segment in `plans` (hidden rows each), with at
    most `width` slots live at once.  Returns one Generation (or the
    exception that ended it) per segment, in input order."""
    events = events or BatchEvents()
    n = len(plans)
    if len(max_news) != n:
        raise ValueError("one max_new per segment")
    out = _Outcomes(n, events)
    lens = [int(p.shape[0]) for p in plans]
    long = [i for i in range(n) if kv_cap(lens[i], max_news[i]) > BATCH_SEQ_CAP]
    pending = [i for i in range(n) if kv_cap(lens[i], max_news[i]) <= BATCH_SEQ_CAP]
    _single(decoder, plans, max_news, long, eos, events, out)
    width = max(width, 1)
    while pending:
        if width < 2:
            # Nothing to share a weight read with: the single path.
            _single(decoder, plans, max_news, pending, eos, events, out)
            break
        ended, err = _attempt(decoder, plans, lens, max_news, pending, width, eos, events, out)
        if ended == "all":
            pending = []
        elif ended == "stopped":
            for i in pending:
                out.done(i, Cancelled())
            pending = []
        else:
            # The slots could not hold this group: halve, keep what finished.
            print(f"[batch] width {width} failed ({err}); retrying narrower", file=sys.stderr)
            width = max(width // 2, 1)
            pending = [i for i in pending if not out.emitted[i]]
    return out.finish()


def _attempt(decoder, plans, lens, max_news, run, width, eos, events, out):
    """("all" | "stopped" | "failed", the exception of a failure)."""
    nslots = min(width, len(run))
    cap = max(kv_cap(lens[i], max_news[i]) for i in run)
    try:
        decoder.reset_pool(nslots, cap)
    except Exception as e:
        return "failed", e
    gen = {i: Generation() for i in run}
    active: List[Optional[int]] = [None] * nslots
    # Longest prompt first: the step cost is the weight stream, not the live
    # slot count, so slots that finish together are what makes a batch pay.
    order = sorted(run, key=lambda i: -lens[i])
    frontier = [0]

    def fill() -> None:
        while True:
            free = [s for s in range(nslots) if active[s] is None]
            take = min(len(free), len(order) - frontier[0])
            if take == 0:
                return
            segs = order[frontier[0]:frontier[0] + take]
            firsts = decoder.prefill_batch([(free[k], plans[g]) for k, g in enumerate(segs)])
            for k, g in enumerate(segs):
                s = free[k]
                events.on_admit(g, s)
                if firsts[k] in eos:
                    # Nothing to transcribe; reported like the single path.
                    gen[g].stop_reason = StopReason.EOS
                    out.done(g, gen[g])
                else:
                    gen[g].ids.append(firsts[k])
                    active[s] = g
            frontier[0] += take

    def take(s: int, tok: int) -> bool:
        """Slot s's next token; True when it ended the slot's segment."""
        g = active[s]
        if tok in eos:
            gen[g].stop_reason = StopReason.EOS
        elif len(gen[g].ids) >= max_news[g]:
            gen[g].stop_reason = StopReason.MAX_TOKENS
        else:
            gen[g].ids.append(tok)
            return False
        active[s] = None
        out.done(g, gen[g])
        return True

    try:
        fill()
        if not pipelined(decoder):
            while any(a is not None for a in active):
                if events.should_stop():
                    return "stopped", None
                live = [s for s in range(nslots) if active[s] is not None]
                toks = dict(zip(live, decoder.step(live)))
                for s in live:
                    if take(s, toks[s]):
                        fill()
            return "all", None
        # One step in flight.  While the live slots stay the same, each step
        # is launched before the previous one's tokens are read.  When a slot
        # ends, the step in flight (which still carried it) is read too, its
        # token for the ended slot dropped, and the slots are refilled before
        # the next launch.
        live = [s for s in range(nslots) if active[s] is not None]
        h = decoder.step_async(live) if live else None
        while h is not None:
            if events.should_stop():
                return "stopped", None
            nh = decoder.step_async(live)
            ended = False
            for s, tok in zip(live, decoder.step_result(h)):
                ended |= take(s, tok)
            if ended:
                for s, tok in zip(live, decoder.step_result(nh)):
                    if active[s] is not None:
                        take(s, tok)
                fill()
                live = [s for s in range(nslots) if active[s] is not None]
                nh = decoder.step_async(live) if live else None
            h = nh
    except Exception as e:
        return "failed", e
    return "all", None
