"""Pins the oracle's whole-decoder restatement (TextDecoder, restating
src/cpu_decoder.rs:261-272 and 367-532) on small shapes, without the
reference running:

  * against NumpyDecoder, an independent float64 restatement with the same f16
    rounding points (catches any mis-wired projection, norm, residual or
    activation: the logits would move by O(spread));
  * a planted mistake (the attention residual left out of the float64 model)
    fails that comparison, so the comparison can fail;
  * exact invariants of the reference's row-independent forward: a prefill of
    s rows followed by a step equals a prefill of s + 1 rows whose last row is
    the embedding of the argmax token, and a chunked prefill equals the whole
    one -- bit for bit.
"""
from __future__ import annotations

import numpy as np

from decoder_model import NumpyDecoder, host_bits, rope_tables_f16, synth_weights

TINY = dict(hs=64, nqh=4, nkvh=2, hd=16, inter=96, layers=2, vocab=97, max_seq=64, eps=1e-6)
CAP = 64


def _setup(O, seed=11):
    W = host_bits(synth_weights(TINY, seed))
    cs, sn = rope_tables_f16(TINY["max_seq"], TINY["hd"])
    rng = np.random.default_rng(seed)
    hidden = rng.standard_normal((12, TINY["hs"])).astype(np.float16).view(np.uint16)
    return W, cs, sn, hidden


def _run(dec, hidden, steps):
    out = [dec.prefill(hidden, 0)]
    for _ in range(steps):
        out.append(dec.step())
    return out


def _max_rel(a, b):
    return max(float(np.max(np.abs(x[1] - y[1]))) / float(np.std(x[1])) for x, y in zip(a, b))


def test_decoder_oracle_matches_float64_model(O):
    W, cs, sn, hidden = _setup(O)
    got = _run(O.TextDecoder(TINY, W, CAP, cs, sn), hidden, 6)
    want = _run(NumpyDecoder(TINY, W, CAP, cs, sn), hidden, 6)
    assert _max_rel(got, want) < 5e-3
    assert [t for t, _ in got] == [t for t, _ in want]


def test_decoder_comparison_catches_planted_mistake(O):
    W, cs, sn, hidden = _setup(O)
    got = _run(O.TextDecoder(TINY, W, CAP, cs, sn), hidden, 2)
    bad = _run(NumpyDecoder(TINY, W, CAP, cs, sn, skip="attn_residual"), hidden, 2)
    assert _max_rel(got, bad) > 0.05


def test_decoder_step_equals_longer_prefill_bitwise(O):
    W, cs, sn, hidden = _setup(O, seed=12)
    a = O.TextDecoder(TINY, W, CAP, cs, sn)
    tok, _ = a.prefill(hidden, 0)
    tok2, lg_step = a.step()
    b = O.TextDecoder(TINY, W, CAP, cs, sn)
    longer = np.concatenate([hidden, W["embed"][tok][None, :]])
    tok2b, lg_pre = b.prefill(longer, 0)
    assert tok2 == tok2b and a.pos == b.pos == hidden.shape[0] + 1
    assert np.array_equal(lg_step.view(np.uint32), lg_pre.view(np.uint32))


def test_decoder_chunked_prefill_equals_whole_bitwise(O):
    W, cs, sn, hidden = _setup(O, seed=13)
    a = O.TextDecoder(TINY, W, CAP, cs, sn)
    a.prefill(hidden[:5], 0)
    tok_a, lg_a = a.prefill(hidden[5:], 5)
    b = O.TextDecoder(TINY, W, CAP, cs, sn)
    tok_b, lg_b = b.prefill(hidden, 0)
    assert tok_a == tok_b
    assert np.array_equal(lg_a.view(np.uint32), lg_b.view(np.uint32))
    sa = [a.step()[0] for _ in range(4)]
    sb = [b.step()[0] for _ in range(4)]
    assert sa == sb
