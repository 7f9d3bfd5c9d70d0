"""Batched serving on the GPU: qasr_decoder_prefill_batch (prefill_batch /
prefill_multi, decoder.rs:3599-3700) and the slot scheduler (serving.py,
inference.rs:707-764, 1944-2227) against this library's single-sequence
path, on seeded random weights of the 0.6B decoder shape (3 layers).

The reference's batched output is byte-identical to `--batch 1`
(README "byte-identical"; decoder.rs:686-693, 1930-1931), and so is this
library's: a prefill's projections run one GEMM whose per-element K order
does not depend on the row count, its attention runs each prompt's own
plan, a decode step's projections run the kernels of a lone slot's step
(groups of at most 16 rows) and its attention cuts each slot's keys by the
slot's own length.  So batched and single paths agree bitwise here: logits,
KV rows and every token of every stream."""
from __future__ import annotations

import numpy as np
import pytest

from decoder_model import CFG_0P6B, synth_weights
from workloads import SEED_BASE

pytestmark = pytest.mark.gpu

CFG = dict(CFG_0P6B, layers=3, vocab=4096)


def _prompt(seed, rows):
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randn((rows, CFG["hs"]), device="cuda", generator=g).half()


def _decoder(W, slots, max_rows=512, cap=1024):
    import qasr_attn

    c = CFG
    return qasr_attn.TextDecoder(W, c["nqh"], c["nkvh"], c["hd"], c["layers"], c["eps"],
                                 c["max_seq"], slots=slots, max_rows=max_rows, cap=cap)


@pytest.fixture(scope="module")
def weights(gpu):
    return synth_weights(CFG, SEED_BASE + 1100, device="cuda")


def _prefill_both(W, lens, seed):
    import torch

    from gpu_helpers import say

    hidden = [_prompt(seed + i, n) for i, n in enumerate(lens)]
    n = len(lens)
    say(f"prefill_batch of {n} segments, rows {lens}")
    a = _decoder(W, n)
    lg_a = torch.empty((n, CFG["vocab"]), dtype=torch.float32, device="cuda")
    tok_a = a.prefill_batch([(i, h) for i, h in enumerate(hidden)], logits=lg_a)
    b = _decoder(W, n)
    lg_b = torch.empty_like(lg_a)
    tok_b = [b.prefill(h, 0, slot=i, logits=lg_b[i]) for i, h in enumerate(hidden)]
    torch.cuda.synchronize()
    return a, b, tok_a, tok_b, lg_a.cpu().numpy(), lg_b.cpu().numpy()


def test_prefill_batch_short_segments_bitwise(weights):
    """16 rows in all: the same bits as one prefill per slot, logits and KV."""
    a, b, tok_a, tok_b, lg_a, lg_b = _prefill_both(weights, [2, 5, 3, 6], SEED_BASE + 1110)
    assert tok_a == tok_b
    assert np.array_equal(lg_a, lg_b)
    ka, kb = a.kv.tensor(), b.kv.tensor()
    for i, n in enumerate([2, 5, 3, 6]):
        assert ka[i, :, :, :, :n].equal(kb[i, :, :, :, :n]), f"slot {i} KV differs"
    assert a.pos == b.pos and a.last == b.last
    # a step of all four slots after either prefill is the same step
    assert a.step() == b.step()
    a.close()
    b.close()


def test_prefill_batch_long_segments_bitwise(weights):
    """474 rows in one batched prefill (GEMM projections, attention split
    plans per prompt): the same logits, tokens and KV rows, bit for bit, as
    one prefill per slot."""
    lens = [100, 37, 260, 77]
    a, b, tok_a, tok_b, lg_a, lg_b = _prefill_both(weights, lens, SEED_BASE + 1120)
    assert tok_a == tok_b
    assert np.array_equal(lg_a, lg_b)
    ka, kb = a.kv.tensor(), b.kv.tensor()
    for i, n in enumerate(lens):
        assert ka[i, :, :, :, :n].equal(kb[i, :, :, :, :n]), f"slot {i} KV differs"
    assert a.step() == b.step()
    a.close()
    b.close()


def _quantized(W):
    import torch

    W8 = dict(W)
    for key in list(W):
        if isinstance(key, tuple) and key[1].endswith("_proj"):
            w = W[key].float()
            s = (w.abs().amax(dim=1) / 127.0).clamp_min(1e-8)
            W8[key] = torch.round(w / s[:, None]).clamp(-128, 127).to(torch.int8)
            W8[(key[0], key[1] + "_scale")] = s
    return W8


@pytest.mark.parametrize("int8", [False, True])
def test_decode_step_bits_independent_of_batch(weights, int8):
    """A slot's decode steps alone, inside a batch of 5 and inside a batch
    of 20 (two groups: 16 + 4 rows) give the same logits and tokens bit for
    bit, step after step, for f16 and int8 weights; the prompt itself is
    prefilled alone, in a batch of 5 and in a batch of 20."""
    import torch

    from gpu_helpers import say

    W = _quantized(weights) if int8 else weights
    shared = _prompt(SEED_BASE + 1180, 33)
    others = [_prompt(SEED_BASE + 1181 + i, 5 + 7 * i) for i in range(19)]
    runs = {}
    for n in (1, 5, 20):
        say(f"int8={int8}: slot 0 among {n} slots")
        dec = _decoder(W, n)
        lg = torch.empty((n, CFG["vocab"]), dtype=torch.float32, device="cuda")
        if n == 1:
            toks = [dec.prefill(shared, 0, slot=0, logits=lg[0])]
        else:
            toks = [dec.prefill_batch([(0, shared)] + [(i, others[i - 1]) for i in range(1, n)],
                                      logits=lg)[0]]
        lgs = [lg[0].cpu().numpy().copy()]
        for _ in range(6):
            toks.append(dec.step(logits=lg)[0])
            lgs.append(lg[0].cpu().numpy().copy())
        runs[n] = (toks, np.stack(lgs))
        dec.close()
    for n in (5, 20):
        assert runs[n][0] == runs[1][0], n
        assert np.array_equal(runs[n][1], runs[1][1]), n


def test_prefill_batch_rejects_bad_segments(weights):
    import qasr_attn

    dec = _decoder(weights, 2, max_rows=64)
    h = _prompt(SEED_BASE + 1130, 40)
    with pytest.raises(qasr_attn.QasrError, match="share a slot"):
        dec.prefill_batch([(0, h), (0, h)])
    # 80 rows over max_rows 64: split into two calls, same result as separate
    toks = dec.prefill_batch([(0, h), (1, h)])
    assert toks[0] == toks[1]
    dec.close()


def _single_with_margins(dec, plans, max_news, eos):
    """The single path (serving.generate) with the top-2 margin of every token
    and the spread (standard deviation) of each prompt's first logits."""
    import torch

    import serving

    out = []
    for h, m in zip(plans, max_news):
        dec.reset_pool(1, serving.kv_cap(int(h.shape[0]), m))
        lg = torch.empty((1, CFG["vocab"]), dtype=torch.float32, device="cuda")
        first = dec.prefill(h, 0, slot=0, logits=lg[0])
        spread = float(lg[0].std())
        ids, margins = [], []

        def margin():
            t = torch.topk(lg[0], 2).values
            return float(t[0] - t[1])

        if first not in eos:
            ids.append(first)
            margins.append(margin())
            for _ in range(1, m):
                tok = dec.step([0], logits=lg)[0]
                margins.append(margin())
                if tok in eos:
                    break
                ids.append(tok)
        out.append((ids, margins, spread))
    return out


def _run_both(weights, lens, max_news, width, seed, eos=()):
    import serving
    from gpu_helpers import say

    plans = [_prompt(seed + i, n) for i, n in enumerate(lens)]
    dec = _decoder(weights, 1)
    say(f"single path over {len(lens)} segments")
    single = _single_with_margins(dec, plans, max_news, eos)
    plain = serving.decode_batch(dec, plans, max_news, 1, eos=eos)
    say(f"scheduler at width {width}")
    batched = serving.decode_batch(dec, plans, max_news, width, eos=eos)
    dec.close()
    return single, plain, batched


def test_scheduler_short_prompts_bitwise(weights):
    """Prompts of 2-6 rows (the first admission is 16 rows): every segment's
    tokens from width 3 equal the single path's, including EOS stops."""
    lens = [4, 5, 6, 3, 2, 5, 4, 4]
    max_news = [9, 12, 7, 10, 12, 8, 11, 6]
    single, plain, _ = _run_both(weights, lens, max_news, 3, SEED_BASE + 1140)
    # an EOS id that occurs in some streams, so some segments stop early
    eos = (single[0][0][3], single[5][0][2])
    single, plain, batched = _run_both(weights, lens, max_news, 3, SEED_BASE + 1140, eos=eos)
    stopped_early = 0
    for g in range(len(lens)):
        assert plain[g].ids == single[g][0], g
        assert batched[g].ids == single[g][0], g
        stopped_early += len(batched[g].ids) < max_news[g]
    assert stopped_early >= 2


def test_scheduler_long_prompts_bitwise(weights):
    """Prompts of 40-300 rows at width 4 (GEMM prefills of several prompts at
    once, decode over contexts of hundreds of keys): every segment's tokens
    equal the single path's."""
    rng = np.random.default_rng(11)
    lens = [int(x) for x in rng.integers(40, 300, size=10)]
    max_news = [int(x) for x in rng.integers(8, 24, size=10)]
    single, plain, batched = _run_both(weights, lens, max_news, 4, SEED_BASE + 1150)
    for g in range(len(lens)):
        ids = single[g][0]
        assert plain[g].ids == ids, g
        assert batched[g].ids == ids, g


def test_scheduler_width_past_16_bitwise(weights):
    """Width 20 over 24 segments: decode steps of up to 20 rows (groups of 16
    + 4) and prefills of up to 20 prompts; every segment's tokens equal the
    single path's."""
    rng = np.random.default_rng(12)
    lens = [int(x) for x in rng.integers(3, 120, size=24)]
    max_news = [int(x) for x in rng.integers(4, 14, size=24)]
    single, plain, batched = _run_both(weights, lens, max_news, 20, SEED_BASE + 1155)
    for g in range(len(lens)):
        ids = single[g][0]
        assert plain[g].ids == ids, g
        assert batched[g].ids == ids, g


def test_decoder_prefill_batch_abi_refuses_bad_segments(weights):
    """The C ABI's own checks (the Python wrapper catches some of these
    first): a shared slot, an empty segment, more rows than max_rows, more
    than 64 segments -- each refused with QASR_EINVAL before any launch."""
    import ctypes

    import torch

    import qasr_attn

    dec = _decoder(weights, 4, max_rows=64)
    lib = qasr_attn.load()
    hidden = torch.zeros((80, CFG["hs"]), dtype=torch.float16, device="cuda")
    nxt = torch.zeros(70, dtype=torch.int32, device="cuda")

    def call(segs):
        arr = (qasr_attn.Segment * len(segs))(*[qasr_attn.Segment(*sg) for sg in segs])
        return lib.qasr_decoder_prefill_batch(dec.handle, dec.kv.handle, arr, len(segs),
                                              ctypes.c_void_p(hidden.data_ptr()),
                                              ctypes.c_void_p(nxt.data_ptr()), None, None)

    assert call([(0, 0, 10), (0, 0, 10)]) == qasr_attn.QASR_EINVAL
    assert call([(0, 0, 10), (1, 0, 0)]) == qasr_attn.QASR_EINVAL
    assert call([(0, 0, 40), (1, 0, 40)]) == qasr_attn.QASR_EINVAL  # 80 rows > max_rows 64
    assert call([(i % 4, 0, 1) for i in range(65)]) == qasr_attn.QASR_EINVAL
    assert call([(0, 0, 10), (1, 0, 10)]) == qasr_attn.QASR_OK
    torch.cuda.synchronize()
    dec.close()


def test_pipelined_steps_equal_synchronous_steps(weights):
    """step_async / step_result (tokens fed back on the device, one step in
    flight) give the synchronous step()'s tokens, step for step."""
    prompts = [_prompt(SEED_BASE + 1160 + i, 20 + 13 * i) for i in range(3)]
    runs = []
    for mode in ("sync", "pipelined"):
        dec = _decoder(weights, 3)
        dec.prefill_batch([(i, h) for i, h in enumerate(prompts)])
        toks = []
        if mode == "sync":
            for _ in range(12):
                toks.append(dec.step())
        else:
            h = dec.step_async([0, 1, 2])
            for k in range(12):
                nh = dec.step_async([0, 1, 2]) if k + 1 < 12 else None
                toks.append(dec.step_result(h))
                h = nh
        runs.append((toks, list(dec.pos)))
        dec.close()
    assert runs[0] == runs[1]


def test_int8_prefill_batch_equals_dequantized_f16(weights):
    """Int8 projections through the batched prefill (the layer's matrix
    dequantised for the GEMM) against f16 weights dequantised on the host:
    identical tokens and logits, bitwise."""
    import torch

    W8, Wdq = dict(weights), dict(weights)
    for key in list(weights):
        if isinstance(key, tuple) and key[1].endswith("_proj"):
            w = weights[key].float()
            s = (w.abs().amax(dim=1) / 127.0).clamp_min(1e-8)
            q = torch.round(w / s[:, None]).clamp(-128, 127).to(torch.int8)
            W8[key], W8[(key[0], key[1] + "_scale")] = q, s
            Wdq[key] = (q.float() * s[:, None]).half()
    prompts = [_prompt(SEED_BASE + 1170 + i, n) for i, n in enumerate((30, 50, 20))]
    out = []
    for W in (W8, Wdq):
        dec = _decoder(W, 3)
        lg = torch.empty((3, CFG["vocab"]), dtype=torch.float32, device="cuda")
        toks = dec.prefill_batch([(i, h) for i, h in enumerate(prompts)], logits=lg)
        out.append((toks, lg.cpu().numpy()))
        dec.close()
    assert out[0][0] == out[1][0]
    assert np.array_equal(out[0][1], out[1][1])
