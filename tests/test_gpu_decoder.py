"""The whole text decoder on the GPU (qasr_decoder_*: rocBLAS projections,
this library's norm / SiLU / argmax kernels and attention path) against the
reference CPU decoder restated by the oracle (src/cpu_decoder.rs:367-532,
oracle's TextDecoder), on seeded random weights of the Qwen3-ASR decoder
shapes (no checkpoint exists offline).

The two sides differ by rounding (GEMM summation order, tree sums in the
norms): logits must agree to 2% of their spread at every step.  The greedy
comparison is teacher-forced: both sides take the CPU reference's previous
token at every step, and every step's argmax must agree except at a near-tie
(the CPU's top-2 margin below twice that step's logit difference), which is
counted and recorded (decoder_model.compare_teacher_forced), over a
pre-declared list of 8 seeds per test (16 distinct prompts for the 16-slot
test), at both decoder shapes.
"""
from __future__ import annotations

import numpy as np
import pytest

from decoder_model import (CFG_0P6B, CFG_1P7B, compare_teacher_forced, host_bits,
                           synth_weights)
from workloads import SEED_BASE

pytestmark = pytest.mark.gpu

# Pre-declared seed offsets of the teacher-forced greedy checks.
SEEDS = (910, 930, 940, 950, 960, 970, 980, 990)


def _prompt(seed: int, rows: int, hs: int):
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randn((rows, hs), device="cuda", generator=g).half()


def _native(cfg, W, slots, cap, max_rows=512):
    import qasr_attn

    return qasr_attn.TextDecoder(W, cfg["nqh"], cfg["nkvh"], cfg["hd"], cfg["layers"], cfg["eps"],
                                 cfg["max_seq"], slots=slots, max_rows=max_rows, cap=cap)


def _logits(vocab):
    import torch

    return torch.empty(vocab, dtype=torch.float32, device="cuda")


def _teacher_forced_single(O, cfg, wseed, label, s=40, steps=16):
    """One set of weights; for each pre-declared seed a prompt of s rows and
    `steps` teacher-forced steps, CPU reference decoder against the native
    GPU decoder (one slot, re-prefilled from position 0 per seed)."""
    from gpu_helpers import say

    W = synth_weights(cfg, SEED_BASE + wseed, device="cuda")
    Wh = host_bits(W)
    cos, sin = O.text_rope_tables_f16(cfg["max_seq"])
    dec = _native(cfg, W, 1, 1024)
    lg = _logits(cfg["vocab"])
    lgb = lg.view(1, -1)
    flips = 0
    for seed in SEEDS:
        hidden = _prompt(SEED_BASE + seed + 11, s, cfg["hs"])
        say(f"native decoder {label} seed {seed}: CPU reference decoder")
        cpu = O.TextDecoder(cfg, Wh, 1024, cos, sin)
        cpu_out = [cpu.prefill(hidden.cpu().numpy().view(np.uint16), 0)]
        for _ in range(steps):
            cpu_out.append(cpu.step())
        cpu.close()
        say(f"native decoder {label} seed {seed}: GPU")
        tok = dec.prefill(hidden, 0, logits=lg)
        gpu_out = [(tok, lg.cpu().numpy())]
        for k in range(steps):
            dec.last[0] = cpu_out[k][0]  # teacher forcing
            t = dec.step(logits=lgb)[0]
            gpu_out.append((t, lgb[0].cpu().numpy()))
        flips += compare_teacher_forced(cpu_out, gpu_out, f"native {label} seed {seed}")
    dec.close()
    print(f"native {label}: {flips} near-tie disagreements over {len(SEEDS)} seeds x {steps + 1} steps")


def test_native_decoder_teacher_forced_0p6b_single_slot(O, gpu):
    """0.6B shape, 28 layers, full vocabulary: per seed a 40-row prompt and
    16 teacher-forced steps."""
    _teacher_forced_single(O, dict(CFG_0P6B), 920, "0.6B")


def test_native_decoder_teacher_forced_1p7b_single_slot(O, gpu):
    """1.7B shape, 28 layers, full vocabulary: per seed a 40-row prompt and
    16 teacher-forced steps."""
    _teacher_forced_single(O, dict(CFG_1P7B), 1300, "1.7B")


def test_native_decoder_1p7b_16_slot_batched_steps(O, gpu):
    """1.7B shape, 28 layers, full vocabulary, 16 slots (--batch 16): each
    slot's prompt (3-18 rows, 16 distinct prompt seeds) is prefilled, then
    two teacher-forced steps run all 16 slots in one batch (the skinny GEMM's
    16-row case and 16-entry decode attention), each slot against its own
    CPU reference decoder."""
    import torch

    from gpu_helpers import say

    cfg = dict(CFG_1P7B)
    nslot, steps = 16, 2
    lens = [3 + i for i in range(nslot)]
    W = synth_weights(cfg, SEED_BASE + 1310, device="cuda")
    Wh = host_bits(W)
    cos, sin = O.text_rope_tables_f16(cfg["max_seq"])
    prompts = [_prompt(SEED_BASE + 1311 + i, L, cfg["hs"]) for i, L in enumerate(lens)]
    cpu_out = []
    for i in range(nslot):
        say(f"native decoder 1.7B x16: CPU reference, slot {i}")
        cpu = O.TextDecoder(cfg, Wh, 1024, cos, sin)
        seq = [cpu.prefill(prompts[i].cpu().numpy().view(np.uint16), 0)]
        for _ in range(steps):
            seq.append(cpu.step())
        cpu_out.append(seq)
        cpu.close()
    del Wh

    say("native decoder 1.7B x16: GPU")
    dec = _native(cfg, W, nslot, 1024)
    lg = _logits(cfg["vocab"])
    gpu_out = []
    for i in range(nslot):
        tok = dec.prefill(prompts[i], 0, slot=i, logits=lg)
        gpu_out.append([(tok, lg.cpu().numpy())])
    lgb = torch.empty((nslot, cfg["vocab"]), dtype=torch.float32, device="cuda")
    for k in range(steps):
        for i in range(nslot):
            dec.last[i] = cpu_out[i][k][0]  # teacher forcing
        toks = dec.step(list(range(nslot)), logits=lgb)
        host = lgb.cpu().numpy()
        for i in range(nslot):
            gpu_out[i].append((toks[i], host[i]))
    dec.close()
    for i in range(nslot):
        compare_teacher_forced(cpu_out[i], gpu_out[i], f"native 1.7B slot {i}")


@pytest.mark.parametrize("seed", SEEDS)
def test_native_decoder_two_slots_chunked_prefill(O, gpu, seed):
    """Two sequences, 2 layers of the 0.6B shape: prompts of 1100 and 700 rows
    prefilled in 512-row calls (max_rows), then 12 teacher-forced batched
    steps of both slots with split-K decode contexts."""
    from gpu_helpers import say

    cfg = dict(CFG_0P6B, layers=2)
    lens, steps = [1100, 700], 12
    W = synth_weights(cfg, SEED_BASE + seed, device="cuda")
    Wh = host_bits(W)
    cos, sin = O.text_rope_tables_f16(cfg["max_seq"])
    prompts = [_prompt(SEED_BASE + seed + 1 + i, L, cfg["hs"]) for i, L in enumerate(lens)]
    cpu_out = []
    for i, L in enumerate(lens):
        say(f"native decoder batch seed {seed}: CPU reference, slot {i}")
        cpu = O.TextDecoder(cfg, Wh, 2048, cos, sin)
        h = prompts[i].cpu().numpy().view(np.uint16)
        for k0 in range(0, L, 512):
            last = cpu.prefill(h[k0:k0 + 512], k0)
        seq = [last]
        for _ in range(steps):
            seq.append(cpu.step())
        cpu_out.append(seq)
        cpu.close()
    del Wh

    say(f"native decoder batch seed {seed}: GPU")
    import torch

    dec = _native(cfg, W, 2, 1024, max_rows=512)
    gpu_out = []
    lg = _logits(cfg["vocab"])
    for i in range(2):
        tok = dec.prefill(prompts[i], 0, slot=i, logits=lg)  # chunks of 512 rows inside
        gpu_out.append([(tok, lg.cpu().numpy())])
    lgb = torch.empty((2, cfg["vocab"]), dtype=torch.float32, device="cuda")
    for k in range(steps):
        for i in range(2):
            dec.last[i] = cpu_out[i][k][0]  # teacher forcing
        toks = dec.step([0, 1], logits=lgb)
        for i in range(2):
            gpu_out[i].append((toks[i], lgb[i].cpu().numpy()))
    assert dec.kv.cap >= max(lens) + steps
    dec.close()
    for i in range(2):
        compare_teacher_forced(cpu_out[i], gpu_out[i], f"native seed {seed} slot {i}")


def test_native_decoder_step_graph_replays_equal_eager(O, gpu):
    """A decoder step captured in a HIP graph: every replay (with eager work
    and synchronisations between replays) reproduces the eager step's logits
    and tokens bitwise.  The step rewrites the same KV rows each time, so
    replays are idempotent."""
    import torch

    from gpu_helpers import say

    cfg = dict(CFG_0P6B, layers=3, vocab=4096)
    W = synth_weights(cfg, SEED_BASE + 940, device="cuda")
    dec = _native(cfg, W, 4, 1024, max_rows=64)
    for i in range(4):
        dec.prefill(_prompt(SEED_BASE + 941 + i, 100 + 50 * i, cfg["hs"]), 0, slot=i)
    slots, pos = [0, 1, 2, 3], [dec.pos[i] for i in range(4)]
    tok = torch.tensor([dec.last[i] for i in range(4)], dtype=torch.int32, device="cuda")
    nxt = torch.empty(4, dtype=torch.int32, device="cuda")
    lg = torch.empty((4, cfg["vocab"]), dtype=torch.float32, device="cuda")
    say("graph test: eager step")
    dec.step_tokens(slots, pos, tok, nxt, lg)
    torch.cuda.synchronize()
    want_lg, want_tok = lg.clone(), nxt.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        dec.step_tokens(slots, pos, tok, nxt, lg)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dec.step_tokens(slots, pos, tok, nxt, lg)
    for rep in range(3):
        lg.fill_(float("nan"))
        nxt.fill_(-1)
        junk = torch.randn((512, 512), device="cuda") @ torch.randn((512, 512), device="cuda")
        torch.cuda.synchronize()
        say(f"graph test: replay {rep}")
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(lg, want_lg), f"replay {rep}: logits differ"
        assert torch.equal(nxt, want_tok), f"replay {rep}: tokens differ"
        del junk
    del graph
    dec.close()


@pytest.mark.parametrize("model,batch,lds", [("1.7B", 16, "1"), ("0.6B", 1, "1"), ("0.6B", 5, "1"),
                                             ("1.7B", 16, "2"), ("0.6B", 3, "2")])
def test_skinny_projections_match_rocblas(gpu, model, batch, lds, monkeypatch):
    """The decode-step projections (at most 16 rows: this library's MFMA
    skinny GEMMs, split across workgroups for a long K; with
    QASR_SKINNY_LDS=2 the LDS-staged kernel takes every shape it fits, not
    just the widest) against rocBLAS for the same steps (QASR_DECODER_BLAS=1):
    logits within rounding of each other, the same tokens wherever the top-2
    margin is clear."""
    import torch

    from decoder_model import CFG_1P7B
    from gpu_helpers import say

    cfg = dict(CFG_1P7B if model == "1.7B" else CFG_0P6B, layers=3)
    W = synth_weights(cfg, SEED_BASE + 950 + batch, device="cuda")
    dec = _native(cfg, W, batch, 1024, max_rows=16)
    for i in range(batch):
        dec.prefill(_prompt(SEED_BASE + 960 + i, 30 + 7 * i, cfg["hs"]), 0, slot=i)
    slots, pos = list(range(batch)), [dec.pos[i] for i in range(batch)]
    tok = torch.tensor([dec.last[i] for i in range(batch)], dtype=torch.int32, device="cuda")
    monkeypatch.setenv("QASR_SKINNY_LDS", lds)
    out = {}
    for name, blas in (("skinny", "0"), ("rocblas", "1")):
        monkeypatch.setenv("QASR_DECODER_BLAS", blas)
        nxt = torch.empty(batch, dtype=torch.int32, device="cuda")
        lg = torch.empty((batch, cfg["vocab"]), dtype=torch.float32, device="cuda")
        say(f"{model} batch {batch}: step via {name}")
        dec.step_tokens(slots, pos, tok, nxt, lg)
        torch.cuda.synchronize()
        out[name] = (nxt.cpu().numpy(), lg.cpu().numpy())
    dec.close()
    t2, l2 = out["rocblas"]
    spread = float(np.std(l2))
    for name in ("skinny",):
        t1, l1 = out[name]
        diff = float(np.max(np.abs(l1 - l2)))
        say(f"{name}: max logit diff {diff:.3g} (spread {spread:.3g})")
        # f16 roundings between the layers turn summation-order differences
        # into last-bit flips; a wrong operand layout would differ by the
        # spread itself.
        assert diff <= 2e-2 * spread
        for b in range(batch):
            top = np.partition(l2[b], -2)[-2:]
            if top[1] - top[0] > 2 * diff:
                assert t1[b] == t2[b], f"{name} entry {b}: {t1[b]} vs {t2[b]} at a clear margin"


def test_decoder_from_checkpoint_equals_decoder_from_weights(gpu, tmp_path):
    """checkpoint.open_text_decoder over a synthetic HF-native checkpoint (two
    shards + index, some tensors stored as f32 holding f16 values, config.json
    in the transformers-native layout) runs the same decoder as TextDecoder
    over the in-memory weights: identical tokens and logits, bitwise."""
    import json

    import torch
    from safetensors.torch import save_file

    import checkpoint
    from gpu_helpers import say

    cfg = dict(CFG_0P6B, layers=2, vocab=4096)
    W = synth_weights(cfg, SEED_BASE + 970, device="cuda")
    names = {"embed": "model.language_model.embed_tokens.weight",
             "norm": "model.language_model.norm.weight"}
    for l in range(cfg["layers"]):
        for key, suffix in checkpoint._LAYER_TENSORS:
            names[(l, key)] = f"model.language_model.layers.{l}.{suffix}"
    shards = [{}, {}]
    index = {}
    for i, (k, n) in enumerate(sorted(names.items(), key=lambda kv: kv[1])):
        t = W[k].cpu()
        shards[i % 2][n] = t.float() if i % 3 == 0 else t  # f32 copies of f16 values are exact
        index[n] = f"model-0000{i % 2 + 1}-of-00002.safetensors"
    for j, sh in enumerate(shards):
        save_file(sh, str(tmp_path / f"model-0000{j + 1}-of-00002.safetensors"))
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": index}))
    (tmp_path / "config.json").write_text(json.dumps({"text_config": {
        "vocab_size": cfg["vocab"], "hidden_size": cfg["hs"], "intermediate_size": cfg["inter"],
        "num_hidden_layers": cfg["layers"], "num_attention_heads": cfg["nqh"],
        "num_key_value_heads": cfg["nkvh"], "head_dim": cfg["hd"], "rms_norm_eps": cfg["eps"],
        "rope_parameters": {"rope_theta": 1000000, "rope_type": "default"}}}))

    hidden = _prompt(SEED_BASE + 971, 33, cfg["hs"])
    runs = []
    for label in ("weights", "checkpoint"):
        say(f"decoder from {label}")
        dec = (_native(cfg, W, 1, 1024) if label == "weights"
               else checkpoint.open_text_decoder(str(tmp_path), slots=1, max_rows=512))
        lg = torch.empty((1, cfg["vocab"]), dtype=torch.float32, device="cuda")
        toks = [dec.prefill(hidden, 0, logits=lg[0])]
        lgs = [lg.cpu().numpy().copy()]
        for _ in range(6):
            toks.append(dec.step(logits=lg)[0])
            lgs.append(lg.cpu().numpy().copy())
        dec.close()
        runs.append((toks, np.stack(lgs)))
    assert runs[0][0] == runs[1][0]
    assert np.array_equal(runs[0][1], runs[1][1])


PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def _quantize_rows(w):
    """Symmetric per-row int8 of an f16 [out][in] matrix: (q, f32 scales)."""
    import torch

    s = (w.float().abs().amax(dim=1) / 127.0).clamp_min(1e-8)
    q = torch.round(w.float() / s[:, None]).clamp(-128, 127).to(torch.int8)
    return q.contiguous(), s.contiguous()


@pytest.mark.parametrize("model,batch,blas", [("1.7B", 16, "0"), ("0.6B", 1, "0"), ("0.6B", 3, "1")])
def test_int8_projections_equal_dequantized_f16(gpu, model, batch, blas, monkeypatch):
    """Resident int8 projections (per-row f32 scale; the reference's int8
    checkpoints, weights.rs:296-427) against the same decoder over f16
    weights dequantized on the host as f16(q * s): the decode steps (int8
    skinny GEMM that dequantizes in registers, or rocBLAS over a dequantized
    copy when QASR_DECODER_BLAS=1) and the prefill (dequantized copy +
    rocBLAS) must give identical tokens and logits, bitwise."""
    import torch

    from decoder_model import CFG_1P7B
    from gpu_helpers import say

    monkeypatch.setenv("QASR_DECODER_BLAS", blas)
    cfg = dict(CFG_1P7B if model == "1.7B" else CFG_0P6B, layers=3, vocab=8192)
    W = synth_weights(cfg, SEED_BASE + 980 + batch, device="cuda")
    W8, Wdq = dict(W), dict(W)
    for key in list(W):
        if isinstance(key, tuple) and key[1] in PROJECTIONS:
            q, s = _quantize_rows(W[key])
            W8[key], W8[(key[0], key[1] + "_scale")] = q, s
            Wdq[key] = (q.float() * s[:, None]).half()
    del W
    runs = []
    for label, weights in (("int8", W8), ("f16", Wdq)):
        say(f"{model} batch {batch} blas={blas}: decoder over {label} weights")
        dec = _native(cfg, weights, batch, 1024, max_rows=64)
        lg = torch.empty((batch, cfg["vocab"]), dtype=torch.float32, device="cuda")
        toks, lgs = [], []
        for i in range(batch):
            toks.append(dec.prefill(_prompt(SEED_BASE + 990 + i, 70 + 9 * i, cfg["hs"]), 0,
                                    slot=i, logits=lg[i]))
        lgs.append(lg.cpu().numpy().copy())
        for _ in range(5):
            toks.extend(dec.step(logits=lg))
            lgs.append(lg.cpu().numpy().copy())
        dec.close()
        runs.append((toks, np.stack(lgs)))
    assert runs[0][0] == runs[1][0]
    assert np.array_equal(runs[0][1], runs[1][1])


@pytest.mark.parametrize("model,batch,int8,lds", [("1.7B", 16, False, "1"), ("0.6B", 1, False, "1"),
                                                  ("0.6B", 3, False, "1"), ("1.7B", 2, False, "1"),
                                                  ("1.7B", 16, True, "1"), ("0.6B", 5, True, "1"),
                                                  ("0.6B", 4, True, "1"), ("1.7B", 16, False, "2"),
                                                  ("0.6B", 5, True, "2")])
def test_fused_epilogues_equal_unfused(gpu, model, batch, int8, lds, monkeypatch):
    """The decode step's fusions -- the input, post-attention and final
    RMSNorms folded into the qkv, gate|up and logits projections, and gate|up
    with SiLU * up in one skinny launch -- against the same step with them off
    (QASR_DECODER_FUSE=0: rms_norm_kernel launches, gate|up, then
    silu_mul_kernel): identical logits and tokens, bitwise -- the fusion moves
    where values are rounded to f16, not how."""
    import torch

    from decoder_model import CFG_1P7B
    from gpu_helpers import say

    cfg = dict(CFG_1P7B if model == "1.7B" else CFG_0P6B, layers=3, vocab=8192)
    W = synth_weights(cfg, SEED_BASE + 1200 + batch, device="cuda")
    if int8:
        for key in list(W):
            if isinstance(key, tuple) and key[1] in PROJECTIONS:
                q, s = _quantize_rows(W[key])
                W[key], W[(key[0], key[1] + "_scale")] = q, s
    dec = _native(cfg, W, batch, 1024, max_rows=16)
    for i in range(batch):
        dec.prefill(_prompt(SEED_BASE + 1210 + i, 9 + 3 * i, cfg["hs"]), 0, slot=i)
    slots, pos = list(range(batch)), [dec.pos[i] for i in range(batch)]
    tok = torch.tensor([dec.last[i] for i in range(batch)], dtype=torch.int32, device="cuda")
    monkeypatch.setenv("QASR_SKINNY_LDS", lds)
    out = {}
    for name, fuse in (("fused", "1"), ("unfused", "0")):
        monkeypatch.setenv("QASR_DECODER_FUSE", fuse)
        nxt = torch.empty(batch, dtype=torch.int32, device="cuda")
        lg = torch.empty((batch, cfg["vocab"]), dtype=torch.float32, device="cuda")
        say(f"{model} batch {batch} int8={int8}: {name} step")
        dec.step_tokens(slots, pos, tok, nxt, lg)
        torch.cuda.synchronize()
        out[name] = (nxt.cpu().numpy(), lg.cpu().numpy())
    dec.close()
    assert np.array_equal(out["fused"][0], out["unfused"][0])
    assert np.array_equal(out["fused"][1], out["unfused"][1])


@pytest.mark.parametrize("model,batch", [("1.7B", 16), ("0.6B", 1), ("0.6B", 9), ("1.7B", 3)])
def test_argmax_from_logits_tiles_equals_two_pass(gpu, model, batch, monkeypatch):
    """The greedy token from the logits kernel's per-tile candidates
    (argmax_tiles_kernel) against the two passes over the f32 logits
    (QASR_ARGMAX_TILES=0) and numpy's first maximal index, with ties planted:
    the tied embedding repeats 256 distinct rows in adjacent pairs and every
    512 columns, so each logit value occurs 32 times, inside a 16-column tile
    and across tiles.  The smaller index must win, as the reference's
    `if v > logits[best]` loop keeps the first maximum.  Also without logits
    requested (the scratch logits are then not written)."""
    import torch

    from decoder_model import CFG_1P7B
    from gpu_helpers import say

    cfg = dict(CFG_1P7B if model == "1.7B" else CFG_0P6B, layers=2, vocab=8192)
    W = synth_weights(cfg, SEED_BASE + 1300 + batch, device="cuda")
    base = W["embed"][:256].clone()
    idx = torch.arange(cfg["vocab"], device="cuda")
    W["embed"] = base[(idx % 512) // 2].contiguous()
    dec = _native(cfg, W, batch, 1024, max_rows=16)
    for i in range(batch):
        dec.prefill(_prompt(SEED_BASE + 1310 + i, 7 + 2 * i, cfg["hs"]), 0, slot=i)
    slots, pos = list(range(batch)), [dec.pos[i] for i in range(batch)]
    tok = torch.tensor([dec.last[i] for i in range(batch)], dtype=torch.int32, device="cuda")
    out = {}
    for name, tiles, want_logits in (("tiles", "1", True), ("tiles, no logits", "1", False),
                                     ("two-pass", "0", True)):
        monkeypatch.setenv("QASR_ARGMAX_TILES", tiles)
        nxt = torch.empty(batch, dtype=torch.int32, device="cuda")
        lg = torch.empty((batch, cfg["vocab"]), dtype=torch.float32, device="cuda") if want_logits else None
        say(f"{model} batch {batch}: {name}")
        dec.step_tokens(slots, pos, tok, nxt, lg)
        torch.cuda.synchronize()
        out[name] = (nxt.cpu().numpy(), lg.cpu().numpy() if want_logits else None)
    dec.close()
    logits = out["two-pass"][1]
    first_max = np.argmax(logits, axis=1).astype(np.int32)
    # the planted ties: the first copy of each value (an even index below 512) wins
    assert (first_max < 512).all() and (first_max % 2 == 0).all()
    assert np.array_equal(out["two-pass"][0], first_max)
    assert np.array_equal(out["tiles"][0], first_max)
    assert np.array_equal(out["tiles, no logits"][0], first_max)
    assert np.array_equal(out["tiles"][1], logits)


@pytest.mark.parametrize("variant", ["shared=2", "shared=3", "shared=4", "multi=2", "multi=3", "multi=4"])
@pytest.mark.parametrize("model,batch,int8", [("1.7B", 16, False), ("1.7B", 8, True),
                                              ("0.6B", 16, True), ("0.6B", 9, False)])
def test_wide_projection_variants_equal_per_tile(gpu, model, batch, int8, variant, monkeypatch):
    """The decode step's projections through the kernels that cut activation
    reloads -- activation rows shared in LDS by several column tiles
    (QASR_SKINNY_SHARED, skinny_shared_kernel) or several column tiles per
    wave (QASR_SKINNY_MULTI, skinny_multi_kernel, f16 weights), both with the
    per-tile kernel's K slices, summation order and norm rounding -- against
    the per-tile kernel alone: identical logits and tokens, bitwise -- at both
    model shapes, f16 and int8, with the folded norms, gate|up with SiLU * up,
    the residual projections and down_proj's K split across workgroups."""
    import torch

    from decoder_model import CFG_1P7B
    from gpu_helpers import say

    knob, value = variant.split("=")
    cfg = dict(CFG_1P7B if model == "1.7B" else CFG_0P6B, layers=3, vocab=8192)
    W = synth_weights(cfg, SEED_BASE + 1300 + batch, device="cuda")
    if int8:
        for key in list(W):
            if isinstance(key, tuple) and key[1] in PROJECTIONS:
                q, s = _quantize_rows(W[key])
                W[key], W[(key[0], key[1] + "_scale")] = q, s
    dec = _native(cfg, W, batch, 1024, max_rows=16)
    for i in range(batch):
        dec.prefill(_prompt(SEED_BASE + 1310 + i, 7 + 2 * i, cfg["hs"]), 0, slot=i)
    slots, pos = list(range(batch)), [dec.pos[i] for i in range(batch)]
    tok = torch.tensor([dec.last[i] for i in range(batch)], dtype=torch.int32, device="cuda")
    out = {}
    monkeypatch.setenv("QASR_SKINNY_SHARED_MIN_TILES", "0")  # every eligible projection, not only the widest
    for name, shared, multi in (("per_tile", "0", "0"),
                                (variant, value if knob == "shared" else "0", value if knob == "multi" else "0")):
        monkeypatch.setenv("QASR_SKINNY_SHARED", shared)
        monkeypatch.setenv("QASR_SKINNY_MULTI", multi)
        nxt = torch.empty(batch, dtype=torch.int32, device="cuda")
        lg = torch.empty((batch, cfg["vocab"]), dtype=torch.float32, device="cuda")
        say(f"{model} batch {batch} int8={int8}: {name} step")
        dec.step_tokens(slots, pos, tok, nxt, lg)
        torch.cuda.synchronize()
        out[name] = (nxt.cpu().numpy(), lg.cpu().numpy())
    dec.close()
    assert np.array_equal(out[variant][0], out["per_tile"][0])
    assert np.array_equal(out[variant][1], out["per_tile"][1])


@pytest.mark.parametrize("model,int8", [("1.7B", False), ("0.6B", True)])
def test_prefill_own_gemm_close_to_rocblas(gpu, model, int8, monkeypatch):
    """The prefill projections through the build's own MFMA GEMM
    (QASR_PREFILL_GEMM=own: gemm.hip, f32 accumulation in another order than
    rocBLAS, the same rounding points) against rocBLAS: a 300-row prompt and
    three decode steps after it give logits within 2% of their spread, and
    the same token wherever the top-2 margin exceeds 2% of the spread."""
    import torch

    from decoder_model import CFG_1P7B
    from gpu_helpers import say

    cfg = dict(CFG_1P7B if model == "1.7B" else CFG_0P6B, layers=3, vocab=8192)
    W = synth_weights(cfg, SEED_BASE + 1400, device="cuda")
    if int8:
        for key in list(W):
            if isinstance(key, tuple) and key[1] in PROJECTIONS:
                q, s = _quantize_rows(W[key])
                W[key], W[(key[0], key[1] + "_scale")] = q, s
    runs = {}
    for gemm in ("blas", "own"):
        monkeypatch.setenv("QASR_PREFILL_GEMM", gemm)
        say(f"{model} int8={int8}: prefill projections through {gemm}")
        dec = _native(cfg, W, 1, 1024, max_rows=512)
        lg = torch.empty((1, cfg["vocab"]), dtype=torch.float32, device="cuda")
        toks = [dec.prefill(_prompt(SEED_BASE + 1410, 300, cfg["hs"]), 0, slot=0, logits=lg[0])]
        lgs = [lg.cpu().numpy().copy()]
        for _ in range(3):
            toks.extend(dec.step(logits=lg))
            lgs.append(lg.cpu().numpy().copy())
        dec.close()
        runs[gemm] = (toks, np.concatenate(lgs))
    (tb, lb), (to, lo) = runs["blas"], runs["own"]
    for i in range(lb.shape[0]):
        spread = float(lb[i].max() - lb[i].min())
        assert np.abs(lo[i] - lb[i]).max() <= 0.02 * spread, f"row {i}"
        top2 = np.sort(lb[i])[-2:]
        if top2[1] - top2[0] > 0.02 * spread:
            assert to[i] == tb[i], f"row {i}: token {to[i]} against {tb[i]}"
