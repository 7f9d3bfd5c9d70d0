"""End-to-end greedy check: the attention path inside a whole decoder.

The north-star parity requirement beyond per-stage tolerances: with this
library's stage (a) + attention in every layer (qasr_prefill_layer for the
prompt, qasr_decode_step for each generated token), the per-step argmax
equals the reference CPU decoder's (src/cpu_decoder.rs, restated by the
oracle's TextDecoder) on identical seeded weights and inputs.

Everything outside the attention path runs in torch on the GPU (test
plumbing, f32 math with the reference's f16 rounding points); the two sides
differ by rounding, so the logits agree to a small fraction of their spread.
The comparison is teacher-forced: at every step both sides take the CPU
reference's previous token, and every step's argmax must agree except at a
near-tie (the CPU's top-2 margin below twice that step's measured logit
difference), which is counted and recorded (decoder_model.
compare_teacher_forced).  Each test runs the same pre-declared list of 8
seeds, among them the ones the earlier free-running check used (910/911).
No checkpoint exists offline, so the weights are seeded random weights of
the Qwen3-ASR decoder shapes.
"""
from __future__ import annotations

import numpy as np
import pytest

from decoder_model import CFG_0P6B, GpuDecoder, compare_teacher_forced, host_bits, synth_weights
from workloads import SEED_BASE

pytestmark = pytest.mark.gpu

# Pre-declared seed offsets (weights seed = SEED_BASE + s, prompts from s + 1).
SEEDS = (910, 930, 940, 950, 960, 970, 980, 990)


def _cap(need: int) -> int:
    return max(1024, (need + 255) // 256 * 256)


def _prompt(seed: int, rows: int, hs: int):
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randn((rows, hs), device="cuda", generator=g).half()


def test_e2e_teacher_forced_0p6b_shape_single_slot(O, gpu):
    """0.6B decoder shape, all 28 layers, full vocabulary (one set of
    weights): for each seed a 40-row prompt, then 16 teacher-forced steps."""
    from gpu_helpers import say

    cfg = dict(CFG_0P6B)
    s, steps = 40, 16
    cap = _cap(s + steps + 1)
    say("e2e 0.6B: weights")
    W = synth_weights(cfg, SEED_BASE + 900, device="cuda")
    Wh = host_bits(W)
    cos, sin = O.text_rope_tables_f16(cfg["max_seq"])
    dec = GpuDecoder(cfg, W, slots=1, cap=cap)
    flips = 0
    for seed in SEEDS:
        hidden = _prompt(SEED_BASE + seed + 1, s, cfg["hs"])
        say(f"e2e 0.6B seed {seed}: CPU reference decoder")
        cpu = O.TextDecoder(cfg, Wh, cap, cos, sin)
        cpu_out = [cpu.prefill(hidden.cpu().numpy().view(np.uint16), 0)]
        for _ in range(steps):
            cpu_out.append(cpu.step())
        cpu.close()
        say(f"e2e 0.6B seed {seed}: GPU decoder (library attention path)")
        tok, lg = dec.prefill(0, hidden, 0)
        gpu_out = [(tok, lg)]
        for k in range(steps):
            toks, lgs = dec.step([0], [s + k], [cpu_out[k][0]])
            gpu_out.append((toks[0], lgs[0]))
        flips += compare_teacher_forced(cpu_out, gpu_out, f"0.6B seed {seed}")
    dec.close()
    print(f"0.6B: {flips} near-tie disagreements over {len(SEEDS)} seeds x {steps + 1} steps")


@pytest.mark.parametrize("seed", SEEDS)
def test_e2e_teacher_forced_two_slots_chunked_prefill_split_decode(O, gpu, seed):
    """Two sequences in one KV pool (the reference's --batch 2), 2 layers of
    the 0.6B shape: prompts of 1100 and 700 rows prefilled in 512-row chunks
    (kv_start > 0), then 12 teacher-forced steps of batched decode over both
    slots, whose contexts take split-K decode."""
    from gpu_helpers import say

    cfg = dict(CFG_0P6B, layers=2)
    lens, steps, chunk = [1100, 700], 12, 512
    cap = _cap(max(lens) + steps + 1)
    W = synth_weights(cfg, SEED_BASE + seed, device="cuda")
    Wh = host_bits(W)
    cos, sin = O.text_rope_tables_f16(cfg["max_seq"])
    prompts = [_prompt(SEED_BASE + seed + 1 + i, L, cfg["hs"]) for i, L in enumerate(lens)]

    cpu_out = []
    for i, L in enumerate(lens):
        say(f"e2e batch seed {seed}: CPU reference decoder, slot {i}")
        cpu = O.TextDecoder(cfg, Wh, cap, cos, sin)
        h = prompts[i].cpu().numpy().view(np.uint16)
        for k0 in range(0, L, chunk):
            last = cpu.prefill(h[k0:k0 + chunk], k0)
        seq = [last]
        for _ in range(steps):
            seq.append(cpu.step())
        cpu_out.append(seq)
        cpu.close()
    del Wh

    say(f"e2e batch seed {seed}: GPU decoder, chunked prefill then batched steps")
    dec = GpuDecoder(cfg, W, slots=2, cap=cap)
    gpu_out = []
    for i, L in enumerate(lens):
        for k0 in range(0, L, chunk):
            last = dec.prefill(i, prompts[i][k0:k0 + chunk], k0)
        gpu_out.append([last])
    for k in range(steps):
        toks, lgs = dec.step([0, 1], [L + k for L in lens], [cpu_out[0][k][0], cpu_out[1][k][0]])
        for i in range(2):
            gpu_out[i].append((toks[i], lgs[i]))
    dec.close()
    for i in range(2):
        compare_teacher_forced(cpu_out[i], gpu_out[i], f"seed {seed} slot {i}")
