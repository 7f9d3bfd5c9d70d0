#!/usr/bin/env python3
"""Benchmark of the MI355X Qwen3-ASR decoder self-attention path.

Headline (BASELINE.json metric, config 3): one decode step of the 1.7B decoder
shape (16 q / 8 kv heads, head_dim 128) for 16 slots with ragged contexts
U[400, 2400], across 28 layers.  Each layer is one launch of the fused stage
(a)+(b) kernel (q/k RMSNorm + MRoPE + KV append + split-K GQA attention) on
its own KV cache, so the working set (~2.6 GB of K/V) is far beyond the
256 MB Infinity Cache.  The 28 launches are captured in one HIP graph and
replayed; the timed region is K replays bracketed by events and syncs.

value = algorithmic bytes / time (GB/s), bytes per slot-layer =
  4096*(L+1) (K+V rows) + 8192 (Q, O) + 16384 (stage (a) row in/out).
Also reported: configs 1, 2, 4, 5 (us/layer, GB/s, TFLOP/s with causal-exact
FLOPs 4*hd*nqh*sum_r(kv_start+r+1)), the roofline of the dominant kernel, and
the reference CPU path (the C++ restatement of cpu_decoder.rs in oracle/)
timed on a bounded sample of config 3 on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
                       [--only decode3|decode1|decode4|decode5|decode16x2k|prefill2|prefill4|
                               config4_whole|streamread|streamread_per_cu|mfma_ceiling|copycal|
                               decoder16|decoder1|
                               decoder16_int8|decoder1_int8|serving|prefill_batch|prefill_one|
                               gemm]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "qwen3-asr-wgpu_amd")
sys.path.insert(0, PKG)

METRIC = "decode attn µs/layer + HBM GB/s; prefill attn TFLOP/s (1.7B shape, 1 GPU)"
NQH, NKVH, HD, LAYERS = 16, 8, 128, 28
TOT = (NQH + 2 * NKVH) * HD
QDIM = NQH * HD
SEED_BASE = 0x51A50000
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, vendor figure
MFMA_F16_PEAK_TFS = 2500.0  # MI355X dense fp16 MFMA, vendor figure


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def splitmix_lengths(seed: int, n: int, lo: int, hi: int):
    """Per-slot lengths U[lo, hi] from SplitMix64 (the tests' generator)."""
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


def decode_bytes(lengths):
    """Algorithmic bytes of one decode layer: lengths = keys attended (pos+1)."""
    return sum(4096 * L + 8192 + 16384 for L in lengths)


def prefill_flops(s: int, kv_start: int) -> float:
    return 4.0 * HD * NQH * sum(kv_start + r + 1 for r in range(s))


def cap_for(need: int) -> int:
    return max(1024, (need + 255) // 256 * 256)


class Setup:
    def __init__(self, slots: int, cap: int, layers: int = LAYERS):
        import torch

        import qasr_attn

        self.torch = torch
        self.q = qasr_attn
        self.ctx = qasr_attn.Context(NQH, NKVH, HD, layers, 1e-6, 16384, 0)
        c, s = qasr_attn.mrope_text_tables(16384)
        self.ctx.set_rope_tables(c, s)
        self.kv = qasr_attn.KVPool(self.ctx, slots, cap)
        pool = self.kv.tensor()
        g = torch.Generator(device="cuda")
        g.manual_seed(1234)
        for sl in range(pool.shape[0]):  # synthetic cache contents, N(0,1) f16
            pool[sl].normal_(generator=g)
        self.layers = layers
        gains = torch.randn((layers, 2, HD), device="cuda", generator=g) * 0.1 + 1.0
        self.gains = gains.half().contiguous()

    def close(self):
        self.kv.close()
        self.ctx.close()


def graph_time(torch, fn_step, steps: int, warmup: int):
    """Capture fn_step (a sequence of launches on the current stream) in a HIP
    graph, replay `warmup` times, then time `steps` replays with events."""
    fn_step()  # eager: argument checks, lazy workspace growth
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn_step()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    return ms, graph


def bench_decode(slots: int, lengths, steps: int, warmup: int, layers: int = LAYERS):
    """Fused stage (a)+(b) decode step over `layers` layers; lengths = cached
    positions per slot before the step (the step attends lengths[i]+1 keys)."""
    import torch

    st = Setup(slots, cap_for(max(lengths) + 1), layers)
    g = torch.Generator(device="cuda")
    g.manual_seed(99)
    qkv = torch.randn((layers, slots, TOT), device="cuda", generator=g).half()
    out = torch.empty((layers, slots, QDIM), device="cuda", dtype=torch.float16)
    pos = list(lengths)

    def step():
        for l in range(layers):
            st.q.decode_step(st.ctx, st.kv, l, pos, qkv[l], st.gains[l, 0], st.gains[l, 1], out[l])

    ms, graph = graph_time(torch, step, steps, warmup)
    del graph
    nbytes = decode_bytes([L + 1 for L in lengths]) * layers
    st.close()
    return {"ms_per_step": ms, "us_per_layer": ms * 1e3 / layers,
            "bytes_per_step": nbytes, "GBps": nbytes / (ms * 1e-3) / 1e9}


def bench_prefill(s: int, kv_start: int, steps: int, warmup: int, layers: int = LAYERS):
    """Stage (c) prefill attention of s rows at kv_start, per layer on its own
    cache; stage (a) timed separately."""
    import torch

    st = Setup(1, cap_for(kv_start + s), layers)
    g = torch.Generator(device="cuda")
    g.manual_seed(98)
    q = torch.randn((layers, s, QDIM), device="cuda", generator=g).half()
    qkv = torch.randn((layers, s, TOT), device="cuda", generator=g).half()
    out = torch.empty((layers, s, QDIM), device="cuda", dtype=torch.float16)
    qw = torch.empty((layers, s, QDIM), device="cuda", dtype=torch.float16)

    def attn():
        for l in range(layers):
            st.q.prefill_attn(st.ctx, st.kv, l, 0, kv_start, s, q[l], out[l])

    def stage_a():
        for l in range(layers):
            st.q.qk_norm_rope_append(st.ctx, st.kv, l, [(0, kv_start, s)], qkv[l],
                                     st.gains[l, 0], st.gains[l, 1], qw[l])

    ms_a, g1 = graph_time(torch, attn, steps, warmup)
    ms_s, g2 = graph_time(torch, stage_a, steps, warmup)
    del g1, g2
    fl = prefill_flops(s, kv_start)
    st.close()
    us = ms_a * 1e3 / layers
    return {"us_per_layer": us, "TFLOPs": fl / (us * 1e-6) / 1e12, "flops_per_layer": fl,
            "stage_a_us_per_layer": ms_s * 1e3 / layers}


def copy_calibration(steps: int):
    """A plain device copy of 1 GiB (reads 1 GiB, writes 1 GiB): the reference
    point for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes."""
    import torch

    x = torch.empty(512 * 1024 * 1024, dtype=torch.float16, device="cuda").normal_()
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(max(1, steps)):
        y.copy_(x)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / max(1, steps)
    return {"bytes_read": x.numel() * 2, "bytes_written": y.numel() * 2, "ms": ms,
            "GBps_rw": 2 * x.numel() * 2 / (ms * 1e-3) / 1e9}


def mfma_calibration(wgs: int = 256, mfma_iters: int = 20000):
    """Matrix-core calibration by qasr_mfma_probe, one workgroup per CU:
    - the densest v_mfma_f32_32x32x16_f16 stream (four independent chains per
      wave, one and two waves per SIMD), as TFLOP/s and as a fraction of the
      2.5 PFLOP/s dense f16 peak, with the shader clock under that load
      (s_memtime against the 100 MHz s_memrealtime);
    - a softmax-shaped VALU block (the prefill kernel's per-score mix, and
      each of its instructions alone) in one wave of each SIMD while the
      other wave streams MFMAs, and what fraction of the shorter part the
      overlap hid: 1 = fully hidden, 0 = serial.
    - the same blocks interleaved inside every wave (one and two waves per
      SIMD), the schedule of a kernel overlapping its own softmax and MFMAs.
    The prefill kernel's MFMA fraction is read against these."""
    import torch

    import qasr_attn

    ctx = qasr_attn.Context(NQH, NKVH, HD, LAYERS, 1e-6, 16384, 0)
    sink = torch.empty(wgs * 8, dtype=torch.float32, device="cuda")
    clk = torch.zeros(4, dtype=torch.int64, device="cuda")

    def run(mode, waves, mi, vi, reps=5):
        for _ in range(2):
            qasr_attn.mfma_probe(ctx, mode, wgs, waves, mi, vi, sink, clk)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            qasr_attn.mfma_probe(ctx, mode, wgs, waves, mi, vi, sink, clk)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        c = [int(x) for x in clk.cpu().tolist()]
        ghz = (c[2] - c[0]) / max(1, c[3] - c[1]) * 0.1  # shader cycles per 10 ns tick
        return us, ghz

    flop = lambda waves, mi: wgs * waves * mi * 4 * 32768.0
    out = {"workgroups": wgs, "mfma_iters": mfma_iters}
    for _ in range(20):  # the shader clock ramps up under the first launches
        qasr_attn.mfma_probe(ctx, 0, wgs, 4, mfma_iters, 0, sink, clk)
    torch.cuda.synchronize()
    for waves in (4, 8):
        us, ghz = run(0, waves, mfma_iters, 0)
        tf = flop(waves, mfma_iters) / (us * 1e-6) / 1e12
        out[f"mfma_only_{waves // 4}_wave_per_simd"] = {
            "us": round(us, 1), "TFLOPs": round(tf, 1), "frac_of_peak": round(tf / MFMA_F16_PEAK_TFS, 4),
            "shader_GHz": round(ghz, 3)}
    t_m, _ = run(0, 4, mfma_iters, 0)
    out["mfma_only_us"] = round(t_m, 1)
    # VALU blocks (qasr_mfma_probe mode / 4): the prefill softmax's whole
    # mix, and its instructions one kind at a time; iterations scaled so the
    # VALU part alone takes about as long as the MFMA part.
    kinds = {"softmax_mix": 0, "exp_only": 1, "fma_only": 2, "dot2_only": 3, "cvt_pk_only": 4,
             "max3_only": 5, "softmax_mix_f32_sum": 6}
    out["mfma_and_valu_in_different_waves_of_a_simd"] = {}
    for name, kind in kinds.items():
        t1, _ = run(1 + 4 * kind, 4, 0, 1000)
        vi = max(100, int(1000 * t_m / t1))
        t_v, _ = run(1 + 4 * kind, 4, 0, vi)
        t_split, ghz_s = run(2 + 4 * kind, 8, mfma_iters, vi)
        out["mfma_and_valu_in_different_waves_of_a_simd"][name] = {
            "valu_iters": vi, "valu_only_us": round(t_v, 1), "together_us": round(t_split, 1),
            "hidden_fraction": round((t_m + t_v - t_split) / min(t_m, t_v), 3),
            "shader_GHz": round(ghz_s, 3)}
    # The same blocks interleaved inside every wave (probe mode 3): the
    # schedule of a kernel that overlaps its own softmax with its own MFMAs,
    # at one and at two waves per SIMD.
    out["mfma_and_valu_in_the_same_wave"] = {}
    for waves in (4, 8):
        t_mw, _ = run(0, waves, mfma_iters, 0)
        for name in ("softmax_mix", "softmax_mix_f32_sum"):
            kind = kinds[name]
            t1, _ = run(1 + 4 * kind, waves, 0, 1000)
            vi = max(100, int(1000 * t_mw / t1))
            t_v, _ = run(1 + 4 * kind, waves, 0, vi)
            t_both, ghz_b = run(3 + 4 * kind, waves, mfma_iters, vi)
            out["mfma_and_valu_in_the_same_wave"][f"{name}_{waves // 4}_wave_per_simd"] = {
                "valu_iters": vi, "mfma_only_us": round(t_mw, 1), "valu_only_us": round(t_v, 1),
                "together_us": round(t_both, 1),
                "hidden_fraction": round((t_mw + t_v - t_both) / min(t_mw, t_v), 3),
                "shader_GHz": round(ghz_b, 3)}
    ctx.close()
    return out


def stream_read_calibration(nbytes: int, steps: int, warmup: int, copies: int = LAYERS,
                            shapes=((256, 4), (256, 8), (512, 4), (512, 8), (1024, 4))):
    """A bare streaming read of `nbytes` per launch (config 3's decode bytes
    by default) by qasr_stream_read: non-temporal dwordx4 buffer loads as in
    the decode kernel, one contiguous share per workgroup, no compute.
    `copies` distinct buffers rotate (2.6 GB at config 3, beyond the 256 MB
    Infinity Cache), 28 launches per HIP-graph replay as in bench_decode.
    Returns the time per launch for each (workgroups, waves) shape: what HBM
    delivers to one launch of this size, the ceiling the decode kernel's
    bandwidth is read against."""
    import torch

    import qasr_attn

    ctx = qasr_attn.Context(NQH, NKVH, HD, LAYERS, 1e-6, 16384, 0)
    out = {"bytes_per_launch": None, "copies": copies, "shapes": {}}
    best = None
    for wgs, waves in shapes:
        per = -(-nbytes // (wgs * 16)) * 16
        total = per * wgs
        out["bytes_per_launch"] = total
        bufs = [torch.empty(total // 2, dtype=torch.float16, device="cuda").normal_()
                for _ in range(copies)]
        sink = torch.empty(wgs * waves, dtype=torch.int32, device="cuda")

        def step():
            for b in bufs:
                qasr_attn.stream_read(ctx, b, wgs, waves, sink)

        ms, graph = graph_time(torch, step, steps, warmup)
        del graph
        us = ms * 1e3 / copies
        gbs = total / (us * 1e-6) / 1e9
        out["shapes"][f"{wgs}x{waves}"] = {"us_per_launch": round(us, 3), "GBps": round(gbs, 1),
                                           "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4)}
        if best is None or us < best[0]:
            best = (us, gbs, f"{wgs}x{waves}")
        del bufs
        torch.cuda.empty_cache()
    ctx.close()
    out["best"] = {"shape": best[2], "us_per_launch": round(best[0], 3), "GBps": round(best[1], 1),
                   "frac_of_peak": round(best[1] / HBM_PEAK_GBS, 4)}
    return out


def stream_per_cu_calibration(steps: int, warmup: int, per_wg: int = 1216 * 1024,
                              counts=(8, 32, 128, 256), waves=(4, 8)):
    """What one CU streams: qasr_stream_read with few workgroups (at most one
    per CU), each reading `per_wg` contiguous bytes (about the largest config-3
    entry's K+V of one kv head), four rotating buffers per count so that no
    launch reads data the previous one left in the Infinity Cache.  A CU's
    rate does not rise when others are idle: the decode planner keeps most
    CUs streaming until the end for that reason."""
    import torch

    import qasr_attn

    ctx = qasr_attn.Context(NQH, NKVH, HD, LAYERS, 1e-6, 16384, 0)
    out = {"bytes_per_workgroup": per_wg, "shapes": {}}
    for w in waves:
        for n in counts:
            total = n * per_wg
            bufs = [torch.empty(total // 2, dtype=torch.float16, device="cuda").normal_() for _ in range(4)]
            sink = torch.empty(n * w, dtype=torch.int32, device="cuda")

            def step():
                for b in bufs:
                    qasr_attn.stream_read(ctx, b, n, w, sink)

            ms, graph = graph_time(torch, step, steps, warmup)
            del graph
            us = ms * 1e3 / len(bufs)
            out["shapes"][f"{n}x{w}"] = {"us_per_launch": round(us, 2),
                                        "GBps_per_workgroup": round(per_wg / (us * 1e-6) / 1e9, 1),
                                        "GBps": round(total / (us * 1e-6) / 1e9, 1)}
            del bufs
            torch.cuda.empty_cache()
    ctx.close()
    return out


def bench_config4_whole(steps: int, warmup: int, layers: int = LAYERS, decode_steps: int = 64):
    """Config 4 as its workload states it: per layer (each on its own cache),
    16 chunked prefills of 512 rows at kv_start = 0, 512, .., 7680 (stage (a)
    + attention per chunk), then 64 decode steps at positions 8192..8255
    (fused stage (a)+(b)).  One replay = the prefill phase of all 28 layers
    chunk by chunk, then the decode phase step by step (layer-major inside a
    step, as a decoder runs them); both phases are timed separately."""
    import torch

    chunks, chunk, ctx_len = 16, 512, 8192
    st = Setup(1, cap_for(ctx_len + decode_steps), layers)
    g = torch.Generator(device="cuda")
    g.manual_seed(97)
    qkv = torch.randn((layers, ctx_len, TOT), device="cuda", generator=g).half()
    qw = torch.empty((layers, chunk, QDIM), device="cuda", dtype=torch.float16)
    out = torch.empty((layers, chunk, QDIM), device="cuda", dtype=torch.float16)
    dq = torch.randn((decode_steps, layers, 1, TOT), device="cuda", generator=g).half()
    dout = torch.empty((layers, 1, QDIM), device="cuda", dtype=torch.float16)

    def prefill_phase():
        for c in range(chunks):
            for l in range(layers):
                st.q.prefill_layer(st.ctx, st.kv, l, 0, c * chunk, chunk,
                                   qkv[l, c * chunk:(c + 1) * chunk], st.gains[l, 0],
                                   st.gains[l, 1], qw[l], out[l])

    def decode_phase():
        for t in range(decode_steps):
            for l in range(layers):
                st.q.decode_step(st.ctx, st.kv, l, [ctx_len + t], dq[t, l], st.gains[l, 0],
                                 st.gains[l, 1], dout[l])

    ms_p, g1 = graph_time(torch, prefill_phase, steps, warmup)
    ms_d, g2 = graph_time(torch, decode_phase, steps, warmup)
    del g1, g2
    st.close()
    fl = sum(prefill_flops(chunk, c * chunk) for c in range(chunks)) * layers
    dbytes = sum(decode_bytes([ctx_len + t + 1]) for t in range(decode_steps)) * layers
    return {"prefill_ms": ms_p, "prefill_TFLOPs_attention_and_stage_a": fl / (ms_p * 1e-3) / 1e12,
            "prefill_us_per_layer_chunk": ms_p * 1e3 / (layers * chunks),
            "decode_ms": ms_d, "decode_us_per_layer_step": ms_d * 1e3 / (layers * decode_steps),
            "decode_GBps": dbytes / (ms_d * 1e-3) / 1e9, "total_ms": ms_p + ms_d,
            "layers": layers, "chunks": chunks, "decode_steps": decode_steps}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


DECODERS = {"0.6B": dict(hs=1024, inter=3072), "1.7B": dict(hs=2048, inter=6144)}
VOCAB = 151936


def decoder_weights(hs: int, inter: int, layers: int = LAYERS, seed: int = 7, int8: bool = False):
    """Random f16 weights of the Qwen3 text decoder shapes (values do not
    change the timing; no checkpoint exists offline).  With `int8` the seven
    linears of each layer are stored as the reference's int8 checkpoints hold
    them: int8 [out][in] with an f32 scale per row (embedding and norms stay
    f16)."""
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    qd, kd = NQH * HD, NKVH * HD

    def mat(rows, cols):
        return (torch.randn((rows, cols), device="cuda", generator=g) * cols ** -0.5).half()

    def gain(n):
        return (torch.randn(n, device="cuda", generator=g) * 0.1 + 1.0).half()

    W = {"embed": (torch.randn((VOCAB, hs), device="cuda", generator=g) * 0.1).half(),
         "norm": gain(hs)}
    for l in range(layers):
        W[(l, "input_layernorm")], W[(l, "post_attention_layernorm")] = gain(hs), gain(hs)
        W[(l, "q_norm")], W[(l, "k_norm")] = gain(HD), gain(HD)
        W[(l, "q_proj")], W[(l, "k_proj")], W[(l, "v_proj")] = mat(qd, hs), mat(kd, hs), mat(kd, hs)
        W[(l, "o_proj")] = mat(hs, qd)
        W[(l, "gate_proj")], W[(l, "up_proj")] = mat(inter, hs), mat(inter, hs)
        W[(l, "down_proj")] = mat(hs, inter)
    if int8:
        for key in [k for k in W if isinstance(k, tuple) and k[1].endswith("_proj")]:
            w = W[key].float()
            s = w.abs().amax(dim=1).clamp_min(1e-8) / 127.0
            W[key] = torch.round(w / s[:, None]).clamp(-128, 127).to(torch.int8)
            W[(key[0], key[1] + "_scale")] = s
    return W


def bench_text_decoder(model: str, lengths, steps: int, warmup: int, int8: bool = False):
    """One greedy token step of the whole text decoder (qasr_decoder_step:
    28 layers of norms, projections, this library's attention, MLP; logits and
    argmax) for len(lengths) slots at those cached lengths, HIP-graph replay.
    The weights are streamed once per step: their bytes over the step time is
    the step's weight bandwidth."""
    import torch

    import qasr_attn

    dims = DECODERS[model]
    W = decoder_weights(dims["hs"], dims["inter"], int8=int8)
    wbytes = sum(t.numel() * t.element_size() for t in W.values())
    b = len(lengths)
    dec = qasr_attn.TextDecoder(W, NQH, NKVH, HD, LAYERS, 1e-6, 16384, slots=b, max_rows=max(b, 16),
                                cap=cap_for(max(lengths) + 1))
    del W
    slots, pos = list(range(b)), list(lengths)
    tok = torch.randint(0, VOCAB, (b,), dtype=torch.int32, device="cuda")
    nxt = torch.empty(b, dtype=torch.int32, device="cuda")
    ms, graph = graph_time(torch, lambda: dec.step_tokens(slots, pos, tok, nxt), steps, warmup)
    del graph
    dec.close()
    torch.cuda.empty_cache()
    return {"model": model, "slots": b, "weights": "int8" if int8 else "f16",
            "us_per_step": ms * 1e3, "weight_bytes": wbytes,
            "weight_GBps": wbytes / (ms * 1e-3) / 1e9}


def bench_serving(model: str, segments: int, width: int, max_new: int, seed: int = 21):
    """A batch job through the slot scheduler (serving.decode_batch: prompts
    prefilled together, longest first, all live slots stepped together, a
    finished slot refilled at once) against the same job one segment at a
    time (width 1).  Prompts of U[150, 450] rows (12-36 s of audio); random
    weights never emit an EOS id, so every segment generates max_new tokens.
    Wall-clock, host scheduling included."""
    import numpy as np
    import torch

    import qasr_attn
    import serving

    dims = DECODERS[model]
    W = decoder_weights(dims["hs"], dims["inter"])
    dec = qasr_attn.TextDecoder(W, NQH, NKVH, HD, LAYERS, 1e-6, 16384, slots=1, max_rows=8192,
                                cap=1024)
    del W
    rng = np.random.default_rng(seed)
    lens = [int(x) for x in rng.integers(150, 450, size=segments)]
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    plans = [torch.randn((n, dims["hs"]), device="cuda", generator=g).half() for n in lens]
    out = {"model": model, "segments": segments, "max_new": max_new,
           "prompt_rows": int(sum(lens))}
    serving.decode_batch(dec, plans[:2], [4, 4], 2)  # warm-up: rocBLAS, allocator
    for w in (width, 1):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        res = serving.decode_batch(dec, plans, [max_new] * segments, w)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        toks = sum(len(r.ids) for r in res)
        out[f"width{w}"] = {"seconds": dt, "tokens": toks, "tokens_per_s": toks / dt}
    dec.close()
    torch.cuda.empty_cache()
    out["speedup"] = out[f"width{width}"]["tokens_per_s"] / out["width1"]["tokens_per_s"]
    return out


def bench_prefill_one(model: str, rows: int, steps: int, warmup: int, seed: int = 29):
    """qasr_decoder_prefill of one prompt of `rows` rows through 28 layers
    (the time to the first token of one segment)."""
    import torch

    import qasr_attn

    dims = DECODERS[model]
    W = decoder_weights(dims["hs"], dims["inter"])
    dec = qasr_attn.TextDecoder(W, NQH, NKVH, HD, LAYERS, 1e-6, 16384, slots=1, max_rows=4096,
                                cap=cap_for(rows + 1))
    del W
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    hidden = torch.randn((rows, dims["hs"]), device="cuda", generator=g).half()
    for _ in range(warmup):
        dec.prefill(hidden)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dec.prefill(hidden)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    dec.close()
    torch.cuda.empty_cache()
    return {"model": model, "rows": rows, "ms": dt * 1e3, "rows_per_s": rows / dt}


GEMM_SHAPES = [(4269, 4096, 2048, False), (4269, 2048, 2048, True), (4269, 12288, 2048, False),
               (4269, 2048, 6144, True), (420, 4096, 2048, False), (420, 2048, 2048, True),
               (420, 12288, 2048, False), (420, 2048, 6144, True), (16384, 12288, 2048, False)]


def bench_gemm(steps: int, warmup: int, seed: int = 31):
    """The build's prefill GEMM (qasr_gemm_f16) against the vendor BLAS
    (torch.mm / addmm) at the 1.7B projections' shapes: the batched prefill's
    4,269 rows, one prompt's down_proj, and a large square-ish product.  Event
    timing on the current stream, operands resident."""
    import torch

    import qasr_attn

    ctx = qasr_attn.Context()
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    out = []

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / steps

    for m, n, k, acc in GEMM_SHAPES:
        a = torch.randn((m, k), device="cuda", generator=g).half()
        b = (torch.randn((n, k), device="cuda", generator=g) * 0.05).half()
        c = torch.zeros((m, n), device="cuda", dtype=torch.float16)
        bt = b.t()
        t_own = timed(lambda: qasr_attn.gemm_f16(ctx, a, b, c, accumulate=acc))
        t_lib = timed(lambda: c.addmm_(a, bt) if acc else torch.mm(a, bt, out=c))
        fl = 2.0 * m * n * k
        out.append({"m": m, "n": n, "k": k, "residual": acc, "own_us": round(t_own, 1),
                    "library_us": round(t_lib, 1), "own_TFLOPs": round(fl / t_own / 1e6, 1),
                    "library_TFLOPs": round(fl / t_lib / 1e6, 1)})
        del a, b, c, bt
    ctx.close()
    torch.cuda.empty_cache()
    return out


def bench_prefill_batch(model: str, segments: int, steps: int, warmup: int, seed: int = 23):
    """qasr_decoder_prefill_batch over `segments` prompts of U[150, 450] rows
    (projections once over all rows, attention per segment), 28 layers:
    prompt rows per second and projection TFLOP/s (2 x weights x rows)."""
    import numpy as np
    import torch

    import qasr_attn

    dims = DECODERS[model]
    W = decoder_weights(dims["hs"], dims["inter"])
    proj_params = sum(t.numel() for k, t in W.items() if isinstance(k, tuple) and k[1].endswith("_proj"))
    dec = qasr_attn.TextDecoder(W, NQH, NKVH, HD, LAYERS, 1e-6, 16384, slots=segments,
                                max_rows=8192, cap=1024)
    del W
    rng = np.random.default_rng(seed)
    lens = [int(x) for x in rng.integers(150, 450, size=segments)]
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    items = [(i, torch.randn((n, dims["hs"]), device="cuda", generator=g).half())
             for i, n in enumerate(lens)]
    for _ in range(warmup):
        dec.prefill_batch(items)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dec.prefill_batch(items)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    dec.close()
    torch.cuda.empty_cache()
    rows = sum(lens)
    return {"model": model, "segments": segments, "rows": rows, "ms": dt * 1e3,
            "rows_per_s": rows / dt, "projection_TFLOPs": 2.0 * proj_params * rows / dt / 1e12}


def cpu_baseline(lengths, budget_s: float = 10.0):
    """Reference CPU path (C++ restatement of cpu_decoder.rs, oracle/) on config
    3: stage (a) + attention for each of the 16 slots, one layer at a time,
    repeated until `budget_s` of CPU time is spent.  Returns GB/s-equivalent
    (same algorithmic bytes) and us/layer."""
    import numpy as np

    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or O.hardware_threads()
    threads = max(1, min(threads, O.hardware_threads()))
    cap = cap_for(max(lengths) + 1)
    sh = O.make_shape()
    rng = O.Rng(SEED_BASE + 3)
    tab_c, tab_s = O.text_rope_tables_f16(cap)
    cos, sin = O.f32_from_f16(tab_c), O.f32_from_f16(tab_s)
    qg = rng.normal_f16((HD,), 1.0, 0.1)
    kg = rng.normal_f16((HD,), 1.0, 0.1)
    caches = []
    for L in lengths:
        k = np.zeros((NKVH, cap, HD), np.float32)
        v = np.zeros((NKVH, cap, HD), np.float32)
        k[:, :L] = O.f32_from_f16(rng.normal_f16((NKVH, L, HD)))
        v[:, :L] = O.f32_from_f16(rng.normal_f16((NKVH, L, HD)))
        caches.append((k, v))
    rows = rng.normal_f16((len(lengths), TOT))
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        for i, L in enumerate(lengths):
            O.layer_attn(sh, cap, rows[i:i + 1], L, qg, kg, cos, sin, caches[i][0], caches[i][1],
                         nthreads=threads)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    nbytes = decode_bytes([L + 1 for L in lengths])
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_layer": med * 1e6, "cpu_model": cpu_model(),
            "sample": f"config 3 decode layer-steps (16 slots, lengths as the GPU run), "
                      f"{len(times)} reps over ~{budget_s:.0f} s, median; oracle/oracle.cpp "
                      f"(C++ restatement of cpu_decoder.rs:274-423, f32), {threads} threads"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline config only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="", help="run one workload (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(no multi-GPU path is built; decode would shard by slot with no exchange, one "
              "process per GPU)", file=sys.stderr)
        sys.exit(2)

    import torch

    import qasr_attn

    qasr_attn.load()
    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    K, W = args.steps, args.warmup
    lens3 = splitmix_lengths(SEED_BASE + 3, 16, 400, 2400)

    only = args.only
    if only:
        runs = {
            "decode3": lambda: bench_decode(16, lens3, K, W),
            "decode1": lambda: bench_decode(1, [511], K, W),
            "decode4": lambda: bench_decode(1, [8192], K, W),
            "decode5": lambda: bench_decode(64, splitmix_lengths(SEED_BASE + 5, 64, 64, 4096), K, W),
            "decode16x2k": lambda: bench_decode(16, [2048] * 16, K, W),
            "prefill2": lambda: bench_prefill(420, 0, K, W),
            "prefill4": lambda: bench_prefill(512, 7680, K, W),
            "copycal": lambda: copy_calibration(K),
            "streamread": lambda: stream_read_calibration(decode_bytes([L + 1 for L in lens3]), K, W),
            "streamread_per_cu": lambda: stream_per_cu_calibration(K, W),
            "mfma_ceiling": lambda: mfma_calibration(),
            "config4_whole": lambda: bench_config4_whole(max(3, K // 10), 1),
            "decoder16": lambda: bench_text_decoder("1.7B", lens3, K, W),
            "decoder1": lambda: bench_text_decoder("0.6B", [511], K, W),
            "decoder16_int8": lambda: bench_text_decoder("1.7B", lens3, K, W, int8=True),
            "decoder1_int8": lambda: bench_text_decoder("0.6B", [511], K, W, int8=True),
            "serving": lambda: bench_serving("1.7B", 32, 16, 48),
            "prefill_batch": lambda: bench_prefill_batch("1.7B", 16, max(3, K // 10), 1),
            "prefill_one": lambda: bench_prefill_one("1.7B", 420, max(5, K // 5), 2),
            "gemm": lambda: bench_gemm(max(5, K // 5), 3),
        }
        log(json.dumps({only: runs[only]()}))
        return

    log(f"[bench] config 3: 16 slots, lengths {lens3}")
    d3 = bench_decode(16, lens3, K, W)
    log(f"[bench] config 3: {d3['us_per_layer']:.2f} us/layer, {d3['GBps']:.0f} GB/s")
    extra = {}
    if not args.quick:
        log("[bench] config 1")
        extra["config1_decode"] = bench_decode(1, [511], K, W)
        log("[bench] config 2")
        extra["config2_prefill"] = bench_prefill(420, 0, K, W)
        log("[bench] config 4 (last 512-row chunk at kv_start 7680; decode at 8192)")
        extra["config4_prefill_last_chunk"] = bench_prefill(512, 7680, K, W)
        extra["config4_decode"] = bench_decode(1, [8192], K, W)
        log("[bench] config 4 whole workload (16 chunked prefills + 64 decode steps, 28 layers)")
        extra["config4_whole_workload"] = bench_config4_whole(max(3, K // 10), 1)
        log("[bench] config 5")
        lens5 = splitmix_lengths(SEED_BASE + 5, 64, 64, 4096)
        extra["config5_decode"] = bench_decode(64, lens5, max(5, K // 5), W)
        log("[bench] 16 slots at a uniform 2048-token context (the target's ~2k context)")
        extra["decode_16slots_2k_context"] = bench_decode(16, [2048] * 16, K, W)
        log("[bench] text decoder steps (whole decoder around the attention path)")
        extra["text_decoder_1p7b_16slots"] = bench_text_decoder("1.7B", lens3, K, W)
        extra["text_decoder_0p6b_1slot"] = bench_text_decoder("0.6B", [511], K, W)
        extra["text_decoder_1p7b_16slots_int8"] = bench_text_decoder("1.7B", lens3, K,
                                                                     W, int8=True)
        extra["text_decoder_0p6b_1slot_int8"] = bench_text_decoder("0.6B", [511], K,
                                                                   W, int8=True)
        log("[bench] whole-decoder prefill: one 420-row prompt, 16 prompts batched")
        extra["decoder_prefill_1p7b_420rows"] = bench_prefill_one("1.7B", 420, max(5, K // 5), 2)
        extra["decoder_prefill_batch_1p7b_16prompts"] = bench_prefill_batch("1.7B", 16, max(3, K // 10), 1)
        log("[bench] batch job through the slot scheduler (32 segments, width 16 vs 1)")
        extra["serving_1p7b_32seg_width16"] = bench_serving("1.7B", 32, 16, 48)
        # Calibrations last: the matrix-core probe's long dense launches can
        # leave the clocks lower for whatever runs right after them.
        log("[bench] streaming-read calibration at config 3's bytes per launch")
        extra["streamread_config3_bytes"] = stream_read_calibration(
            decode_bytes([L + 1 for L in lens3]), K, W)
        log("[bench] what one CU streams (few workgroups)")
        extra["stream_per_cu"] = stream_per_cu_calibration(max(5, K // 5), 2)
        log("[bench] matrix-core calibration")
        extra["mfma_calibration"] = mfma_calibration()
        for k, v in extra.items():
            log(f"[bench] {k}: {json.dumps(v)}")

    us = d3["us_per_layer"]
    per_launch_bytes = decode_bytes([L + 1 for L in lens3])
    achieved = per_launch_bytes / (us * 1e-6) / 1e9
    traffic = traffic_pf = None
    tf = os.path.join(REPO, "profiles", "decode_attn_traffic.json")
    if os.path.exists(tf):
        try:
            tj = json.load(open(tf))
            traffic = tj.get("config3_hbm_bytes_per_launch")
            traffic_pf = tj.get("prefill4_hbm_bytes_per_launch")
        except Exception:
            traffic = traffic_pf = None
    if "config4_prefill_last_chunk" in extra:
        p4 = extra["config4_prefill_last_chunk"]
        extra["roofline_prefill_config4"] = {
            "bound": "mfma", "kernel": "prefill_attn_kernel (512 rows at kv_start 7680)",
            "achieved": round(p4["TFLOPs"], 1), "peak": MFMA_F16_PEAK_TFS, "unit": "TFLOP/s",
            "frac": round(p4["TFLOPs"] / MFMA_F16_PEAK_TFS, 4), "traffic": traffic_pf,
            "flops_per_launch": p4["flops_per_layer"], "avg_launch_us": round(p4["us_per_layer"], 3)}
    roofline = {"bound": "hbm", "kernel": "decode_attn_kernel<true> (fused stage a+b)",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "bytes_per_launch": per_launch_bytes, "avg_launch_us": round(us, 3)}
    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (oracle) ...")
        cpu = cpu_baseline(lens3)
        log(f"[bench] cpu baseline {cpu['us_per_layer']:.0f} us/layer on {cpu['cores']} threads")
    line = {
        "metric": METRIC,
        "value": round(d3["GBps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(d3["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "config3: decode step of the 1.7B decoder shape (16 q / 8 kv "
                               "heads, hd 128), 16 slots, ragged contexts U[400,2400], 28 "
                               "layers (fused q/k-norm+MRoPE+KV append+GQA attention per "
                               "layer, HIP-graph replay)",
                   "global_batch": 16, "seq_len": int(max(lens3) + 1), "parallelism": "none (1 GPU)",
                   "decode_us_per_layer": round(us, 3)},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if extra:
        line["extra"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
