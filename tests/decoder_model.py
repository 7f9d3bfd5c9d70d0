"""Synthetic Qwen3 text decoders for the end-to-end greedy check.

Three implementations of the same layer sequence (src/cpu_decoder.rs:367-532:
input RMSNorm, q/k/v projections, q/k RMSNorm + RoPE, KV append, causal GQA
attention, o_proj + residual, post-attention RMSNorm, SiLU(gate) * up, down +
residual; final RMSNorm, logits against the tied embedding, greedy argmax),
with f16 rounding at the reference's points:

  * the CPU oracle's TextDecoder (oracle/oracle.cpp, f32, the reference order);
  * `NumpyDecoder` below, float64 between the rounding points -- an
    independent restatement that pins the oracle on small shapes;
  * `GpuDecoder` below: torch on the GPU for everything outside the attention
    path (test plumbing: f32 matmuls, f16 storage) and this library's C ABI
    (qasr_prefill_layer / qasr_decode_step) for the attention path under test.

Weights are random (no checkpoint is available offline), seeded, shaped like
the Qwen3-ASR decoders: projections N(0, 1/fan_in) with o_proj and down_proj
scaled by 3, norm gains N(1, 0.1), embedding N(0, 0.1).  With a tied embedding
an unscaled random model only ever repeats its last token (the residual path
carries the token's own embedding to the logits); these scales make the
layers dominate and the greedy stream vary.
"""
from __future__ import annotations

import numpy as np

from oracle import LAYER_TENSORS

CFG_0P6B = dict(hs=1024, nqh=16, nkvh=8, hd=128, inter=3072, layers=28, vocab=151936,
                max_seq=16384, eps=1e-6)
CFG_1P7B = dict(CFG_0P6B, hs=2048, inter=6144)


def synth_weights(cfg: dict, seed: int, device: str = "cpu", embed_std: float = 0.1,
                  out_scale: float = 3.0):
    """Seeded f16 weights as torch tensors on `device` (layer tensors keyed by
    (layer, name) with the names of oracle.LAYER_TENSORS)."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    hs, hd, inter = cfg["hs"], cfg["hd"], cfg["inter"]
    qd, kd = cfg["nqh"] * hd, cfg["nkvh"] * hd

    def normal(shape, std, mean=0.0):
        return (torch.randn(shape, generator=g, device=device) * std + mean).half()

    W = {"embed": normal((cfg["vocab"], hs), embed_std), "norm": normal((hs,), 0.1, 1.0)}
    for l in range(cfg["layers"]):
        W[(l, "input_layernorm")] = normal((hs,), 0.1, 1.0)
        W[(l, "post_attention_layernorm")] = normal((hs,), 0.1, 1.0)
        W[(l, "q_norm")] = normal((hd,), 0.1, 1.0)
        W[(l, "k_norm")] = normal((hd,), 0.1, 1.0)
        W[(l, "q_proj")] = normal((qd, hs), hs ** -0.5)
        W[(l, "k_proj")] = normal((kd, hs), hs ** -0.5)
        W[(l, "v_proj")] = normal((kd, hs), hs ** -0.5)
        W[(l, "o_proj")] = normal((hs, qd), out_scale * qd ** -0.5)
        W[(l, "gate_proj")] = normal((inter, hs), hs ** -0.5)
        W[(l, "up_proj")] = normal((inter, hs), hs ** -0.5)
        W[(l, "down_proj")] = normal((hs, inter), out_scale * inter ** -0.5)
    return W


def host_bits(W):
    """torch f16 tensors -> uint16 numpy arrays (what the oracle consumes)."""
    return {k: v.detach().cpu().contiguous().numpy().view(np.uint16) for k, v in W.items()}


def rope_tables_f16(rows: int, hd: int, theta: float = 1e6):
    """1-D rotate-half RoPE tables rounded to f16 (text positions make MRoPE
    1-D; any head size)."""
    half = hd // 2
    inv = theta ** (-2.0 * np.arange(half) / hd)
    ang = np.arange(rows, dtype=np.float64)[:, None] * inv[None, :]
    cos = np.concatenate([np.cos(ang), np.cos(ang)], 1).astype(np.float32).astype(np.float16)
    sin = np.concatenate([np.sin(ang), np.sin(ang)], 1).astype(np.float32).astype(np.float16)
    return cos.view(np.uint16), sin.view(np.uint16)


def _f16(x):
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


class NumpyDecoder:
    """float64 restatement of the decoder with the reference's f16 rounding
    points; `skip` names a step to leave out (planted-mistake tests)."""

    def __init__(self, cfg, Wbits, cap, cos_u16, sin_u16, skip=None):
        self.c = cfg
        self.W = {k: v.view(np.float16).astype(np.float64) for k, v in Wbits.items()}
        self.cos = cos_u16.view(np.float16).astype(np.float64)
        self.sin = sin_u16.view(np.float16).astype(np.float64)
        L, nkvh, hd = cfg["layers"], cfg["nkvh"], cfg["hd"]
        self.k = np.zeros((L, nkvh, cap, hd))
        self.v = np.zeros((L, nkvh, cap, hd))
        self.pos = 0
        self.last = 0
        self.skip = skip

    def _rms(self, x, w):
        inv = 1.0 / np.sqrt((x * x).sum(-1, keepdims=True) / x.shape[-1] + self.c["eps"])
        return _f16(x * inv * w)

    def _norm_rope(self, raw, g, pos):
        hd = self.c["hd"]
        h = hd // 2
        inv = 1.0 / np.sqrt((raw * raw).sum() / hd + self.c["eps"])
        y = raw * inv * g
        rot = np.concatenate([-y[h:], y[:h]])
        return _f16(y * self.cos[pos] + rot * self.sin[pos])

    def _forward(self, x, q0):
        c, W = self.c, self.W
        nqh, nkvh, hd = c["nqh"], c["nkvh"], c["hd"]
        rep = nqh // nkvh
        rows = x.shape[0]
        for l in range(c["layers"]):
            n = self._rms(x, W[(l, "input_layernorm")])
            q = _f16(n @ W[(l, "q_proj")].T).reshape(rows, nqh, hd)
            k = _f16(n @ W[(l, "k_proj")].T).reshape(rows, nkvh, hd)
            v = _f16(n @ W[(l, "v_proj")].T).reshape(rows, nkvh, hd)
            for r in range(rows):
                p = q0 + r
                for hh in range(nqh):
                    q[r, hh] = self._norm_rope(q[r, hh], W[(l, "q_norm")], p)
                for hh in range(nkvh):
                    self.k[l, hh, p] = self._norm_rope(k[r, hh], W[(l, "k_norm")], p)
                    self.v[l, hh, p] = v[r, hh]
            attn = np.zeros((rows, nqh * hd))
            for r in range(rows):
                valid = q0 + r + 1
                for hh in range(nqh):
                    kk, vv = self.k[l, hh // rep, :valid], self.v[l, hh // rep, :valid]
                    s = kk @ q[r, hh] / np.sqrt(hd)
                    e = np.exp(s - s.max())
                    attn[r, hh * hd:(hh + 1) * hd] = (e / e.sum()) @ vv
            attn = _f16(attn)
            if self.skip != "attn_residual":
                x = _f16(x + attn @ W[(l, "o_proj")].T)
            n2 = self._rms(x, W[(l, "post_attention_layernorm")])
            g = _f16(n2 @ W[(l, "gate_proj")].T)
            u = _f16(n2 @ W[(l, "up_proj")].T)
            hmid = _f16(g / (1.0 + np.exp(-g)) * u)
            x = _f16(x + hmid @ W[(l, "down_proj")].T)
        return x

    def _logits(self, xl):
        n = self._rms(xl, self.W["norm"])
        lg = self.W["embed"] @ n
        return int(np.argmax(lg)), lg

    def prefill(self, hidden_u16, kv_start):
        x = hidden_u16.view(np.float16).astype(np.float64)
        x = self._forward(x, kv_start)
        self.pos = kv_start + x.shape[0]
        tok, lg = self._logits(x[-1])
        self.last = tok
        return tok, lg

    def step(self):
        x = self.W["embed"][self.last][None, :]
        x = self._forward(x, self.pos)
        self.pos += 1
        tok, lg = self._logits(x[0])
        self.last = tok
        return tok, lg


class GpuDecoder:
    """The decoder on the GPU: this library's attention path (stage (a) + (b)
    or (c) through qasr_decode_step / qasr_prefill_layer) inside a torch layer
    sequence.  One KV pool slot per sequence; `step` runs any subset of slots
    as one batch (the reference's --batch N)."""

    def __init__(self, cfg, W, slots: int, cap: int):
        import torch

        import qasr_attn

        torch.backends.cuda.matmul.allow_tf32 = False
        torch.set_float32_matmul_precision("highest")
        self.t, self.q, self.c = torch, qasr_attn, cfg
        self.ctx = qasr_attn.Context(cfg["nqh"], cfg["nkvh"], cfg["hd"], cfg["layers"], cfg["eps"],
                                     cfg["max_seq"], 0)
        cs, sn = qasr_attn.mrope_text_tables(cfg["max_seq"], cfg["hd"])
        self.ctx.set_rope_tables(cs, sn)
        self.kv = qasr_attn.KVPool(self.ctx, slots, cap)
        f = lambda k: W[k].float().contiguous()
        self.L = []
        for l in range(cfg["layers"]):
            self.L.append(dict(
                iln=f((l, "input_layernorm")), pln=f((l, "post_attention_layernorm")),
                qn=W[(l, "q_norm")].contiguous(), kn=W[(l, "k_norm")].contiguous(),
                qkv=torch.cat([W[(l, "q_proj")], W[(l, "k_proj")], W[(l, "v_proj")]]).float(),
                o=f((l, "o_proj")), gate=f((l, "gate_proj")), up=f((l, "up_proj")),
                down=f((l, "down_proj"))))
        self.embed16 = W["embed"].contiguous()
        self.embed32 = W["embed"].float()
        self.norm = f("norm")
        self.qdim = cfg["nqh"] * cfg["hd"]

    def _rms(self, x16, w):
        x = x16.float()
        inv = 1.0 / self.t.sqrt((x * x).sum(-1, keepdim=True) / x.shape[-1] + self.c["eps"])
        return ((x * inv) * w).half()

    def _layers(self, x, attn_fn):
        for l, P in enumerate(self.L):
            n = self._rms(x, P["iln"])
            qkv = (n.float() @ P["qkv"].T).half().contiguous()
            a = attn_fn(l, qkv, P)
            x = (x.float() + a.float() @ P["o"].T).half()
            n2 = self._rms(x, P["pln"]).float()
            g = (n2 @ P["gate"].T).half().float()
            u = (n2 @ P["up"].T).half().float()
            h = (g / (1.0 + self.t.exp(-g)) * u).half()
            x = (x.float() + h.float() @ P["down"].T).half()
        return x

    def _logits(self, x16):
        n = self._rms(x16, self.norm)
        return n.float() @ self.embed32.T

    def prefill(self, slot: int, hidden16, kv_start: int):
        t = self.t
        s = hidden16.shape[0]
        out = t.empty((s, self.qdim), device="cuda", dtype=t.float16)
        qw = t.empty((s, self.qdim), device="cuda", dtype=t.float16)

        def attn(l, qkv, P):
            self.q.prefill_layer(self.ctx, self.kv, l, slot, kv_start, s, qkv, P["qn"], P["kn"],
                                 qw, out)
            return out

        x = self._layers(hidden16.contiguous(), attn)
        lg = self._logits(x[-1:])[0]
        return int(t.argmax(lg).item()), lg.cpu().numpy()

    def step(self, slots, pos, tokens):
        t = self.t
        x = self.embed16[t.tensor(tokens, device="cuda", dtype=t.long)].contiguous()
        out = t.empty((len(slots), self.qdim), device="cuda", dtype=t.float16)

        def attn(l, qkv, P):
            self.q.decode_step(self.ctx, self.kv, l, pos, qkv, P["qn"], P["kn"], out, slots=slots)
            return out

        x = self._layers(x, attn)
        lg = self._logits(x)
        toks = t.argmax(lg, dim=-1).tolist()
        return toks, lg.cpu().numpy()

    def close(self):
        self.kv.close()
        self.ctx.close()


def compare_teacher_forced(cpu, gpu, label: str, rel_logit_tol: float = 0.02):
    """cpu, gpu: lists of (token, logits), step by step, where every step of
    both sides was fed the CPU reference's previous token (teacher forcing),
    so one step's argmax cannot change what the later steps see.  At every
    step the logits must agree to `rel_logit_tol` of their spread, and the
    argmax must agree except where the CPU's top-2 margin is below twice the
    measured logit difference of that step: such a near-tie is counted, any
    other disagreement fails (the reference's own batch check bails on any
    difference, src/bin/batch_step_bench.rs:141-168).  Returns the number of
    near-tie disagreements; the figures go to the parity report."""
    assert len(cpu) == len(gpu), f"{label}: {len(cpu)} CPU steps against {len(gpu)} GPU steps"
    worst_diff, min_gap, near = 0.0, float("inf"), 0
    for i, ((tc, lc), (tg, lg)) in enumerate(zip(cpu, gpu)):
        d = float(np.max(np.abs(lc - lg)))
        spread = float(np.std(lc))
        top = np.partition(lc, -2)[-2:]
        gap = float(top[1] - top[0])
        worst_diff, min_gap = max(worst_diff, d), min(min_gap, gap)
        assert d <= rel_logit_tol * spread, f"{label} step {i}: logit diff {d} vs spread {spread}"
        if tc != tg:
            assert gap < 2.0 * d, (f"{label} step {i}: argmax differs at a clear margin: cpu {tc} "
                                   f"gpu {tg} (CPU top-2 gap {gap:.4g}, logit diff {d:.4g})")
            near += 1
    print(f"{label}: {len(cpu)} steps, {near} near-tie disagreements; min top-2 gap "
          f"{min_gap:.4g}, max logit diff {worst_diff:.4g}", flush=True)
    from workloads import REPORT
    REPORT.append({"label": f"teacher-forced {label}", "steps": len(cpu), "near_tie_flips": near,
                   "min_top2_gap": min_gap, "max_logit_diff": worst_diff})
    return near
