"""Helpers for the gpu-marked tests: host <-> device copies of f16 bit
patterns, a context + KV pool set up like the reference decoder at load time,
and readback of cache rows.  Every compute call goes through the C ABI."""
from __future__ import annotations

import sys

import numpy as np

import qasr_attn
from workloads import HD, MAX_SEQ, NKVH, NQH, QDIM


def say(msg: str):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def dev(u16: np.ndarray):
    import torch

    a = np.ascontiguousarray(u16, dtype=np.uint16)
    return torch.from_numpy(a.view(np.float16)).cuda()


def host(t) -> np.ndarray:
    import torch

    torch.cuda.synchronize()
    return t.detach().cpu().contiguous().numpy().view(np.uint16)


def empty(rows: int, cols: int):
    import torch

    return torch.empty((rows, cols), dtype=torch.float16, device="cuda")


_TABLES = None


def rope_tables():
    global _TABLES
    if _TABLES is None:
        _TABLES = qasr_attn.mrope_text_tables(MAX_SEQ)
    return _TABLES


class Gpu:
    """Context (layers) + KV pool (slots x cap) with the RoPE tables loaded."""

    def __init__(self, slots: int, cap: int, layers: int = 1, max_seq: int = MAX_SEQ):
        self.ctx = qasr_attn.Context(NQH, NKVH, HD, layers, 1e-6, max_seq, 0)
        c, s = rope_tables()
        self.ctx.set_rope_tables(c, s)
        self.kv = qasr_attn.KVPool(self.ctx, slots, cap)

    def gains(self, lay):
        return dev(lay.q_gain), dev(lay.k_gain)

    def append(self, layer: int, lay, segments, qkv_u16: np.ndarray) -> np.ndarray:
        """Stage (a) over segments [(slot, pos0, rows)]; returns roped q rows."""
        rows = qkv_u16.shape[0]
        q_out = empty(rows, QDIM)
        qg, kg = self.gains(lay)
        qasr_attn.qk_norm_rope_append(self.ctx, self.kv, layer, segments, dev(qkv_u16), qg, kg, q_out)
        return host(q_out)

    def cache(self, slot: int, layer: int, rows: int):
        """(K, V) rows 0..rows-1 of (slot, layer) as u16 [nkvh][rows][hd]."""
        t = self.kv.tensor()
        return host(t[slot, layer, 0, :, :rows].contiguous()), host(t[slot, layer, 1, :, :rows].contiguous())

    def cache_row(self, slot: int, layer: int, pos: int):
        """(K, V) row `pos` of (slot, layer) as u16 [nkvh][hd]."""
        t = self.kv.tensor()
        return host(t[slot, layer, 0, :, pos].contiguous()), host(t[slot, layer, 1, :, pos].contiguous())

    def close(self):
        self.kv.close()
        self.ctx.close()
