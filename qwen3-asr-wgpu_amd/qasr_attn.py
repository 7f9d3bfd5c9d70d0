"""Python binding of libqasr_attn.so (ctypes) and a host-side mirror of the
reference decoder's backend contract for the attention path.

The reference's seam is `TextBackend` (src/inference.rs:213-269):
`prefill(hidden, s, kv_start)`, `step()`, `max_seq()`, `ensure_capacity(need)`,
`set_rope_tables(cos, sin)`.  `AttnBackend` below keeps those names and their
argument meaning for the attention part of one decoder layer, on a pooled
per-slot KV cache (`--batch N` slots, src/decoder.rs:2453-2457, 2856-2883).
Errors raise `QasrError` carrying the library's status code, as the reference
returns `Err` from the same bounds checks (src/cpu_decoder.rs:489-495, 520).

Device tensors are torch tensors (torch supplies device memory and streams;
every computation runs in the HIP library).  Calls are enqueued on torch's
current stream.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqasr_attn.so")

QASR_OK, QASR_EINVAL, QASR_ERANGE, QASR_ENOMEM, QASR_EDEVICE, QASR_ESTATE = range(6)
KV_INITIAL_CAP = 1024
KV_STEP = 256
DECODER_MAX_SEQ = 16384

# Every symbol include/qasr_attn.h declares.
ABI_SYMBOLS = (
    "qasr_abi_version", "qasr_last_error", "qasr_ctx_create", "qasr_ctx_destroy",
    "qasr_mrope_text_tables", "qasr_set_rope_tables", "qasr_kv_create", "qasr_kv_destroy",
    "qasr_kv_get_info", "qasr_kv_ensure_capacity", "qasr_qk_norm_rope_append",
    "qasr_decode_attn", "qasr_decode_step", "qasr_prefill_attn", "qasr_prefill_layer",
    "qasr_decoder_create", "qasr_decoder_destroy", "qasr_decoder_step", "qasr_decoder_prefill",
    "qasr_decoder_prefill_batch", "qasr_dequant_i8", "qasr_prefill_attn_batch",
    "qasr_softmax_weights", "qasr_stream_read", "qasr_prefill_attn_noalloc", "qasr_gemm_f16",
    "qasr_mfma_probe", "qasr_plan_decode", "qasr_plan_prefill",
)
MAX_PREFILL_SEGMENTS = 64  # segments per qasr_decoder_prefill_batch call


class QasrError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[qasr status {code}] {message}")
        self.code = code


class AttnCfg(ctypes.Structure):
    _fields_ = [
        ("num_attention_heads", ctypes.c_int32),
        ("num_key_value_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("num_hidden_layers", ctypes.c_int32),
        ("rms_norm_eps", ctypes.c_float),
        ("max_seq", ctypes.c_int32),
    ]


class Segment(ctypes.Structure):
    _fields_ = [("slot", ctypes.c_int32), ("pos0", ctypes.c_int32), ("rows", ctypes.c_int32)]


class KvInfo(ctypes.Structure):
    _fields_ = [
        ("base_dev", ctypes.c_void_p),
        ("slots", ctypes.c_int32),
        ("layers", ctypes.c_int32),
        ("nkvh", ctypes.c_int32),
        ("cap", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("slot_stride", ctypes.c_int64),
        ("layer_stride", ctypes.c_int64),
        ("kv_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64),
        ("bytes", ctypes.c_size_t),
    ]


class LayerWeights(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in (
        "input_norm", "qkv_proj", "q_norm", "k_norm", "o_proj", "post_norm", "gate_up_proj",
        "down_proj", "qkv_scale", "o_scale", "gate_up_scale", "down_scale")]


class DecoderCfg(ctypes.Structure):
    _fields_ = [
        ("hidden_size", ctypes.c_int32),
        ("intermediate_size", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32),
        ("max_rows", ctypes.c_int32),
    ]


_lib = None
_vp = ctypes.c_void_p
_i32p = ctypes.POINTER(ctypes.c_int32)
_u16p = ctypes.POINTER(ctypes.c_uint16)


def load(path: str = LIB_PATH):
    """Load the HIP library; raises if it has not been built (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python qwen3-asr-wgpu_amd/build.py` "
            "(there is no CPU fallback for the attention path)")
    L = ctypes.CDLL(path)
    L.qasr_abi_version.restype = ctypes.c_int
    L.qasr_last_error.restype = ctypes.c_char_p
    L.qasr_ctx_create.argtypes = [ctypes.POINTER(AttnCfg), ctypes.c_int, ctypes.POINTER(_vp)]
    L.qasr_ctx_destroy.argtypes = [_vp]
    L.qasr_ctx_destroy.restype = None
    L.qasr_mrope_text_tables.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_double, _i32p,
                                         ctypes.c_int, ctypes.c_int, _u16p, _u16p]
    L.qasr_set_rope_tables.argtypes = [_vp, _u16p, _u16p, ctypes.c_int]
    L.qasr_kv_create.argtypes = [_vp, ctypes.c_int, ctypes.c_int, ctypes.POINTER(_vp)]
    L.qasr_kv_destroy.argtypes = [_vp]
    L.qasr_kv_destroy.restype = None
    L.qasr_kv_get_info.argtypes = [_vp, ctypes.POINTER(KvInfo)]
    L.qasr_kv_ensure_capacity.argtypes = [_vp, ctypes.c_int, ctypes.c_int, _i32p]
    L.qasr_qk_norm_rope_append.argtypes = [_vp, _vp, ctypes.c_int, ctypes.POINTER(Segment),
                                           ctypes.c_int, _vp, _vp, _vp, _vp, _vp]
    L.qasr_decode_attn.argtypes = [_vp, _vp, ctypes.c_int, ctypes.c_int, _i32p, _i32p, _vp, _vp,
                                   _vp]
    L.qasr_decode_step.argtypes = [_vp, _vp, ctypes.c_int, ctypes.c_int, _i32p, _i32p, _vp, _vp,
                                   _vp, _vp, _vp]
    L.qasr_prefill_attn.argtypes = [_vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, _vp, _vp, _vp]
    L.qasr_prefill_attn_noalloc.argtypes = [_vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, _vp, _vp, _vp]
    L.qasr_prefill_layer.argtypes = [_vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _vp]
    L.qasr_prefill_attn_batch.argtypes = [_vp, _vp, ctypes.c_int, ctypes.POINTER(Segment),
                                          ctypes.c_int, _vp, _vp, _vp]
    L.qasr_decoder_create.argtypes = [_vp, ctypes.POINTER(DecoderCfg), _vp, _vp,
                                      ctypes.POINTER(LayerWeights), ctypes.POINTER(_vp)]
    L.qasr_decoder_destroy.argtypes = [_vp]
    L.qasr_decoder_destroy.restype = None
    L.qasr_decoder_step.argtypes = [_vp, _vp, ctypes.c_int, _i32p, _i32p, _vp, _vp, _vp, _vp]
    L.qasr_decoder_prefill.argtypes = [_vp, _vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp,
                                       _vp, _vp, _vp]
    L.qasr_decoder_prefill_batch.argtypes = [_vp, _vp, ctypes.POINTER(Segment), ctypes.c_int, _vp,
                                             _vp, _vp, _vp]
    L.qasr_dequant_i8.argtypes = [_vp, _vp, _vp, ctypes.c_int64, ctypes.c_int32, _vp, _vp]
    L.qasr_gemm_f16.argtypes = [_vp, _vp, _vp, _vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                ctypes.c_int, _vp]
    L.qasr_softmax_weights.argtypes = [_vp, _vp, _vp, ctypes.c_int64, _vp, _vp, _vp]
    L.qasr_stream_read.argtypes = [_vp, _vp, ctypes.c_int64, ctypes.c_int, ctypes.c_int, _vp, _vp]
    L.qasr_mfma_probe.argtypes = [_vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, _vp, _vp, _vp]
    i32p = ctypes.POINTER(ctypes.c_int32)
    L.qasr_plan_decode.argtypes = [ctypes.c_int, i32p, ctypes.c_int, ctypes.c_int, i32p, i32p, i32p]
    L.qasr_plan_prefill.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, i32p, i32p, i32p, i32p]
    _lib = L
    return L


def _check(rc: int):
    if rc != QASR_OK:
        msg = load().qasr_last_error()
        raise QasrError(rc, msg.decode() if msg else "")


def _i32(seq) -> ctypes.Array:
    a = (ctypes.c_int32 * len(seq))()
    for i, v in enumerate(seq):
        a[i] = int(v)
    return a


def mrope_text_tables(rows: int, head_dim: int = 128, rope_theta: float = 1e6,
                      section: Sequence[int] = (24, 20, 20), interleaved: bool = True):
    """f16 cos/sin tables ([rows][head_dim] uint16 bit patterns) for text
    positions, as src/inference.rs:1038-1049 builds them."""
    c = np.empty((rows, head_dim), dtype=np.uint16)
    s = np.empty((rows, head_dim), dtype=np.uint16)
    sec = _i32(section)
    _check(load().qasr_mrope_text_tables(rows, head_dim, rope_theta, sec, len(section),
                                         int(interleaved), c.ctypes.data_as(_u16p),
                                         s.ctypes.data_as(_u16p)))
    return c, s


def _stream(stream) -> Optional[int]:
    if stream is not None:
        return int(stream)
    import torch

    return int(torch.cuda.current_stream().cuda_stream)


def _dev(t, name: str, dtype=None) -> int:
    """Device pointer of a contiguous CUDA tensor (f16 unless `dtype`)."""
    import torch

    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must live on the GPU")
    want = dtype or torch.float16
    if t.dtype != want:
        raise ValueError(f"{name} must be {want}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


def _need(t, elems: int, name: str, exact: bool = False):
    """The C ABI receives raw device pointers: a tensor smaller than the rows
    the call implies would be read or written out of bounds, so it is refused
    here, before any launch, with the library's EINVAL."""
    n = int(t.numel())
    if n < elems or (exact and n != elems):
        raise QasrError(QASR_EINVAL, f"{name} holds {n} elements, the call needs "
                                     f"{'exactly ' if exact else ''}{elems}")


def _rows_of(segments) -> int:
    return sum(int(r) for _, _, r in segments)


class Context:
    """Device + shape binding (qasr_ctx)."""

    def __init__(self, nqh: int = 16, nkvh: int = 8, head_dim: int = 128, layers: int = 28,
                 eps: float = 1e-6, max_seq: int = DECODER_MAX_SEQ, device: int = 0):
        self.cfg = AttnCfg(nqh, nkvh, head_dim, layers, eps, max_seq)
        self.device = device
        h = _vp()
        _check(load().qasr_ctx_create(ctypes.byref(self.cfg), device, ctypes.byref(h)))
        self.handle = h

    @property
    def nqh(self):
        return self.cfg.num_attention_heads

    @property
    def nkvh(self):
        return self.cfg.num_key_value_heads

    @property
    def layers(self):
        return self.cfg.num_hidden_layers

    def set_rope_tables(self, cos_u16: np.ndarray, sin_u16: np.ndarray):
        cos_u16 = np.ascontiguousarray(cos_u16, dtype=np.uint16)
        sin_u16 = np.ascontiguousarray(sin_u16, dtype=np.uint16)
        if cos_u16.shape != sin_u16.shape or cos_u16.ndim != 2:
            raise ValueError("cos/sin must be equal [rows][head_dim] arrays")
        _check(load().qasr_set_rope_tables(self.handle, cos_u16.ctypes.data_as(_u16p),
                                           sin_u16.ctypes.data_as(_u16p), cos_u16.shape[0]))

    def close(self):
        if self.handle:
            load().qasr_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KVPool:
    """Pooled per-slot KV cache (qasr_kv): [slot][layer][K|V][kvh][cap][hd] f16."""

    def __init__(self, ctx: Context, slots: int, cap: int = KV_INITIAL_CAP):
        self.ctx = ctx
        h = _vp()
        _check(load().qasr_kv_create(ctx.handle, slots, cap, ctypes.byref(h)))
        self.handle = h

    def info(self) -> KvInfo:
        inf = KvInfo()
        _check(load().qasr_kv_get_info(self.handle, ctypes.byref(inf)))
        return inf

    @property
    def cap(self) -> int:
        return self.info().cap

    @property
    def slots(self) -> int:
        return self.info().slots

    def ensure_capacity(self, need: int, keep_rows: int) -> int:
        out = ctypes.c_int32(0)
        _check(load().qasr_kv_ensure_capacity(self.handle, need, keep_rows, ctypes.byref(out)))
        return out.value

    def tensor(self):
        """A torch view of the whole pool, shaped [slot][layer][2][kvh][cap][hd]."""
        import torch

        inf = self.info()
        n = inf.bytes // 2
        storage = _DeviceView(inf.base_dev, inf.bytes, self.ctx.device)
        t = torch.as_tensor(storage, device=f"cuda:{self.ctx.device}")
        assert t.numel() == n
        return t.view(inf.slots, inf.layers, 2, inf.nkvh, inf.cap, inf.head_dim)

    def close(self):
        if self.handle:
            load().qasr_kv_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _DeviceView:
    """__cuda_array_interface__ over library-owned device memory (f16)."""

    def __init__(self, ptr: int, nbytes: int, device: int):
        self.__cuda_array_interface__ = {
            "shape": (nbytes // 2,),
            "typestr": "<f2",
            "data": (int(ptr), False),
            "version": 3,
            "strides": None,
            "stream": None,
        }


# ---- stage entry points (thin wrappers over the C ABI) --------------------

def _widths(ctx: Context):
    """(fused qkv row, q/out row) widths in elements for this context."""
    hd = ctx.cfg.head_dim
    return (ctx.nqh + 2 * ctx.nkvh) * hd, ctx.nqh * hd


def _gains(ctx: Context, q_gain, k_gain):
    _need(q_gain, ctx.cfg.head_dim, "q_gain", exact=True)
    _need(k_gain, ctx.cfg.head_dim, "k_gain", exact=True)


def qk_norm_rope_append(ctx: Context, kv: KVPool, layer: int, segments, qkv, q_gain, k_gain,
                        q_out, stream=None):
    tot, qd = _widths(ctx)
    rows = _rows_of(segments)
    _need(qkv, rows * tot, "qkv")
    _need(q_out, rows * qd, "q_out")
    _gains(ctx, q_gain, k_gain)
    segs = (Segment * len(segments))(*[Segment(int(s), int(p), int(r)) for s, p, r in segments])
    _check(load().qasr_qk_norm_rope_append(
        ctx.handle, kv.handle, layer, segs, len(segments), _dev(qkv, "qkv"),
        _dev(q_gain, "q_gain"), _dev(k_gain, "k_gain"), _dev(q_out, "q_out"), _stream(stream)))


def decode_attn(ctx: Context, kv: KVPool, layer: int, cur_len, q, out, slots=None, stream=None):
    b = len(cur_len)
    _, qd = _widths(ctx)
    _need(q, b * qd, "q")
    _need(out, b * qd, "out")
    if slots is not None and len(slots) != b:
        raise QasrError(QASR_EINVAL, f"{len(slots)} slots for {b} entries")
    _check(load().qasr_decode_attn(ctx.handle, kv.handle, layer, b,
                                   _i32(slots) if slots is not None else None, _i32(cur_len),
                                   _dev(q, "q"), _dev(out, "out"), _stream(stream)))


def decode_step(ctx: Context, kv: KVPool, layer: int, pos, qkv, q_gain, k_gain, out, slots=None,
                stream=None):
    b = len(pos)
    tot, qd = _widths(ctx)
    _need(qkv, b * tot, "qkv")
    _need(out, b * qd, "out")
    _gains(ctx, q_gain, k_gain)
    if slots is not None and len(slots) != b:
        raise QasrError(QASR_EINVAL, f"{len(slots)} slots for {b} entries")
    _check(load().qasr_decode_step(ctx.handle, kv.handle, layer, b,
                                   _i32(slots) if slots is not None else None, _i32(pos),
                                   _dev(qkv, "qkv"), _dev(q_gain, "q_gain"),
                                   _dev(k_gain, "k_gain"), _dev(out, "out"), _stream(stream)))


def prefill_attn(ctx: Context, kv: KVPool, layer: int, slot: int, kv_start: int, s: int, q, out,
                 stream=None):
    _, qd = _widths(ctx)
    _need(q, max(s, 0) * qd, "q")
    _need(out, max(s, 0) * qd, "out")
    _check(load().qasr_prefill_attn(ctx.handle, kv.handle, layer, slot, kv_start, s,
                                    _dev(q, "q"), _dev(out, "out"), _stream(stream)))


def prefill_attn_noalloc(ctx: Context, kv: KVPool, layer: int, slot: int, kv_start: int, s: int,
                         q, out, stream=None):
    """qasr_prefill_attn_noalloc: prefill_attn without any allocation (split
    partials in the library's static per-GPU scratch; at most 2048 rows per
    call with 8 kv heads; calls overlapping on one GPU race)."""
    _, qd = _widths(ctx)
    _need(q, max(s, 0) * qd, "q")
    _need(out, max(s, 0) * qd, "out")
    _check(load().qasr_prefill_attn_noalloc(ctx.handle, kv.handle, layer, slot, kv_start, s,
                                            _dev(q, "q"), _dev(out, "out"), _stream(stream)))


def prefill_attn_batch(ctx: Context, kv: KVPool, layer: int, segments, q, out, stream=None):
    """Stage (c) for segments [(slot, kv_start, rows)] whose q rows (and
    output rows) are concatenated in order; one launch where the key ranges
    are short."""
    _, qd = _widths(ctx)
    rows = _rows_of(segments)
    _need(q, rows * qd, "q")
    _need(out, rows * qd, "out")
    segs = (Segment * len(segments))(*[Segment(int(s), int(p), int(r)) for s, p, r in segments])
    _check(load().qasr_prefill_attn_batch(ctx.handle, kv.handle, layer, segs, len(segments),
                                          _dev(q, "q"), _dev(out, "out"), _stream(stream)))


def prefill_layer(ctx: Context, kv: KVPool, layer: int, slot: int, kv_start: int, s: int, qkv,
                  q_gain, k_gain, q_work, out, stream=None):
    tot, qd = _widths(ctx)
    _need(qkv, max(s, 0) * tot, "qkv")
    _need(q_work, max(s, 0) * qd, "q_work")
    _need(out, max(s, 0) * qd, "out")
    _gains(ctx, q_gain, k_gain)
    _check(load().qasr_prefill_layer(ctx.handle, kv.handle, layer, slot, kv_start, s,
                                     _dev(qkv, "qkv"), _dev(q_gain, "q_gain"),
                                     _dev(k_gain, "k_gain"), _dev(q_work, "q_work"),
                                     _dev(out, "out"), _stream(stream)))


class AttnBackend:
    """The attention half of the reference's TextBackend (src/inference.rs:
    213-269) on one GPU: the same method names, over a pooled KV cache of
    `slots` sequences (`--batch N`).  `prefill` and `step` take the fused qkv
    projection rows ([rows][(nqh+2*nkvh)*hd] f16) where the reference takes
    hidden states, since the projections sit outside this path; they return
    the attention output rows ([rows][nqh*hd] f16) that feed o_proj.
    """

    def __init__(self, nqh=16, nkvh=8, head_dim=128, layers=28, eps=1e-6,
                 max_seq=DECODER_MAX_SEQ, slots=1, device=0, cap=KV_INITIAL_CAP):
        self.ctx = Context(nqh, nkvh, head_dim, layers, eps, max_seq, device)
        self.kv = KVPool(self.ctx, slots, min(cap, max_seq))
        self.max_seq = max_seq
        self.pos = [0] * slots  # positions already in each slot's cache

    def set_rope_tables(self, cos_u16, sin_u16):
        self.ctx.set_rope_tables(cos_u16, sin_u16)

    def ensure_capacity(self, need: int) -> int:
        """Grow-only, KV_STEP granular; keeps every row already written."""
        return self.kv.ensure_capacity(need, max(self.pos))

    def prefill(self, layer: int, qkv, s: int, kv_start: int, q_gain, k_gain, slot: int = 0,
                last_layer: bool = True):
        import torch

        nq = self.ctx.nqh * 128
        q_work = torch.empty((s, nq), dtype=torch.float16, device=qkv.device)
        out = torch.empty((s, nq), dtype=torch.float16, device=qkv.device)
        prefill_layer(self.ctx, self.kv, layer, slot, kv_start, s, qkv, q_gain, k_gain, q_work,
                      out)
        if last_layer:
            self.pos[slot] = kv_start + s
        return out

    def step(self, layer: int, qkv_rows, q_gain, k_gain, slots: Optional[Sequence[int]] = None,
             last_layer: bool = True):
        import torch

        slots = list(range(qkv_rows.shape[0])) if slots is None else list(slots)
        pos = [self.pos[s] for s in slots]
        out = torch.empty((len(slots), self.ctx.nqh * 128), dtype=torch.float16,
                          device=qkv_rows.device)
        decode_step(self.ctx, self.kv, layer, pos, qkv_rows, q_gain, k_gain, out, slots=slots)
        if last_layer:
            for s in slots:
                self.pos[s] += 1
        return out


def dequant_i8(ctx: Context, q, scale, out=None):
    """f16 copy of an int8 [rows][cols] matrix with f32 row scales (the
    reference's dequant_i8, weights.rs:366-385), on the GPU."""
    import torch

    if q.dim() != 2:
        raise QasrError(QASR_EINVAL, "q must be a [rows][cols] int8 matrix")
    rows, cols = int(q.shape[0]), int(q.shape[1])
    _need(scale, rows, "scale", exact=True)
    if out is None:
        out = torch.empty((rows, cols), dtype=torch.float16, device=q.device)
    _need(out, rows * cols, "out", exact=True)
    _check(load().qasr_dequant_i8(ctx.handle, _dev(q, "q", torch.int8),
                                  _dev(scale, "scale", torch.float32), rows, cols,
                                  _dev(out, "out"), _stream(None)))
    return out


def gemm_f16(ctx: Context, a, b, c=None, accumulate: bool = False):
    """c = f16(a . b^T (+ c)) for f16 CUDA matrices a [m][k], b [n][k]: the
    prefill projections' GEMM (f32 accumulation, one rounding).  Returns c."""
    import torch

    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[1]:
        raise QasrError(QASR_EINVAL, "a [m][k] and b [n][k] with the same k")
    m, k = int(a.shape[0]), int(a.shape[1])
    n = int(b.shape[0])
    if c is None:
        if accumulate:
            raise QasrError(QASR_EINVAL, "accumulate needs c")
        c = torch.empty((m, n), dtype=torch.float16, device=a.device)
    _need(c, m * n, "c", exact=True)
    _check(load().qasr_gemm_f16(ctx.handle, _dev(a, "a"), _dev(b, "b"), _dev(c, "c"), m, n, k,
                                1 if accumulate else 0, _stream(None)))
    return c


def softmax_weights(ctx: Context, s, m):
    """The attention kernels' softmax weights for scores s against maxima m
    (f32 CUDA tensors of one size): (decode form, prefill form), each
    2^(s*scale*log2(e) - m*scale*log2(e)) as that kernel rounds it."""
    import torch

    n = int(s.numel())
    _need(m, n, "m", exact=True)
    a = torch.empty_like(s)
    b = torch.empty_like(s)
    _check(load().qasr_softmax_weights(ctx.handle, _dev(s, "s", torch.float32),
                                       _dev(m, "m", torch.float32), n,
                                       _dev(a, "out_scaled", torch.float32),
                                       _dev(b, "out_raw", torch.float32), _stream(None)))
    return a, b


def stream_read(ctx: Context, src, wgs: int, waves: int, sink, stream=None):
    """Bare streaming read of a whole CUDA tensor (calibration, see
    qasr_stream_read); sink: int32 CUDA tensor of >= wgs * waves entries."""
    import torch

    if not src.is_cuda or not src.is_contiguous():
        raise ValueError("src must be a contiguous CUDA tensor")
    _need(sink, wgs * waves, "sink")
    _check(load().qasr_stream_read(ctx.handle, src.data_ptr(), src.numel() * src.element_size(),
                                   wgs, waves, _dev(sink, "sink", torch.int32), _stream(stream)))


def mfma_probe(ctx: Context, mode: int, wgs: int, waves: int, mfma_iters: int, valu_iters: int,
               sink, clk, stream=None):
    """Matrix-core calibration (see qasr_mfma_probe); sink: f32 CUDA tensor of
    >= wgs * waves entries (8 waves for mode 2), clk: int64 CUDA tensor of 4."""
    import torch

    _need(sink, wgs * (8 if mode % 4 == 2 else waves), "sink")
    _need(clk, 4, "clk")
    _check(load().qasr_mfma_probe(ctx.handle, mode, wgs, waves, mfma_iters, valu_iters,
                                  _dev(sink, "sink", torch.float32), _dev(clk, "clk", torch.int64),
                                  _stream(stream)))


def plan_decode(lens, nkvh: int = 8, cus: int = 256):
    """The decode plan the library launches for entries attending lens[b]
    keys (qasr_plan_decode; host only, no device): (keys per granule of each
    entry, granules per workgroup of each entry, workgroup bases [batch + 1])."""
    n = len(lens)
    arr = (ctypes.c_int32 * max(1, n))(*[int(x) for x in lens])
    gran = (ctypes.c_int32 * max(1, n))()
    run = (ctypes.c_int32 * max(1, n))()
    base = (ctypes.c_int32 * (n + 1))()
    _check(load().qasr_plan_decode(n, arr, nkvh, cus, gran, run, base))
    return list(gran[:n]), list(run[:n]), list(base)


def plan_prefill(rows: int, kv_start: int, nkvh: int = 8):
    """The prefill plan of one launch (qasr_plan_prefill; host only): rows
    per block, row blocks, tiles per split and each row block's first item."""
    rpb, nrb, tps = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    sp = (ctypes.c_int32 * 65)()
    _check(load().qasr_plan_prefill(rows, kv_start, nkvh, ctypes.byref(rpb), ctypes.byref(nrb),
                                    ctypes.byref(tps), sp))
    return {"rows_per_block": rpb.value, "nrb": nrb.value, "tiles_per_split": tps.value,
            "sp_base": list(sp[:nrb.value + 1])}


LAYER_WEIGHT_NAMES = ("input_layernorm", "q_proj", "k_proj", "v_proj", "q_norm", "k_norm",
                      "o_proj", "post_attention_layernorm", "gate_proj", "up_proj", "down_proj")


class TextDecoder:
    """The whole text decoder on one GPU (qasr_decoder_*), with the reference
    backend's contract (TextBackend, src/inference.rs:213-269; CpuTextDecoder
    ::prefill / ::step, src/cpu_decoder.rs:486-530): `prefill(hidden, kv_start)`
    returns the greedy token after a prompt, `step()` embeds each slot's last
    token, runs one position and returns the next tokens; `max_seq`,
    `ensure_capacity`, `set_rope_tables` as in the reference.  Slots are the
    pooled sequences of `--batch N`.

    `weights`: f16 CUDA tensors keyed like a checkpoint's tensors --
    "embed" [vocab][hs] (tied lm_head), "norm" [hs], and (layer, name) for the
    names in LAYER_WEIGHT_NAMES, row-major [out][in].  A projection may be int8
    ([out][in] torch.int8) with its f32 per-row scales under (layer, name +
    "_scale") -- the reference's resident-int8 checkpoints; q/k/v and gate/up
    must then be int8 together.  q/k/v and gate/up are concatenated here into
    the fused layouts the library takes (int8 rows with their scales, in the
    same order); the caller's tensors are not modified.  `checkpoint.open_text_decoder` builds one from a
    Qwen3-ASR model directory (config.json + safetensors).
    """

    def __init__(self, weights, nqh=16, nkvh=8, head_dim=128, layers=28, eps=1e-6,
                 max_seq=DECODER_MAX_SEQ, slots=1, max_rows=512, cap=KV_INITIAL_CAP, device=0,
                 rope_theta=1e6, mrope_section=(24, 20, 20), mrope_interleaved=True):
        import torch

        self.t = torch
        self.ctx = Context(nqh, nkvh, head_dim, layers, eps, max_seq, device)
        cs, sn = mrope_text_tables(max_seq, head_dim, rope_theta, tuple(mrope_section),
                                   mrope_interleaved)
        self.ctx.set_rope_tables(cs, sn)
        self.kv = KVPool(self.ctx, slots, min(cap, max_seq))
        self.max_seq = max_seq
        embed = weights["embed"]
        self.vocab, self.hs = int(embed.shape[0]), int(embed.shape[1])
        self.inter = int(weights[(0, "gate_proj")].shape[0])
        self.max_rows = max_rows
        self._keep = [embed, weights["norm"]]
        table = (LayerWeights * layers)()
        for l in range(layers):
            w = {n: weights[(l, n)] for n in LAYER_WEIGHT_NAMES}

            def proj(names, field):
                """Fuse one projection group: f16 rows, or int8 rows + scales."""
                ts = [w[n] for n in names]
                int8 = [t.dtype == torch.int8 for t in ts]
                if any(int8) and not all(int8):
                    raise QasrError(QASR_EINVAL, f"layer {l}: {names} mix int8 and f16")
                mat = torch.cat(ts).contiguous()
                scale = None
                if all(int8):
                    scale = torch.cat([weights[(l, n + "_scale")].float() for n in names])
                    scale = scale.contiguous()
                    if scale.numel() != mat.shape[0]:
                        raise QasrError(QASR_EINVAL, f"layer {l}: {names} scales do not match rows")
                    setattr(table[l], field + "_scale", _dev(scale, f"layer {l} {field} scale",
                                                             torch.float32))
                    self._keep.append(scale)
                    setattr(table[l], field + "_proj", _dev(mat, f"layer {l} {field}", torch.int8))
                else:
                    setattr(table[l], field + "_proj", _dev(mat, f"layer {l} {field}"))
                self._keep.append(mat)

            proj(["q_proj", "k_proj", "v_proj"], "qkv")
            proj(["o_proj"], "o")
            proj(["gate_proj", "up_proj"], "gate_up")
            proj(["down_proj"], "down")
            parts = dict(input_norm=w["input_layernorm"], q_norm=w["q_norm"], k_norm=w["k_norm"],
                         post_norm=w["post_attention_layernorm"])
            for name, t in parts.items():
                setattr(table[l], name, _dev(t, f"layer {l} {name}"))
                self._keep.append(t)
        cfg = DecoderCfg(self.hs, self.inter, self.vocab, max_rows)
        h = _vp()
        _check(load().qasr_decoder_create(self.ctx.handle, ctypes.byref(cfg),
                                          _dev(embed, "embed"), _dev(weights["norm"], "norm"),
                                          table, ctypes.byref(h)))
        self.handle = h
        self.pos = [0] * slots
        self.last = [0] * slots
        self._tok = torch.zeros(max(slots, 1), dtype=torch.int32, device="cuda")
        self._next = torch.zeros(max(slots, 1), dtype=torch.int32, device="cuda")
        self._init_feed(slots)

    def _init_feed(self, slots: int):
        """Device token feed of the pipelined steps (one per slot, written in
        place by each step) and pinned host copies of their results."""
        torch = self.t
        self._feed = torch.zeros(max(slots, 1), dtype=torch.int32, device="cuda")
        self._feed_slots = None  # the slot order _feed currently holds tokens for
        self._pinned = [torch.zeros(max(slots, 1), dtype=torch.int32, pin_memory=True)
                        for _ in range(4)]
        self._ring = 0

    def set_rope_tables(self, cos_u16, sin_u16):
        self.ctx.set_rope_tables(cos_u16, sin_u16)

    def _check_hidden(self, hidden):
        if hidden.dim() != 2 or int(hidden.shape[1]) != self.hs:
            raise QasrError(QASR_EINVAL, f"hidden must be [rows][{self.hs}], got "
                                         f"{list(hidden.shape)}")

    @property
    def slots(self) -> int:
        return len(self.pos)

    def reset_pool(self, slots: int, cap: int):
        """A fresh KV pool of `slots` slots with room for `cap` positions each
        (the reference's fork_capped per slot, decoder.rs:2453-2457); every
        slot starts empty."""
        import torch

        cap = min(max(cap, 1), self.max_seq)
        self.kv.close()
        self.kv = KVPool(self.ctx, slots, cap)
        self.pos = [0] * slots
        self.last = [0] * slots
        self._tok = torch.zeros(max(slots, 1), dtype=torch.int32, device="cuda")
        self._next = torch.zeros(max(slots, 1), dtype=torch.int32, device="cuda")
        self._init_feed(slots)

    def ensure_capacity(self, need: int) -> int:
        """Grow-only, KV_STEP granular; keeps every row already written."""
        return self.kv.ensure_capacity(need, max(self.pos))

    def prefill(self, hidden, kv_start: int = 0, slot: int = 0, logits=None) -> int:
        """hidden: [s][hs] f16 CUDA tensor; prefilled in chunks of max_rows
        rows.  Returns the argmax token after the last row (and fills
        `logits`, a [vocab] f32 CUDA tensor, if given)."""
        self._check_hidden(hidden)
        if logits is not None:
            _need(logits, self.vocab, "logits")
        s = int(hidden.shape[0])
        if kv_start + s > self.max_seq:
            raise QasrError(QASR_ERANGE, f"prefill needs {kv_start + s} positions, "
                                         f"max_seq is {self.max_seq}")
        self.ensure_capacity(kv_start + s)
        hidden = hidden.contiguous()
        for r0 in range(0, s, self.max_rows):
            n = min(self.max_rows, s - r0)
            lg = _dev(logits, "logits", self.t.float32) if logits is not None else None
            _check(load().qasr_decoder_prefill(self.handle, self.kv.handle, slot, kv_start + r0,
                                               n, _dev(hidden[r0:r0 + n], "hidden"),
                                               _dev(self._next, "next", self.t.int32), lg,
                                               _stream(None)))
        tok = int(self._next[0].item())
        self.pos[slot] = kv_start + s
        self.last[slot] = tok
        self._feed_slots = None
        return tok

    def prefill_batch(self, items, logits=None):
        """Prefill several slots at once (prefill_batch, decoder.rs:3599-3637):
        `items` is a sequence of (slot, hidden) or (slot, hidden, kv_start),
        hidden a [s][hs] f16 CUDA tensor.  The projections of segments that fit
        one call together (max_rows rows, 64 segments) run once over all their
        rows; a segment longer than max_rows is prefilled alone in chunks.
        Returns the greedy token after each segment (and fills row i of
        `logits`, [len(items)][vocab] f32, if given)."""
        items = [(int(it[0]), it[1], int(it[2]) if len(it) > 2 else 0) for it in items]
        for _, hidden, _ in items:
            self._check_hidden(hidden)
        if logits is not None:
            _need(logits, len(items) * self.vocab, "logits")
        if len({slot for slot, _, _ in items}) != len(items):
            raise QasrError(QASR_EINVAL, "prefill_batch: two segments share a slot")
        for slot, hidden, start in items:
            if start + int(hidden.shape[0]) > self.max_seq:
                raise QasrError(QASR_ERANGE, f"prefill needs {start + int(hidden.shape[0])} "
                                             f"positions, max_seq is {self.max_seq}")
        if not items:
            return []
        self.ensure_capacity(max(start + int(h.shape[0]) for _, h, start in items))
        toks = [0] * len(items)
        group = []

        def flush():
            if not group:
                return
            idx = [i for i, _ in group]
            rows = [r for _, r in group]
            hidden = self.t.cat([items[i][1] for i in idx]).contiguous()
            segs = (Segment * len(idx))(*[Segment(items[i][0], items[i][2], r)
                                          for i, r in zip(idx, rows)])
            nxt = self.t.zeros(len(idx), dtype=self.t.int32, device="cuda")
            lg, lg_rows = None, None
            if logits is not None:
                lg_rows = self.t.empty((len(idx), self.vocab), dtype=self.t.float32, device="cuda")
                lg = _dev(lg_rows, "logits", self.t.float32)
            _check(load().qasr_decoder_prefill_batch(self.handle, self.kv.handle, segs, len(idx),
                                                     _dev(hidden, "hidden"),
                                                     _dev(nxt, "next", self.t.int32), lg,
                                                     _stream(None)))
            got = nxt.tolist()
            for k, i in enumerate(idx):
                toks[i] = got[k]
                if lg_rows is not None:
                    logits[i].copy_(lg_rows[k])
            group.clear()

        # Calls of about equal row counts (a lone short remainder call would
        # pay every layer's launches for a few rows).
        short = [int(h.shape[0]) for _, h, _ in items if int(h.shape[0]) <= self.max_rows]
        calls = max(1, -(-sum(short) // self.max_rows), -(-len(short) // MAX_PREFILL_SEGMENTS))
        target = -(-sum(short) // calls)
        used = 0
        for i, (slot, hidden, start) in enumerate(items):
            s = int(hidden.shape[0])
            if s > self.max_rows:
                toks[i] = self.prefill(hidden, start, slot=slot,
                                       logits=logits[i] if logits is not None else None)
                continue
            if group and (used + s > self.max_rows or used >= target
                          or len(group) == MAX_PREFILL_SEGMENTS):
                flush()
                used = 0
            group.append((i, s))
            used += s
        flush()
        for i, (slot, hidden, start) in enumerate(items):
            self.pos[slot] = start + int(hidden.shape[0])
            self.last[slot] = toks[i]
        self._feed_slots = None
        return toks

    def step_tokens(self, slots: Sequence[int], pos: Sequence[int], tokens_dev, next_dev,
                    logits=None, stream=None):
        """Asynchronous step: tokens_dev / next_dev are int32 CUDA tensors of
        len(slots) entries (they may be the same tensor)."""
        b = len(slots)
        if len(pos) != b:
            raise QasrError(QASR_EINVAL, f"{len(pos)} positions for {b} slots")
        _need(tokens_dev, b, "tokens")
        _need(next_dev, b, "next")
        if logits is not None:
            _need(logits, b * self.vocab, "logits")
        lg = _dev(logits, "logits", self.t.float32) if logits is not None else None
        _check(load().qasr_decoder_step(self.handle, self.kv.handle, len(slots), _i32(slots),
                                        _i32(pos), _dev(tokens_dev, "tokens", self.t.int32),
                                        _dev(next_dev, "next", self.t.int32), lg,
                                        _stream(stream)))

    def step_async(self, slots: Sequence[int]):
        """Launch one greedy step of `slots` without waiting for it (the
        reference's pipelined decode, record_step/submit_step, decoder.rs:
        2052-2123): each slot's input token comes from the device, where the
        previous step of the same slots left it, so steps can be queued back to
        back; a pinned copy of the results lands with an event.  Returns a
        handle for step_result.  Positions advance at launch."""
        slots = list(slots)
        n = len(slots)
        if any(self.pos[s] >= self.max_seq for s in slots):
            raise QasrError(QASR_ERANGE, f"decode past max_seq {self.max_seq}")
        self.ensure_capacity(max(self.pos[s] for s in slots) + 1)
        if slots != self._feed_slots:
            self._feed[:n].copy_(self.t.tensor([self.last[s] for s in slots], dtype=self.t.int32))
            self._feed_slots = slots
        self.step_tokens(slots, [self.pos[s] for s in slots], self._feed[:n], self._feed[:n])
        host = self._pinned[self._ring]
        self._ring = (self._ring + 1) % len(self._pinned)
        host[:n].copy_(self._feed[:n], non_blocking=True)
        ev = self.t.cuda.Event()
        ev.record()
        for s in slots:
            self.pos[s] += 1
        return (slots, host, ev)

    def step_result(self, handle):
        """The tokens of a step launched by step_async (waits for it)."""
        slots, host, ev = handle
        ev.synchronize()
        toks = host[:len(slots)].tolist()
        for s, t in zip(slots, toks):
            self.last[s] = t
        return toks

    def step(self, slots: Optional[Sequence[int]] = None, logits=None):
        """One greedy step of the given slots (default: all); returns their
        next tokens."""
        slots = list(range(len(self.pos))) if slots is None else list(slots)
        if any(self.pos[s] >= self.max_seq for s in slots):
            raise QasrError(QASR_ERANGE, f"decode past max_seq {self.max_seq}")
        self.ensure_capacity(max(self.pos[s] for s in slots) + 1)
        b = len(slots)
        self._tok[:b].copy_(self.t.tensor([self.last[s] for s in slots], dtype=self.t.int32))
        self.step_tokens(slots, [self.pos[s] for s in slots], self._tok[:b], self._next[:b],
                         logits)
        toks = self._next[:b].tolist()
        self._feed_slots = None
        for s, t in zip(slots, toks):
            self.pos[s] += 1
            self.last[s] = t
        return toks

    def close(self):
        if getattr(self, "handle", None):
            load().qasr_decoder_destroy(self.handle)
            self.handle = None
        self.kv.close()
        self.ctx.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
