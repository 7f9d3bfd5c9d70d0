"""ctypes wrapper over liboracle.so, the CPU restatement of Qwen3-ASR's decoder
self-attention path (oracle.cpp).

TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import this module, as the checker or as the
timed CPU baseline.  The product library (libqasr_attn.so) never calls it.

Each wrapper names the reference lines its C function restates (paths under
the eclipse005/qwen3-asr-wgpu checkout):
  norm_rope_head  src/cpu_decoder.rs:274-290
  attention       src/cpu_decoder.rs:292-365
  layer_attn      src/cpu_decoder.rs:398-427 (q/k norm-RoPE, KV write, attention)
  mrope tables    src/mrope.rs:5-80, src/inference.rs:1038-1049
  kv_target_cap   src/cpu_decoder.rs:227-229, src/decoder.rs:1610
  TextDecoder     src/cpu_decoder.rs:261-272, 367-532 (whole decoder, greedy)
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u64p = ctypes.POINTER(ctypes.c_uint64)


class Shape(ctypes.Structure):
    _fields_ = [
        ("nqh", ctypes.c_int32),
        ("nkvh", ctypes.c_int32),
        ("hd", ctypes.c_int32),
        ("max_seq", ctypes.c_int32),
        ("eps", ctypes.c_float),
    ]


class DecCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("hs", "nqh", "nkvh", "hd", "inter", "layers", "vocab", "max_seq")] + [
        ("eps", ctypes.c_float)]


def build() -> str:
    """Compile liboracle.so with the committed Makefile (g++)."""
    import subprocess

    subprocess.run(["make", "-C", _HERE, "-s", "liboracle.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is not built; run `make -C oracle`")
        L = ctypes.CDLL(_LIB_PATH)
        L.qo_f16_from_f32.restype = ctypes.c_uint16
        L.qo_f16_from_f32.argtypes = [ctypes.c_float]
        L.qo_f32_from_f16.restype = ctypes.c_float
        L.qo_f32_from_f16.argtypes = [ctypes.c_uint16]
        L.qo_f16_to_f32_array.argtypes = [_u16p, _f32p, ctypes.c_int64]
        L.qo_f32_to_f16_array.argtypes = [_f32p, _u16p, ctypes.c_int64]
        L.qo_build_dim_map.argtypes = [_i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p]
        L.qo_mrope_cos_sin.argtypes = [_i64p, ctypes.c_int, ctypes.c_int, ctypes.c_double,
                                       _i32p, ctypes.c_int, ctypes.c_int, _f32p, _f32p]
        L.qo_text_rope_tables_f16.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_double,
                                              _i32p, ctypes.c_int, ctypes.c_int, _u16p, _u16p]
        L.qo_norm_rope_head.argtypes = [_u16p, _f32p, _f32p, _f32p, ctypes.c_int,
                                        ctypes.c_float, _u16p]
        L.qo_layer_attn.argtypes = [ctypes.POINTER(Shape), ctypes.c_int, _u16p, ctypes.c_int,
                                    ctypes.c_int, _u16p, _u16p, _f32p, _f32p, ctypes.c_int,
                                    _f32p, _f32p, _u16p, _u16p, ctypes.c_int]
        L.qo_qk_norm_rope_append.argtypes = [ctypes.POINTER(Shape), ctypes.c_int, _u16p,
                                             ctypes.c_int, ctypes.c_int, _u16p, _u16p, _f32p,
                                             _f32p, ctypes.c_int, _f32p, _f32p, _u16p]
        L.qo_attention.argtypes = [ctypes.POINTER(Shape), ctypes.c_int, _u16p, ctypes.c_int,
                                   ctypes.c_int, _f32p, _f32p, _u16p, ctypes.c_int]
        L.qo_kv_target_cap.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.qo_dec_create.restype = ctypes.c_void_p
        L.qo_dec_create.argtypes = [ctypes.POINTER(DecCfg), _u16p, _u16p,
                                    ctypes.POINTER(_u16p), ctypes.c_int]
        L.qo_dec_destroy.argtypes = [ctypes.c_void_p]
        L.qo_dec_destroy.restype = None
        L.qo_dec_set_rope.argtypes = [ctypes.c_void_p, _u16p, _u16p, ctypes.c_int]
        L.qo_dec_prefill.argtypes = [ctypes.c_void_p, _u16p, ctypes.c_int, ctypes.c_int, _f32p]
        L.qo_dec_step.argtypes = [ctypes.c_void_p, _f32p]
        L.qo_dec_pos.argtypes = [ctypes.c_void_p]
        L.qo_splitmix64.restype = ctypes.c_uint64
        L.qo_splitmix64.argtypes = [_u64p]
        L.qo_fill_normal_f16.argtypes = [_u64p, ctypes.c_int64, ctypes.c_double,
                                         ctypes.c_double, _u16p]
        L.qo_uniform_int.restype = ctypes.c_int32
        L.qo_uniform_int.argtypes = [_u64p, ctypes.c_int32, ctypes.c_int32]
        L.qo_hardware_threads.restype = ctypes.c_int
        L.qo_softmax_weights.argtypes = [_f32p, _f32p, ctypes.c_int64, ctypes.c_float, _f32p]
        L.qo_softmax_weights.restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(t)


def f16_from_f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().qo_f32_to_f16_array(_p(a, _f32p), _p(out, _u16p), a.size)
    return out


def f32_from_f16(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().qo_f16_to_f32_array(_p(h, _u16p), _p(out, _f32p), h.size)
    return out


def build_dim_map(section, half: int, interleaved: bool):
    sec = np.ascontiguousarray(section, dtype=np.int32)
    out = np.full(half, -1, dtype=np.int32)
    rc = lib().qo_build_dim_map(_p(sec, _i32p), len(sec), half, int(interleaved), _p(out, _i32p))
    if rc != 0:
        raise ValueError("dim map shorter than half (quotas too small)")
    return out.tolist()


def mrope_cos_sin(pos3, head_dim: int, theta: float, section, interleaved: bool):
    pos3 = np.ascontiguousarray(pos3, dtype=np.int64)
    assert pos3.ndim == 2 and pos3.shape[0] == 3
    n = pos3.shape[1]
    sec = np.ascontiguousarray(section, dtype=np.int32)
    c = np.empty((n, head_dim), dtype=np.float32)
    s = np.empty((n, head_dim), dtype=np.float32)
    rc = lib().qo_mrope_cos_sin(_p(pos3, _i64p), n, head_dim, theta, _p(sec, _i32p), len(sec),
                                int(interleaved), _p(c, _f32p), _p(s, _f32p))
    if rc != 0:
        raise ValueError("bad mrope arguments")
    return c, s


def text_rope_tables_f16(rows: int, head_dim: int = 128, theta: float = 1e6,
                         section=(24, 20, 20), interleaved: bool = True):
    sec = np.ascontiguousarray(section, dtype=np.int32)
    c = np.empty((rows, head_dim), dtype=np.uint16)
    s = np.empty((rows, head_dim), dtype=np.uint16)
    rc = lib().qo_text_rope_tables_f16(rows, head_dim, theta, _p(sec, _i32p), len(sec),
                                       int(interleaved), _p(c, _u16p), _p(s, _u16p))
    if rc != 0:
        raise ValueError("bad rope table arguments")
    return c, s


def norm_rope_head(raw, gain_f32, cos_row, sin_row, eps: float = 1e-6) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint16)
    g = np.ascontiguousarray(gain_f32, dtype=np.float32)
    c = np.ascontiguousarray(cos_row, dtype=np.float32)
    s = np.ascontiguousarray(sin_row, dtype=np.float32)
    out = np.empty(raw.shape[-1], dtype=np.uint16)
    lib().qo_norm_rope_head(_p(raw, _u16p), _p(g, _f32p), _p(c, _f32p), _p(s, _f32p),
                            raw.shape[-1], eps, _p(out, _u16p))
    return out


def make_shape(nqh=16, nkvh=8, hd=128, max_seq=16384, eps=1e-6) -> Shape:
    return Shape(nqh, nkvh, hd, max_seq, eps)


def layer_attn(shape: Shape, cap: int, qkv, q0: int, q_gain, k_gain, cos_f32, sin_f32,
               k_cache, v_cache, nthreads: int = 0):
    """Stage (a) + attention for rows q0..q0+rows-1 of one sequence; k_cache and
    v_cache ([nkvh][cap][hd] f32) are updated in place.  Returns (q_out, attn_out)."""
    qkv = np.ascontiguousarray(qkv, dtype=np.uint16)
    rows = qkv.shape[0]
    q_gain = np.ascontiguousarray(q_gain, dtype=np.uint16)
    k_gain = np.ascontiguousarray(k_gain, dtype=np.uint16)
    assert k_cache.dtype == np.float32 and v_cache.dtype == np.float32
    assert k_cache.shape == (shape.nkvh, cap, shape.hd) == v_cache.shape
    q_out = np.empty((rows, shape.nqh * shape.hd), dtype=np.uint16)
    attn = np.empty((rows, shape.nqh * shape.hd), dtype=np.uint16)
    rc = lib().qo_layer_attn(ctypes.byref(shape), cap, _p(qkv, _u16p), rows, q0,
                             _p(q_gain, _u16p), _p(k_gain, _u16p),
                             _p(cos_f32, _f32p), _p(sin_f32, _f32p), cos_f32.shape[0],
                             _p(k_cache, _f32p), _p(v_cache, _f32p),
                             _p(q_out, _u16p), _p(attn, _u16p), nthreads)
    if rc != 0:
        raise ValueError("qo_layer_attn rejected its arguments")
    return q_out, attn


def qk_norm_rope_append(shape: Shape, cap: int, qkv, q0: int, q_gain, k_gain, cos_f32, sin_f32,
                        k_cache, v_cache):
    """Stage (a) only (cpu_decoder.rs:398-423): returns roped q; updates the caches."""
    qkv = np.ascontiguousarray(qkv, dtype=np.uint16)
    rows = qkv.shape[0]
    q_gain = np.ascontiguousarray(q_gain, dtype=np.uint16)
    k_gain = np.ascontiguousarray(k_gain, dtype=np.uint16)
    assert k_cache.dtype == np.float32 and v_cache.dtype == np.float32
    assert k_cache.shape == (shape.nkvh, cap, shape.hd) == v_cache.shape
    q_out = np.empty((rows, shape.nqh * shape.hd), dtype=np.uint16)
    rc = lib().qo_qk_norm_rope_append(ctypes.byref(shape), cap, _p(qkv, _u16p), rows, q0,
                                      _p(q_gain, _u16p), _p(k_gain, _u16p), _p(cos_f32, _f32p),
                                      _p(sin_f32, _f32p), cos_f32.shape[0], _p(k_cache, _f32p),
                                      _p(v_cache, _f32p), _p(q_out, _u16p))
    if rc != 0:
        raise ValueError("qo_qk_norm_rope_append rejected its arguments")
    return q_out


def attention(shape: Shape, cap: int, q, q0: int, k_cache, v_cache, nthreads: int = 0):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    rows = q.shape[0]
    out = np.empty((rows, shape.nqh * shape.hd), dtype=np.uint16)
    rc = lib().qo_attention(ctypes.byref(shape), cap, _p(q, _u16p), rows, q0,
                            _p(k_cache, _f32p), _p(v_cache, _f32p), _p(out, _u16p), nthreads)
    if rc != 0:
        raise ValueError("qo_attention rejected its arguments")
    return out


def softmax_weights(s, m, scale: float) -> np.ndarray:
    """expf(f32(s*scale) - f32(m*scale)) per element (glibc expf), the
    reference attention's softmax weight (cpu_decoder.rs:292-365)."""
    s = np.ascontiguousarray(s, dtype=np.float32)
    m = np.ascontiguousarray(m, dtype=np.float32)
    assert s.shape == m.shape
    out = np.empty(s.shape, np.float32)
    lib().qo_softmax_weights(_p(s, _f32p), _p(m, _f32p), s.size, scale, _p(out, _f32p))
    return out


def kv_target_cap(need: int, cap: int, max_seq: int) -> int:
    return int(lib().qo_kv_target_cap(need, cap, max_seq))


def hardware_threads() -> int:
    return int(lib().qo_hardware_threads())


class Rng:
    """SplitMix64 stream; normals by Box-Muller (f64) -> f32 -> f16 RNE."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint64(seed & 0xFFFFFFFFFFFFFFFF)

    def next_u64(self) -> int:
        return int(lib().qo_splitmix64(ctypes.byref(self.state)))

    def normal_f16(self, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        out = np.empty(shape, dtype=np.uint16)
        lib().qo_fill_normal_f16(ctypes.byref(self.state), out.size, mean, std, _p(out, _u16p))
        return out

    def uniform_int(self, lo: int, hi: int) -> int:
        return int(lib().qo_uniform_int(ctypes.byref(self.state), lo, hi))


# Per-layer tensor order of TextDecoder (checkpoint names under model.layers.N).
LAYER_TENSORS = ("input_layernorm", "post_attention_layernorm", "q_norm", "k_norm", "q_proj",
                 "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


class TextDecoder:
    """CpuTextDecoder (src/cpu_decoder.rs) for one sequence: prefill then greedy
    steps, returning argmax tokens and (optionally) the logits.  `weights` maps
    "embed", "norm" and (layer, name) for name in LAYER_TENSORS to f16 arrays
    (uint16 bits, checkpoint layout [out][in])."""

    def __init__(self, cfg: dict, weights, cap: int, cos_f16, sin_f16):
        L = lib()
        self.cfg = cfg
        c = DecCfg(cfg["hs"], cfg["nqh"], cfg["nkvh"], cfg["hd"], cfg["inter"], cfg["layers"],
                   cfg["vocab"], cfg["max_seq"], cfg["eps"])
        self._keep = [np.ascontiguousarray(weights["embed"], dtype=np.uint16),
                      np.ascontiguousarray(weights["norm"], dtype=np.uint16)]
        ptrs = (_u16p * (11 * cfg["layers"]))()
        for l in range(cfg["layers"]):
            for i, n in enumerate(LAYER_TENSORS):
                a = np.ascontiguousarray(weights[(l, n)], dtype=np.uint16)
                self._keep.append(a)
                ptrs[11 * l + i] = _p(a, _u16p)
        self._h = L.qo_dec_create(ctypes.byref(c), _p(self._keep[0], _u16p),
                                  _p(self._keep[1], _u16p), ptrs, cap)
        if not self._h:
            raise ValueError("qo_dec_create rejected the configuration")
        # the decoder reads the weights in place: self._keep stays alive with it
        cs = np.ascontiguousarray(cos_f16, dtype=np.uint16)
        sn = np.ascontiguousarray(sin_f16, dtype=np.uint16)
        if L.qo_dec_set_rope(self._h, _p(cs, _u16p), _p(sn, _u16p), cs.shape[0]):
            raise ValueError("qo_dec_set_rope failed")

    def prefill(self, hidden_f16, kv_start: int, want_logits: bool = True):
        h = np.ascontiguousarray(hidden_f16, dtype=np.uint16)
        logits = np.empty(self.cfg["vocab"], np.float32) if want_logits else None
        tok = lib().qo_dec_prefill(self._h, _p(h, _u16p), h.shape[0], kv_start,
                                   _p(logits, _f32p) if want_logits else None)
        if tok < 0:
            raise ValueError("qo_dec_prefill failed")
        return tok, logits

    def step(self, want_logits: bool = True):
        logits = np.empty(self.cfg["vocab"], np.float32) if want_logits else None
        tok = lib().qo_dec_step(self._h, _p(logits, _f32p) if want_logits else None)
        if tok < 0:
            raise ValueError("qo_dec_step failed")
        return tok, logits

    @property
    def pos(self) -> int:
        return lib().qo_dec_pos(self._h)

    def close(self):
        if self._h:
            lib().qo_dec_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()
