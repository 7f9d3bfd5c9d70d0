"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, its host-side table builder equals the oracle's bit for bit,
and argument errors come back as status codes with a message (never a crash).
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

import qasr_attn
from workloads import tables

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "qasr_attn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qasr_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(qasr_attn.ABI_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = qasr_attn.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.qasr_abi_version() == 2


def test_library_is_gfx950_hip_code():
    data = open(qasr_attn.LIB_PATH, "rb").read()
    assert b"gfx950" in data
    assert b"decode_attn_kernel" in data and b"prefill_attn_kernel" in data


def test_host_tables_equal_oracle(O):
    tab = tables(O)
    c, s = qasr_attn.mrope_text_tables(16384)
    assert np.array_equal(c, tab.cos_u16) and np.array_equal(s, tab.sin_u16)
    # blocked map and other sections give the same text tables
    c2, s2 = qasr_attn.mrope_text_tables(64, section=(16, 24, 24), interleaved=False)
    assert np.array_equal(c2, tab.cos_u16[:64]) and np.array_equal(s2, tab.sin_u16[:64])


def test_host_tables_reject_short_quotas():
    with pytest.raises(qasr_attn.QasrError) as e:
        qasr_attn.mrope_text_tables(4, section=(10, 10, 10), interleaved=True)
    assert e.value.code == qasr_attn.QASR_EINVAL


def test_ctx_create_rejects_bad_shapes():
    lib = qasr_attn.load()
    h = ctypes.c_void_p()
    for cfg in (qasr_attn.AttnCfg(16, 8, 64, 28, 1e-6, 16384),   # head_dim
                qasr_attn.AttnCfg(16, 16, 128, 28, 1e-6, 16384),  # REP 1
                qasr_attn.AttnCfg(16, 8, 128, 0, 1e-6, 16384),    # layers
                qasr_attn.AttnCfg(16, 8, 128, 28, 1e-6, 0),       # max_seq
                qasr_attn.AttnCfg(16, 8, 128, 28, 1e-6, (1 << 24) + 1)):  # max_seq past 2^24
        rc = lib.qasr_ctx_create(ctypes.byref(cfg), 0, ctypes.byref(h))
        assert rc == qasr_attn.QASR_EINVAL
        assert lib.qasr_last_error()
        assert not h.value


def test_null_arguments_are_errors():
    lib = qasr_attn.load()
    assert lib.qasr_ctx_create(None, 0, None) == qasr_attn.QASR_EINVAL
    assert lib.qasr_decode_attn(None, None, 0, 1, None, None, None, None, None) == qasr_attn.QASR_EINVAL
    assert lib.qasr_prefill_attn(None, None, 0, 0, 0, 1, None, None, None) == qasr_attn.QASR_EINVAL
    assert lib.qasr_kv_ensure_capacity(None, 10, 0, None) == qasr_attn.QASR_EINVAL
    lib.qasr_ctx_destroy(None)
    lib.qasr_kv_destroy(None)


def test_ctx_create_without_device_fails_cleanly():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible: covered by the gpu tests")
    lib = qasr_attn.load()
    cfg = qasr_attn.AttnCfg(16, 8, 128, 28, 1e-6, 16384)
    h = ctypes.c_void_p()
    rc = lib.qasr_ctx_create(ctypes.byref(cfg), 0, ctypes.byref(h))
    assert rc in (qasr_attn.QASR_EINVAL, qasr_attn.QASR_EDEVICE)
    assert not h.value
