"""CPU tests of the Python binding's argument checks.

The C ABI receives raw device pointers, so a caller tensor smaller than the
rows a call implies would be read or written out of bounds on the device.
The wrappers refuse such calls with the library's EINVAL before anything is
launched; these tests drive them with CPU tensors and a stand-in context, so
no GPU is needed (a call that passed the size checks would stop at the
"must live on the GPU" check instead).
"""
from __future__ import annotations

import types

import pytest

torch = pytest.importorskip("torch")

import qasr_attn as Q  # noqa: E402

NQH, NKVH, HD = 16, 8, 128
TOT, QD = (NQH + 2 * NKVH) * HD, NQH * HD


def _ctx():
    cfg = types.SimpleNamespace(head_dim=HD, num_attention_heads=NQH, num_key_value_heads=NKVH)
    return types.SimpleNamespace(cfg=cfg, nqh=NQH, nkvh=NKVH, handle=None)


KV = types.SimpleNamespace(handle=None)


def _t(*shape, dtype=torch.float16):
    return torch.zeros(shape, dtype=dtype)


def _refused(fn):
    with pytest.raises(Q.QasrError) as e:
        fn()
    assert e.value.code == Q.QASR_EINVAL
    return str(e.value)


def _passed_size_checks(fn):
    """Correct sizes get past the size checks and stop at the device check."""
    with pytest.raises(ValueError, match="GPU"):
        fn()


def test_stage_a_refuses_short_tensors():
    c = _ctx()
    segs = [(0, 0, 3), (1, 10, 2)]
    g = _t(HD)
    _refused(lambda: Q.qk_norm_rope_append(c, KV, 0, segs, _t(4, TOT), g, g, _t(5, QD)))
    _refused(lambda: Q.qk_norm_rope_append(c, KV, 0, segs, _t(5, TOT), g, g, _t(4, QD)))
    _refused(lambda: Q.qk_norm_rope_append(c, KV, 0, segs, _t(5, TOT), _t(64), g, _t(5, QD)))
    _refused(lambda: Q.qk_norm_rope_append(c, KV, 0, segs, _t(5, TOT), g, _t(256), _t(5, QD)))
    _passed_size_checks(lambda: Q.qk_norm_rope_append(c, KV, 0, segs, _t(5, TOT), g, g,
                                                      _t(5, QD)))


def test_decode_refuses_short_tensors_and_slot_count():
    c = _ctx()
    g = _t(HD)
    _refused(lambda: Q.decode_attn(c, KV, 0, [5, 6, 7], _t(2, QD), _t(3, QD)))
    _refused(lambda: Q.decode_attn(c, KV, 0, [5, 6, 7], _t(3, QD), _t(2, QD)))
    _refused(lambda: Q.decode_attn(c, KV, 0, [5, 6], _t(2, QD), _t(2, QD), slots=[0]))
    _passed_size_checks(lambda: Q.decode_attn(c, KV, 0, [5, 6], _t(2, QD), _t(2, QD)))
    _refused(lambda: Q.decode_step(c, KV, 0, [4, 4], _t(1, TOT), g, g, _t(2, QD)))
    _refused(lambda: Q.decode_step(c, KV, 0, [4, 4], _t(2, TOT), g, g, _t(1, QD)))
    _refused(lambda: Q.decode_step(c, KV, 0, [4, 4], _t(2, TOT), g, g, _t(2, QD),
                                   slots=[0, 1, 2]))
    _passed_size_checks(lambda: Q.decode_step(c, KV, 0, [4, 4], _t(2, TOT), g, g, _t(2, QD)))


def test_prefill_refuses_short_tensors():
    c = _ctx()
    g = _t(HD)
    _refused(lambda: Q.prefill_attn(c, KV, 0, 0, 0, 10, _t(9, QD), _t(10, QD)))
    _refused(lambda: Q.prefill_attn(c, KV, 0, 0, 0, 10, _t(10, QD), _t(9, QD)))
    _passed_size_checks(lambda: Q.prefill_attn(c, KV, 0, 0, 0, 10, _t(10, QD), _t(10, QD)))
    segs = [(0, 0, 7), (1, 0, 9)]
    _refused(lambda: Q.prefill_attn_batch(c, KV, 0, segs, _t(15, QD), _t(16, QD)))
    _refused(lambda: Q.prefill_attn_batch(c, KV, 0, segs, _t(16, QD), _t(15, QD)))
    _passed_size_checks(lambda: Q.prefill_attn_batch(c, KV, 0, segs, _t(16, QD), _t(16, QD)))
    _refused(lambda: Q.prefill_layer(c, KV, 0, 0, 0, 6, _t(5, TOT), g, g, _t(6, QD), _t(6, QD)))
    _refused(lambda: Q.prefill_layer(c, KV, 0, 0, 0, 6, _t(6, TOT), g, g, _t(5, QD), _t(6, QD)))
    _refused(lambda: Q.prefill_layer(c, KV, 0, 0, 0, 6, _t(6, TOT), g, g, _t(6, QD), _t(5, QD)))
    _passed_size_checks(lambda: Q.prefill_layer(c, KV, 0, 0, 0, 6, _t(6, TOT), g, g, _t(6, QD),
                                                _t(6, QD)))


def test_dequant_refuses_mismatched_scale_and_output():
    c = _ctx()
    q = _t(4, 16, dtype=torch.int8)
    _refused(lambda: Q.dequant_i8(c, q, _t(3, dtype=torch.float32), _t(4, 16)))
    _refused(lambda: Q.dequant_i8(c, q, _t(4, dtype=torch.float32), _t(4, 15)))
    _refused(lambda: Q.dequant_i8(c, _t(64, dtype=torch.int8), _t(4, dtype=torch.float32)))
    _passed_size_checks(lambda: Q.dequant_i8(c, q, _t(4, dtype=torch.float32), _t(4, 16)))


def _decoder_stub(hs=1024, vocab=4096):
    """A TextDecoder shell with only the fields its checks read."""
    d = object.__new__(Q.TextDecoder)
    d.t, d.hs, d.vocab, d.max_seq, d.max_rows = torch, hs, vocab, 16384, 512
    d.pos, d.last = [0, 0], [0, 0]
    return d


def test_text_decoder_refuses_bad_hidden_and_outputs():
    d = _decoder_stub()
    msg = _refused(lambda: d.prefill(_t(5, 1000)))
    assert "[rows][1024]" in msg
    _refused(lambda: d.prefill(_t(5 * 1024)))
    _refused(lambda: d.prefill(_t(5, 1024), logits=_t(100, dtype=torch.float32)))
    _refused(lambda: d.prefill_batch([(0, _t(3, 1024)), (1, _t(3, 512))]))
    _refused(lambda: d.prefill_batch([(0, _t(3, 1024)), (1, _t(3, 1024))],
                                     logits=_t(1, 4096, dtype=torch.float32)))
    i32 = lambda n: _t(n, dtype=torch.int32)  # noqa: E731
    _refused(lambda: d.step_tokens([0, 1], [5], i32(2), i32(2)))
    _refused(lambda: d.step_tokens([0, 1], [5, 6], i32(1), i32(2)))
    _refused(lambda: d.step_tokens([0, 1], [5, 6], i32(2), i32(1)))
    _refused(lambda: d.step_tokens([0, 1], [5, 6], i32(2), i32(2),
                                   logits=_t(4096, dtype=torch.float32)))
    _passed_size_checks(lambda: d.step_tokens([0, 1], [5, 6], i32(2), i32(2),
                                              logits=_t(2, 4096, dtype=torch.float32)))
