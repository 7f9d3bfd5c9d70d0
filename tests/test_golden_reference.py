"""The oracle and the library against the known answers the reference's own
unit tests hold for this path (tests/golden/reference_known_answers.json,
written by tests/golden/make_reference_known_answers.py from src/mrope.rs:86-107
and src/config.rs:102-110, 177-195, 261-290)."""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "reference_known_answers.json")))


def test_dim_map_known_answers(O):
    for case in GOLD["build_dim_map"]:
        m = O.build_dim_map(case["section"], case["half"], case["interleaved"])
        if "map" in case:
            assert m == case["map"], case["source"]
        else:
            assert len(m) == case["len"], case["source"]
            for axis, n in case["counts"].items():
                assert m.count(int(axis)) == n, case["source"]
            assert m[:len(case["prefix"])] == case["prefix"], case["source"]


def test_mrope_text_positions_known_answers(O):
    for case in GOLD["compute_mrope_cos_sin"]:
        n = case["text_positions"]
        pos3 = np.tile(np.arange(n, dtype=np.int64), (3, 1))  # text_positions: all axes equal
        c, _ = O.mrope_cos_sin(pos3, case["head_dim"], case["theta"], case["section"],
                               case["interleaved"])
        flat = c.reshape(-1)
        assert flat.size == case["cos_len"], case["source"]
        (a0, a1), (b0, b1) = case["halves_equal"]
        assert np.array_equal(flat[a0:a1], flat[b0:b1]), case["source"]


def test_library_tables_match_oracle_for_reference_defaults(O):
    """The library's host-side table builder (qasr_mrope_text_tables) with the
    reference's default section / theta equals the oracle bitwise."""
    import qasr_attn

    d = GOLD["text_decoder_defaults"]
    c_lib, s_lib = qasr_attn.mrope_text_tables(300, d["head_dim"], d["rope_theta"],
                                               tuple(d["mrope_section"]), d["mrope_interleaved"])
    c_or, s_or = O.text_rope_tables_f16(300, d["head_dim"], d["rope_theta"],
                                        tuple(d["mrope_section"]), d["mrope_interleaved"])
    assert np.array_equal(c_lib, c_or) and np.array_equal(s_lib, s_or)


def test_binding_defaults_are_the_reference_decoder_shape():
    import inspect

    import qasr_attn

    sig = inspect.signature(qasr_attn.Context.__init__).parameters
    for cfg in (GOLD["text_decoder_defaults"], GOLD["hf_native_text_config"]):
        assert sig["nqh"].default == cfg["num_attention_heads"], cfg["source"]
        assert sig["nkvh"].default == cfg["num_key_value_heads"], cfg["source"]
        assert sig["head_dim"].default == cfg["head_dim"], cfg["source"]
        assert sig["layers"].default == cfg["num_hidden_layers"], cfg["source"]
        assert abs(sig["eps"].default - cfg["rms_norm_eps"]) == 0.0, cfg["source"]
