"""checkpoint.py on the CPU: config.json parsing against the reference's own
config tests (transcribed in tests/golden/reference_known_answers.json), HF
name remapping, and loading a synthetic sharded safetensors checkpoint with
bf16 / f32 / f16 tensors: the f16 values must be the RNE narrowing of each
tensor (checked bitwise against numpy's conversion of the exact f32 value)."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

import checkpoint as C

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "reference_known_answers.json")


def _known():
    with open(GOLDEN) as f:
        return json.load(f)


@pytest.mark.parametrize("case", range(6))
def test_config_parsing_matches_reference_known_answers(case):
    c = _known()["config_parsing"][case]
    got = C.parse_text_config(c["json"])
    for k, v in c["expect"].items():
        assert got[k] == v, (c["source"], k, got[k], v)


def test_config_defaults_match_reference():
    want = _known()["text_decoder_defaults"]
    got = C.parse_text_config({"thinker_config": {"audio_config": {}, "text_config": {}}})
    for k in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
              "num_attention_heads", "num_key_value_heads", "head_dim", "rms_norm_eps",
              "rope_theta", "mrope_section", "mrope_interleaved"):
        assert got[k] == want[k], k


def test_config_without_text_section_is_refused():
    with pytest.raises(C.CheckpointError):
        C.parse_text_config({"audio_config": {}})


def test_remap_hf_names():
    assert C.remap_name("model.language_model.layers.3.mlp.up_proj.weight") == \
        "thinker.model.layers.3.mlp.up_proj.weight"
    assert C.remap_name("thinker.model.norm.weight") == "thinker.model.norm.weight"
    assert C.remap_name("model.audio_tower.conv1.weight") == "model.audio_tower.conv1.weight"


SHAPES = dict(hs=256, inter=512, nqh=2, nkvh=1, hd=128, vocab=1000, layers=2)


def _tensors(rng, hf_names: bool):
    """name -> (np float32 values, storage dtype) of a tiny text decoder."""
    s = SHAPES
    qd, kd = s["nqh"] * s["hd"], s["nkvh"] * s["hd"]
    pre = "model.language_model" if hf_names else "thinker.model"
    out = {f"{pre}.embed_tokens.weight": ((s["vocab"], s["hs"]), "bf16"),
           f"{pre}.norm.weight": ((s["hs"],), "f32")}
    for l in range(s["layers"]):
        p = f"{pre}.layers.{l}"
        out.update({
            f"{p}.input_layernorm.weight": ((s["hs"],), "f16"),
            f"{p}.post_attention_layernorm.weight": ((s["hs"],), "bf16"),
            f"{p}.self_attn.q_norm.weight": ((s["hd"],), "bf16"),
            f"{p}.self_attn.k_norm.weight": ((s["hd"],), "f32"),
            f"{p}.self_attn.q_proj.weight": ((qd, s["hs"]), "bf16"),
            f"{p}.self_attn.k_proj.weight": ((kd, s["hs"]), "f16"),
            f"{p}.self_attn.v_proj.weight": ((kd, s["hs"]), "f32"),
            f"{p}.self_attn.o_proj.weight": ((s["hs"], qd), "bf16"),
            f"{p}.mlp.gate_proj.weight": ((s["inter"], s["hs"]), "bf16"),
            f"{p}.mlp.up_proj.weight": ((s["inter"], s["hs"]), "f16"),
            f"{p}.mlp.down_proj.weight": ((s["hs"], s["inter"]), "bf16"),
        })
    vals = {}
    for name, (shape, dt) in out.items():
        v = rng.standard_normal(shape).astype(np.float32) * 0.05
        vals[name] = (v, dt)
    return vals


def _write_checkpoint(tmp, vals, shards: int):
    import torch
    from safetensors.torch import save_file

    names = sorted(vals)
    per = [names[i::shards] for i in range(shards)]
    weight_map = {}
    for i, group in enumerate(per):
        fname = f"model-{i + 1:05d}-of-{shards:05d}.safetensors" if shards > 1 else "model.safetensors"
        ts = {}
        for n in group:
            v, dt = vals[n]
            t = torch.from_numpy(v)
            ts[n] = t.to({"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dt])
            weight_map[n] = fname
        save_file(ts, os.path.join(tmp, fname))
    if shards > 1:
        with open(os.path.join(tmp, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {}, "weight_map": weight_map}, f)


def _expected_f16(v: np.ndarray, dt: str) -> np.ndarray:
    """The stored value, widened exactly to f32, then RNE to f16 (numpy)."""
    if dt == "bf16":  # bf16 keeps the top 16 bits of the f32 pattern, RNE
        b = v.view(np.uint32).astype(np.uint64)
        r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint32) << 16
        stored = r.astype(np.uint32).view(np.float32)
    elif dt == "f16":
        stored = v.astype(np.float16).astype(np.float32)
    else:
        stored = v
    return stored.astype(np.float16)


@pytest.mark.parametrize("hf_names,shards", [(True, 3), (False, 1)])
def test_load_text_weights_narrows_and_maps(tmp_path, hf_names, shards):
    rng = np.random.default_rng(5)
    vals = _tensors(rng, hf_names)
    _write_checkpoint(str(tmp_path), vals, shards)
    W = C.load_text_weights(str(tmp_path), SHAPES["layers"], device="cpu")
    pre = "model.language_model" if hf_names else "thinker.model"
    key_of = {f"{pre}.embed_tokens.weight": "embed", f"{pre}.norm.weight": "norm"}
    for l in range(SHAPES["layers"]):
        for key, suffix in C._LAYER_TENSORS:
            key_of[f"{pre}.layers.{l}.{suffix}"] = (l, key)
    assert len(W) == len(key_of)
    for name, key in key_of.items():
        v, dt = vals[name]
        got = W[key].numpy()
        assert got.dtype == np.float16 and got.shape == v.shape, name
        assert np.array_equal(got.view(np.uint16), _expected_f16(v, dt).view(np.uint16)), name


def test_missing_tensors_are_refused(tmp_path):
    rng = np.random.default_rng(6)
    vals = _tensors(rng, True)
    drop = "model.language_model.layers.1.mlp.down_proj.weight"
    _write_checkpoint(str(tmp_path), {k: v for k, v in vals.items() if k != drop}, 1)
    with pytest.raises(C.CheckpointError, match="missing"):
        C.load_text_weights(str(tmp_path), SHAPES["layers"], device="cpu")


def _int8_checkpoint(tmp, vals, skip_scale=None, float_linear=None):
    """Every decoder linear as I8 with an F32 `.weight_scale` (the reference's
    int8 export layout); returns the int8 arrays and scales written."""
    import torch
    from safetensors.torch import save_file

    rng = np.random.default_rng(8)
    ts, q8 = {}, {}
    for n, (v, _) in vals.items():
        base = n[:-len(".weight")]
        if any(n.endswith(f"{p}.weight") for p in C._LINEARS) and n != float_linear:
            q = rng.integers(-128, 128, size=v.shape, dtype=np.int8)
            sc = (rng.random(v.shape[0]).astype(np.float32) + 0.5) * 1e-3
            ts[n] = torch.from_numpy(q)
            if n != skip_scale:
                ts[base + C.INT8_SCALE_SUFFIX] = torch.from_numpy(sc)
            q8[n] = (q, sc)
        else:
            ts[n] = torch.from_numpy(v).to(torch.float16)
    save_file(ts, os.path.join(tmp, "model.safetensors"))
    return q8


def test_int8_checkpoint_keeps_int8_and_scales(tmp_path):
    vals = _tensors(np.random.default_rng(7), True)
    q8 = _int8_checkpoint(str(tmp_path), vals)
    W = C.load_text_weights(str(tmp_path), SHAPES["layers"], device="cpu")
    for l in range(SHAPES["layers"]):
        for key, suffix in C._LAYER_TENSORS:
            n = f"model.language_model.layers.{l}.{suffix}"
            if key in C._LINEARS:
                q, sc = q8[n]
                assert W[(l, key)].dtype.__str__() == "torch.int8"
                assert np.array_equal(W[(l, key)].numpy(), q)
                assert np.array_equal(W[(l, key + "_scale")].numpy(), sc)
            else:
                assert W[(l, key)].numpy().dtype == np.float16


def test_int8_checkpoint_errors(tmp_path):
    vals = _tensors(np.random.default_rng(9), True)
    d1 = tmp_path / "noscale"
    d1.mkdir()
    _int8_checkpoint(str(d1), vals, skip_scale="model.language_model.layers.0.self_attn.k_proj.weight")
    with pytest.raises(C.CheckpointError, match="missing"):
        C.load_text_weights(str(d1), SHAPES["layers"], device="cpu")
    d2 = tmp_path / "mixed"
    d2.mkdir()
    _int8_checkpoint(str(d2), vals, float_linear="model.language_model.layers.1.mlp.up_proj.weight")
    with pytest.raises(C.CheckpointError, match="int8"):
        C.load_text_weights(str(d2), SHAPES["layers"], device="cpu")
