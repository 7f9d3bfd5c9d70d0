"""Qwen3-ASR checkpoints for the text decoder: config.json and safetensors.

Host-side mirror of the reference's loading path for the text decoder:

  * config.json (src/config.rs:141-195): the text decoder's hyper-parameters
    from `thinker_config.text_config` (legacy layout) or top-level
    `text_config` (transformers-native `-hf` layout), with `rope_parameters.
    rope_theta` overriding `rope_theta`, the MRoPE section defaulting to
    [24, 20, 20] and interleaving to true when `rope_scaling` is absent.
  * safetensors shards (src/weights.rs:150-218): `model.safetensors`, or every
    shard named by `model.safetensors.index.json`; HF-native names
    `model.language_model.*` are read as `thinker.model.*`.
  * per-layer tensors under `thinker.model.layers.{l}` (src/decoder.rs:
    4364-4417) and the f16 narrowing of bf16 / f32 tensors with
    round-to-nearest-even (src/weights.rs:58-79: bf16 -> f32 is exact, then
    f32 -> f16 RNE), done here on the device.

The decoder computes its logits against the tied embedding (cpu_decoder.rs:
458-471), so `embed_tokens` is also the lm_head.  Int8 checkpoints (the
reference's resident-int8 layout, weights.rs:296-427, decoder.rs:4352-4395)
keep their I8 [out][in] linears with the F32 [out] `<name>.weight_scale`
siblings; like the reference, the decoder's linears are int8 all together or
not at all.

`load_text_weights` returns the weight dictionary `qasr_attn.TextDecoder`
takes; `open_text_decoder` builds the decoder from a model directory.
"""
from __future__ import annotations

import json
import os
from typing import Dict, Optional

TEXT_DEFAULTS = dict(vocab_size=151936, hidden_size=1024, intermediate_size=3072,
                     num_hidden_layers=28, num_attention_heads=16, num_key_value_heads=8,
                     head_dim=128, rms_norm_eps=1e-6, rope_theta=1e6)
DEFAULT_MROPE_SECTION = (24, 20, 20)
TEXT_PREFIX = "thinker.model"

INT8_SCALE_SUFFIX = ".weight_scale"
_LINEARS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

# (name in the weight dictionary, tensor under thinker.model.layers.{l})
_LAYER_TENSORS = (
    ("input_layernorm", "input_layernorm.weight"),
    ("post_attention_layernorm", "post_attention_layernorm.weight"),
    ("q_norm", "self_attn.q_norm.weight"),
    ("k_norm", "self_attn.k_norm.weight"),
    ("q_proj", "self_attn.q_proj.weight"),
    ("k_proj", "self_attn.k_proj.weight"),
    ("v_proj", "self_attn.v_proj.weight"),
    ("o_proj", "self_attn.o_proj.weight"),
    ("gate_proj", "mlp.gate_proj.weight"),
    ("up_proj", "mlp.up_proj.weight"),
    ("down_proj", "mlp.down_proj.weight"),
)


class CheckpointError(ValueError):
    pass


def parse_text_config(cfg: dict) -> dict:
    """The text decoder's hyper-parameters from a parsed config.json
    (AsrConfig::from_json_str + TextDecoderConfig::mrope_*, config.rs:148-195)."""
    if cfg.get("thinker_config") is not None:
        text = cfg["thinker_config"].get("text_config")
    else:
        text = cfg.get("text_config")
    if text is None:
        raise CheckpointError("config.json has neither thinker_config.text_config nor text_config")
    out = {k: type(v)(text.get(k, v)) for k, v in TEXT_DEFAULTS.items()}
    rp = text.get("rope_parameters") or {}
    if rp.get("rope_theta") is not None:
        out["rope_theta"] = float(rp["rope_theta"])
    rs = text.get("rope_scaling")
    if rs is None:
        out["mrope_section"] = list(DEFAULT_MROPE_SECTION)
        out["mrope_interleaved"] = True
    else:
        out["mrope_section"] = list(rs.get("mrope_section", DEFAULT_MROPE_SECTION))
        out["mrope_interleaved"] = bool(rs.get("mrope_interleaved", False) or rs.get("interleaved", False))
    return out


def read_text_config(model_dir: str) -> dict:
    with open(os.path.join(model_dir, "config.json")) as f:
        return parse_text_config(json.load(f))


def remap_name(name: str) -> str:
    """HF-native tensor names of the text decoder (weights.rs:172-186)."""
    if name.startswith("model.language_model."):
        return TEXT_PREFIX + "." + name[len("model.language_model."):]
    return name


def _shards(model_dir: str):
    index = os.path.join(model_dir, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            wm = json.load(f).get("weight_map")
        if not isinstance(wm, dict):
            raise CheckpointError("invalid model.safetensors.index.json")
        return [os.path.join(model_dir, s) for s in sorted(set(wm.values()))]
    return [os.path.join(model_dir, "model.safetensors")]


def _to_f16(t, device):
    """bf16 / f32 / f16 tensor -> f16 on `device`: RNE narrowing (bf16 -> f32
    is exact, so narrowing bf16 via f32 equals the reference's)."""
    import torch

    if t.dtype == torch.float16:
        return t.to(device)
    if t.dtype in (torch.bfloat16, torch.float32):
        return t.to(device).float().half()
    raise CheckpointError(f"unsupported dtype {t.dtype} for a floating-point weight")


def load_text_weights(model_dir: str, num_layers: Optional[int] = None,
                      device: str = "cuda") -> Dict:
    """Text-decoder tensors of a checkpoint directory on `device`, keyed
    "embed", "norm" and (layer, name): f16, except int8 linears (torch.int8)
    with their f32 scales under (layer, name + "_scale")."""
    import torch
    from safetensors import safe_open

    if num_layers is None:
        num_layers = read_text_config(model_dir)["num_hidden_layers"]
    wanted = {f"{TEXT_PREFIX}.embed_tokens.weight": "embed", f"{TEXT_PREFIX}.norm.weight": "norm"}
    for l in range(num_layers):
        for key, suffix in _LAYER_TENSORS:
            wanted[f"{TEXT_PREFIX}.layers.{l}.{suffix}"] = (l, key)
            if key in _LINEARS:
                scale = suffix[:-len(".weight")] + INT8_SCALE_SUFFIX
                wanted[f"{TEXT_PREFIX}.layers.{l}.{scale}"] = (l, key + "_scale")
    raw = {}
    for path in _shards(model_dir):
        with safe_open(path, framework="pt") as f:
            for name in f.keys():
                dst = wanted.get(remap_name(name))
                if dst is not None:
                    raw[dst] = f.get_tensor(name)
    linears = [(l, k) for l in range(num_layers) for k in _LINEARS]
    int8 = [k for k in linears if k in raw and raw[k].dtype == torch.int8]
    if int8 and len(int8) != len([k for k in linears if k in raw]):
        raise CheckpointError(f"{int8[0]} is int8 in an otherwise floating-point checkpoint; "
                              "quantise every decoder linear or none")
    out = {}
    for key, t in raw.items():
        if isinstance(key, tuple) and key[1].endswith("_scale"):
            if int8:
                out[key] = t.to(device).float().contiguous()
        elif t.dtype == torch.int8:
            out[key] = t.to(device).contiguous()
        else:
            out[key] = _to_f16(t, device)
    need = [n for n, k in wanted.items()
            if not (isinstance(k, tuple) and k[1].endswith("_scale")) or int8]
    missing = [n for n in need if wanted[n] not in out]
    if missing:
        raise CheckpointError(f"{len(missing)} text-decoder tensors missing, e.g. {missing[0]}")
    return out


def open_text_decoder(model_dir: str, slots: int = 1, max_rows: int = 512, cap: int = 1024,
                      max_seq: int = 16384, device: int = 0):
    """A `qasr_attn.TextDecoder` over a checkpoint directory."""
    import qasr_attn

    cfg = read_text_config(model_dir)
    W = load_text_weights(model_dir, cfg["num_hidden_layers"], device=f"cuda:{device}")
    return qasr_attn.TextDecoder(
        W, cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"],
        cfg["num_hidden_layers"], cfg["rms_norm_eps"], max_seq, slots=slots, max_rows=max_rows,
        cap=cap, device=device, rope_theta=cfg["rope_theta"],
        mrope_section=cfg["mrope_section"], mrope_interleaved=cfg["mrope_interleaved"])
