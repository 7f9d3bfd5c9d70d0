"""Writes reference_known_answers.json: the known answers the reference's own
unit tests hold for this path, transcribed as data (no reference code runs).

Sources (paths relative to the reference checkout):
  src/mrope.rs:86-107   build_dim_map / compute_mrope_cos_sin tests
  src/config.rs:102-110 text-decoder defaults (vocab, heads, head_dim, eps, theta)
  src/config.rs:177-195 mrope_section default [24, 20, 20], interleaved default true
  src/config.rs:261-290 HF-native config layout test (text_config values)
  src/config.rs:212-258, 331-341 mrope_section / mrope_interleaved from rope_scaling
  src/weights.rs:588-625 int8 dequantisation tests (f16(q * scale) per row)

The reference ships no numeric vectors for attention itself (its numeric gate
is transcript identity on audio fixtures kept outside the repository), so
these are the only reference-held answers on this path.

Usage: python tests/golden/make_reference_known_answers.py
"""
import json
import os

KNOWN = {
    "build_dim_map": [
        {"source": "src/mrope.rs:87-94", "section": [24, 20, 20], "half": 64, "interleaved": True,
         "len": 64, "counts": {"0": 24, "1": 20, "2": 20}, "prefix": [0, 1, 2, 0, 1, 2]},
        {"source": "src/mrope.rs:96-100", "section": [2, 1], "half": 4, "interleaved": False,
         "map": [0, 0, 1, 1]},
    ],
    "compute_mrope_cos_sin": [
        {"source": "src/mrope.rs:102-106", "text_positions": 3, "head_dim": 8, "theta": 1e6,
         "section": [2, 1, 1], "interleaved": True, "cos_len": 24, "halves_equal": [[0, 4], [4, 8]]},
    ],
    "text_decoder_defaults": {
        "source": "src/config.rs:102-110, 177-195",
        "vocab_size": 151936, "hidden_size": 1024, "intermediate_size": 3072,
        "num_hidden_layers": 28, "num_attention_heads": 16, "num_key_value_heads": 8,
        "head_dim": 128, "rms_norm_eps": 1e-6, "rope_theta": 1e6,
        "mrope_section": [24, 20, 20], "mrope_interleaved": True,
    },
    "hf_native_text_config": {
        "source": "src/config.rs:261-290",
        "num_attention_heads": 16, "num_key_value_heads": 8, "head_dim": 128,
        "rms_norm_eps": 1e-6, "rope_theta": 1000000, "num_hidden_layers": 28, "hidden_size": 1024,
    },
    # config.json inputs and the text-decoder values the reference derives from
    # them: the HF-native test's own JSON, and the rope_scaling cases of the
    # mrope tests written as the text_config JSON their structs stand for.
    "config_parsing": [
        {"source": "src/config.rs:262-290",
         "json": {"audio_config": {"d_model": 896, "encoder_layers": 18, "encoder_attention_heads": 14,
                                   "encoder_ffn_dim": 3584, "num_mel_bins": 128, "n_window": 50,
                                   "n_window_infer": 800, "conv_chunksize": 500, "output_dim": 1024},
                  "audio_token_id": 151676,
                  "text_config": {"vocab_size": 151936, "hidden_size": 1024, "intermediate_size": 3072,
                                  "num_hidden_layers": 28, "num_attention_heads": 16,
                                  "num_key_value_heads": 8, "head_dim": 128, "rms_norm_eps": 1e-6,
                                  "rope_parameters": {"rope_theta": 1000000, "rope_type": "default"}}},
         "expect": {"hidden_size": 1024, "num_hidden_layers": 28, "rope_theta": 1e6,
                    "mrope_section": [24, 20, 20], "mrope_interleaved": True}},
        {"source": "src/config.rs:212-216, 230-234 (no rope_scaling)",
         "json": {"thinker_config": {"audio_config": {}, "text_config": {}}},
         "expect": {"vocab_size": 151936, "hidden_size": 1024, "intermediate_size": 3072,
                    "rope_theta": 1e6, "mrope_section": [24, 20, 20], "mrope_interleaved": True}},
        {"source": "src/config.rs:218-228",
         "json": {"thinker_config": {"audio_config": {}, "text_config": {
             "rope_scaling": {"rope_type": "mrope", "mrope_section": [4, 4, 8],
                              "interleaved": False, "mrope_interleaved": False}}}},
         "expect": {"mrope_section": [4, 4, 8], "mrope_interleaved": False}},
        {"source": "src/config.rs:236-246",
         "json": {"thinker_config": {"audio_config": {}, "text_config": {
             "rope_scaling": {"rope_type": "mrope", "mrope_section": [24, 20, 20],
                              "interleaved": False, "mrope_interleaved": True}}}},
         "expect": {"mrope_section": [24, 20, 20], "mrope_interleaved": True}},
        {"source": "src/config.rs:248-258",
         "json": {"thinker_config": {"audio_config": {}, "text_config": {
             "rope_scaling": {"rope_type": "mrope", "mrope_section": [24, 20, 20],
                              "interleaved": True, "mrope_interleaved": False}}}},
         "expect": {"mrope_interleaved": True}},
        {"source": "src/config.rs:331-341",
         "json": {"thinker_config": {"audio_config": {}, "text_config": {
             "rope_scaling": {"rope_type": "mrope", "mrope_section": [24, 20, 20],
                              "interleaved": False, "mrope_interleaved": False}}}},
         "expect": {"mrope_interleaved": False}},
    ],
    # int8 [rows][cols] with f32 row scales -> the f16 values the reference's
    # get_f16 / get_matrix return for them.
    "int8_dequant": [
        {"source": "src/weights.rs:588-603", "rows": 2, "cols": 2, "q": [4, -8, -2, 3],
         "scale": [0.25, -0.5], "expect": [1.0, -2.0, 1.0, -1.5]},
        {"source": "src/weights.rs:613-625 (asserts row 0; row 1 by the same rule)", "rows": 2, "cols": 2, "q": [127, 0, 0, 127],
         "scale": [1.0, 2.0], "expect": [127.0, 0.0, 0.0, 254.0]},
    ],
}

if __name__ == "__main__":
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_known_answers.json")
    with open(out, "w") as f:
        json.dump(KNOWN, f, indent=1)
        f.write("\n")
    print(f"wrote {out}")
