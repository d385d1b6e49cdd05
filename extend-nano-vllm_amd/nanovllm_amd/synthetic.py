"""Config-only checkpoints for random-weight runs.

There is no network for real checkpoints, so benchmarks and tests write a
Qwen3 ``config.json`` (and an EAGLE3 speculators-format draft config) into
local directories and start the engine with ``load_format="dummy"``.  The
geometries are the ones the reference's benchmarks target (Qwen3-0.6B / 8B /
32B) plus a tiny one for tests.
"""
from __future__ import annotations

import json
import os

QWEN3_PRESETS = {
    "tiny": dict(hidden_size=256, num_hidden_layers=4, num_attention_heads=4,
                 num_key_value_heads=2, head_dim=128, intermediate_size=512, vocab_size=2048,
                 max_position_embeddings=4096, tie_word_embeddings=False),
    "qwen3-0.6b": dict(hidden_size=1024, num_hidden_layers=28, num_attention_heads=16,
                       num_key_value_heads=8, head_dim=128, intermediate_size=3072,
                       vocab_size=151936, max_position_embeddings=40960,
                       tie_word_embeddings=True),
    "qwen3-8b": dict(hidden_size=4096, num_hidden_layers=36, num_attention_heads=32,
                     num_key_value_heads=8, head_dim=128, intermediate_size=12288,
                     vocab_size=151936, max_position_embeddings=40960,
                     tie_word_embeddings=False),
    "qwen3-32b": dict(hidden_size=5120, num_hidden_layers=64, num_attention_heads=64,
                      num_key_value_heads=8, head_dim=128, intermediate_size=25600,
                      vocab_size=151936, max_position_embeddings=40960,
                      tie_word_embeddings=False),
}


def write_qwen3_config(path: str, preset: str = "tiny", **overrides) -> str:
    """Write a Qwen3 config.json (bf16, RMSNorm eps 1e-6, RoPE theta 1e6)."""
    from transformers import Qwen3Config

    params = dict(QWEN3_PRESETS[preset])
    params.update(overrides)
    cfg = Qwen3Config(rms_norm_eps=1e-6, rope_theta=1000000.0, attention_bias=False,
                      hidden_act="silu", torch_dtype="bfloat16", **params)
    os.makedirs(path, exist_ok=True)
    cfg.save_pretrained(path)
    return path


def write_eagle3_config(path: str, target_preset: str = "tiny",
                        aux_layers: tuple[int, ...] | None = None, **overrides) -> str:
    """Write a speculators-format EAGLE3 config.json for a draft that matches
    the target preset: one Llama layer of the target's width, draft vocab =
    target vocab (d2t all zero)."""
    t = dict(QWEN3_PRESETS[target_preset])
    layer = dict(model_type="llama", hidden_size=t["hidden_size"],
                 intermediate_size=t["intermediate_size"],
                 num_attention_heads=t["num_attention_heads"],
                 num_key_value_heads=t["num_key_value_heads"], head_dim=t["head_dim"],
                 max_position_embeddings=t["max_position_embeddings"], rms_norm_eps=1e-6,
                 rope_theta=1000000.0, attention_bias=False, vocab_size=t["vocab_size"])
    layer.update(overrides)
    if aux_layers is None:
        aux_layers = default_aux_layers(target_preset)
    raw = {
        "speculators_model_type": "eagle3",
        "transformer_layer_config": layer,
        "draft_vocab_size": t["vocab_size"],
        "target_hidden_size": t["hidden_size"],
        "eagle_aux_hidden_state_layer_ids": list(aux_layers),
        "norm_before_residual": True,
        "torch_dtype": "bfloat16",
    }
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(raw, f, indent=2)
    return path


def default_aux_layers(target_preset: str) -> tuple[int, ...]:
    """Aux layer ids used with a preset: the reference default (2, 18, 33) for
    36-layer models, otherwise early / middle / late layers."""
    n = QWEN3_PRESETS[target_preset]["num_hidden_layers"]
    if n == 36:
        return (2, 18, 33)
    return (2, n // 2, n - 3) if n >= 6 else (1, 2, n)
