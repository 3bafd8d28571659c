"""Run configuration (the reference's Config fields, config.py:6-29) and model shapes.

The reference reads the model's HF config with AutoConfig from a local
directory.  Here `model` may be such a directory (its config.json is read as
JSON; Qwen2.5-VL configs with a nested text_config are flattened), a dict of
config values, or an object with the attributes; no network access is needed.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field
from types import SimpleNamespace

import torch

# Public Qwen2.5-VL vision_config (both sizes; out_hidden_size is the text hidden size).
QWEN25_VL_VISION = dict(depth=32, hidden_size=1280, intermediate_size=3420, num_heads=16, in_channels=3,
                        patch_size=14, temporal_patch_size=2, spatial_merge_size=2, window_size=112,
                        fullatt_block_indexes=[7, 15, 23, 31], hidden_act="silu", tokens_per_second=2)
# Public Qwen2.5-VL-3B-Instruct shapes.
QWEN25_VL_3B = dict(
    architectures=["Qwen2_5_VLForConditionalGeneration"],
    hidden_size=2048, intermediate_size=11008, num_hidden_layers=36, num_attention_heads=16,
    num_key_value_heads=2, vocab_size=151936, rms_norm_eps=1e-6, rope_theta=1e6,
    rope_scaling={"type": "mrope", "mrope_section": [16, 24, 24]}, max_position_embeddings=128000,
    tie_word_embeddings=True, image_token_id=151655, vision_start_token_id=151652, eos_token_id=151645,
    spatial_merge_size=2, torch_dtype="bfloat16",
    vision_config=dict(QWEN25_VL_VISION, out_hidden_size=2048),
)
# Public Qwen2.5-VL-7B-Instruct shapes.
QWEN25_VL_7B = dict(QWEN25_VL_3B, hidden_size=3584, intermediate_size=18944, num_hidden_layers=28,
                    num_attention_heads=28, num_key_value_heads=4, vocab_size=152064, tie_word_embeddings=False,
                    vision_config=dict(QWEN25_VL_VISION, out_hidden_size=3584))

_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def load_model_config(model) -> SimpleNamespace:
    if isinstance(model, (str, os.PathLike)):
        with open(os.path.join(model, "config.json")) as f:
            d = json.load(f)
    elif isinstance(model, dict):
        d = dict(model)
    else:
        d = dict(vars(model))
    text = d.pop("text_config", None)
    if isinstance(text, dict):
        d = {**d, **text}
    vision = d.get("vision_config") or {}
    d.setdefault("spatial_merge_size", vision.get("spatial_merge_size", 2) if isinstance(vision, dict) else 2)
    d.setdefault("image_token_id", 151655)
    d.setdefault("rope_theta", (d.get("rope_parameters") or {}).get("rope_theta", 1e6))
    d.setdefault("tie_word_embeddings", False)
    d.setdefault("rms_norm_eps", 1e-6)
    d.setdefault("head_dim", d["hidden_size"] // d["num_attention_heads"])
    dt = d.get("torch_dtype") or d.get("dtype") or "bfloat16"
    d["torch_dtype"] = _DTYPES.get(str(dt).replace("torch.", ""), torch.bfloat16)
    return SimpleNamespace(**d)


@dataclass
class Config:
    model: object
    max_num_batched_tokens: int = 16384
    max_num_seqs: int = 512
    max_model_len: int = 4096
    gpu_memory_utilization: float = 0.9
    tensor_parallel_size: int = 1
    enforce_eager: bool = False
    hf_config: SimpleNamespace | None = None
    eos: int = -1
    kvcache_block_size: int = 256
    num_kvcache_blocks: int = -1
    encoder_cache_ratio: float = 0.2
    recompute_ratio: float = 0.0
    # Additions of this build (not in the reference):
    use_mrope: bool = True      # M-RoPE positions when the model config has mrope_section
    rerotate_reused_kv: bool = True  # re-rotate reused image K to its new position
    seed: int = 0               # weights of a model directory without checkpoint files
    synthetic_vision: bool = False  # encoder-cache miss without image_embeds: seeded synthetic embeddings
    extra: dict = field(default_factory=dict)

    def __post_init__(self):
        assert self.kvcache_block_size % 256 == 0
        assert self.tensor_parallel_size == 1, "this build runs on one GPU (tensor_parallel_size=1)"
        assert 0.0 <= self.recompute_ratio <= 1.0
        self.hf_config = load_model_config(self.model)
        self.max_model_len = min(self.max_model_len, self.hf_config.max_position_embeddings)
        assert self.max_num_batched_tokens >= self.max_model_len
        if not self.use_mrope or not (getattr(self.hf_config, "rope_scaling", None) or {}).get("mrope_section"):
            self.use_mrope = False
            self.hf_config.rope_scaling = None
        if self.eos == -1:
            eos = getattr(self.hf_config, "eos_token_id", -1)
            self.eos = eos[0] if isinstance(eos, list) else eos
