"""Qwen3 hyper-parameters (reference: qwen3/config.py:24-73), read from a
local config.json only (there is no hub access)."""
from __future__ import annotations

import json
import os
from dataclasses import dataclass

__all__ = ["Qwen3Config", "qwen3_0p6b_config"]


@dataclass
class Qwen3Config:
    hidden_size: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    num_hidden_layers: int
    vocab_size: int
    intermediate_size: int
    rms_norm_eps: float
    rope_theta: float
    max_position_embeddings: int = 4096
    tie_word_embeddings: bool = False

    @classmethod
    def from_pretrained(cls, model_path: str) -> "Qwen3Config":
        """Reads <model_path>/config.json (the HF layout, as the reference)."""
        with open(os.path.join(model_path, "config.json")) as f:
            d = json.load(f)
        return cls(
            hidden_size=d["hidden_size"],
            num_attention_heads=d["num_attention_heads"],
            num_key_value_heads=d["num_key_value_heads"],
            head_dim=d.get("head_dim", d["hidden_size"] // d["num_attention_heads"]),
            num_hidden_layers=d["num_hidden_layers"],
            vocab_size=d["vocab_size"],
            intermediate_size=d["intermediate_size"],
            rms_norm_eps=d["rms_norm_eps"],
            rope_theta=d["rope_theta"],
            max_position_embeddings=d.get("max_position_embeddings", 4096),
            tie_word_embeddings=d.get("tie_word_embeddings", False),
        )


def qwen3_0p6b_config(max_position_embeddings: int = 40960) -> Qwen3Config:
    """Qwen3-0.6B: 28 layers, hidden 1024, 16 q / 8 KV heads of 128, SwiGLU
    3072, vocab 151936, tied embeddings, QK-Norm, RoPE theta 1e6."""
    return Qwen3Config(hidden_size=1024, num_attention_heads=16, num_key_value_heads=8,
                       head_dim=128, num_hidden_layers=28, vocab_size=151936,
                       intermediate_size=3072, rms_norm_eps=1e-6, rope_theta=1e6,
                       max_position_embeddings=max_position_embeddings,
                       tie_word_embeddings=True)
