"""Model, cache and scheduler configuration (babyvllm/config.py:12-78).

``ModelConfig`` carries the Qwen2 architecture fields the reference reads from
a checkpoint's config.json. There is no network here, so besides
``from_hf(path)`` (a local directory) the two shapes the benchmarks use are
available as presets: ``qwen2_5_7b()`` and ``qwen2_5_0_5b()``.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass


@dataclass
class ModelConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    rms_norm_eps: float
    max_position_embeddings: int
    rope_theta: float
    tie_word_embeddings: bool
    block_size: int = 16

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def kv_bytes_per_token(self) -> int:
        """K and V of every layer for one token, bf16."""
        return 2 * self.num_hidden_layers * self.num_key_value_heads * self.head_dim * 2

    @classmethod
    def from_hf(cls, path: str, block_size: int = 16) -> "ModelConfig":
        with open(os.path.join(path, "config.json")) as f:
            c = json.load(f)
        if c.get("architectures") != ["Qwen2ForCausalLM"]:
            raise ValueError(f"not a Qwen2ForCausalLM checkpoint: {c.get('architectures')}")
        if c["hidden_size"] % c["num_attention_heads"]:
            raise ValueError("hidden_size must be a multiple of num_attention_heads")
        return cls(
            vocab_size=c["vocab_size"], hidden_size=c["hidden_size"],
            intermediate_size=c["intermediate_size"], num_hidden_layers=c["num_hidden_layers"],
            num_attention_heads=c["num_attention_heads"], num_key_value_heads=c["num_key_value_heads"],
            rms_norm_eps=c["rms_norm_eps"], max_position_embeddings=c["max_position_embeddings"],
            rope_theta=c["rope_theta"], tie_word_embeddings=c.get("tie_word_embeddings", False),
            block_size=block_size,
        )


def qwen2_5_7b(block_size: int = 16) -> ModelConfig:
    """Qwen2.5-7B architecture (28 layers, hidden 3584, 28 / 4 heads, vocab 152,064)."""
    return ModelConfig(vocab_size=152064, hidden_size=3584, intermediate_size=18944, num_hidden_layers=28,
                       num_attention_heads=28, num_key_value_heads=4, rms_norm_eps=1e-6,
                       max_position_embeddings=32768, rope_theta=1e6, tie_word_embeddings=False,
                       block_size=block_size)


def qwen2_5_0_5b(block_size: int = 16) -> ModelConfig:
    """Qwen2.5-0.5B architecture (24 layers, hidden 896, 14 / 2 heads, tied embeddings)."""
    return ModelConfig(vocab_size=151936, hidden_size=896, intermediate_size=4864, num_hidden_layers=24,
                       num_attention_heads=14, num_key_value_heads=2, rms_norm_eps=1e-6,
                       max_position_embeddings=32768, rope_theta=1e6, tie_word_embeddings=True,
                       block_size=block_size)


@dataclass
class CacheConfig:
    block_size: int = 16
    # Pages in the GPU pool; None sizes the pool from free memory.
    num_gpu_blocks: int | None = None
    enable_prefix_caching: bool = False
    # Fraction of free device memory the pool may take when sized automatically.
    gpu_memory_fraction: float = 0.5


@dataclass
class SchedulerConfig:
    max_num_seqs: int = 256
    max_num_batched_tokens: int = 2048
