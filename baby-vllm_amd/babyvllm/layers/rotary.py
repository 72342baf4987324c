"""RoPE cos/sin tables, the inputs of the fused RoPE + append kernel (babyvllm/layers/rotary.py:17-32).

``RotaryEmbedding(dim, max_position_embeddings, base)`` builds fp32 tables with
duplicated halves (``inv_freq = base^(-2i/dim)``, angle = position · inv_freq)
and ``forward(positions, dtype)`` gathers one row per token and casts it to the
model dtype, exactly the tensors the reference's model passes to
``fused_rope_and_cache``.
"""

from __future__ import annotations

import torch
import torch.nn as nn


class RotaryEmbedding(nn.Module):
    def __init__(self, dim: int, max_position_embeddings: int = 2048, base: float = 10000):
        super().__init__()
        half = torch.arange(0, dim, 2).float() / dim
        inv_freq = 1.0 / (base ** half)
        self.register_buffer("inv_freq", inv_freq, persistent=False)
        self.max_seq_len_cached = max_position_embeddings
        angles = torch.outer(torch.arange(max_position_embeddings, dtype=torch.float32), inv_freq)
        table = torch.cat((angles, angles), dim=-1)
        self.register_buffer("cos_cached", table.cos()[None, None], persistent=False)
        self.register_buffer("sin_cached", table.sin()[None, None], persistent=False)

    def forward(self, positions: torch.Tensor, dtype: torch.dtype):
        return (self.cos_cached[0, 0, positions].to(dtype),
                self.sin_cached[0, 0, positions].to(dtype))
