"""Paged attention layer: routes a step to the decode or the prefill HIP kernel.

Mirrors ``Attention`` of babyvllm/layers/attention.py:35-68: with a forward
context and a cache, a step whose ``max_query_len == 1`` runs
``paged_decode_attention`` (with ``max_seq_len`` = the step's context bucket),
any longer step runs ``paged_prefill_attention``. This build has no torch
attention path: a call on a non-ROCm tensor, without a KV cache or without a
forward context raises instead of silently computing elsewhere.

``BABYVLLM_PREFILL_ATTN`` is the reference's switch for multi-token steps
(babyvllm/layers/attention.py:10-12,58): ``"triton"`` (its default, the paged
prefill kernel; here the HIP kernel) or ``"hip"`` selects the kernel; the
reference's ``"torch"`` (its per-sequence SDPA loop) is not part of this build
and raises when a multi-token step reaches it.
"""

from __future__ import annotations

import os

import torch.nn as nn

from babyvllm.worker.context import get_forward_context

_PREFILL_BACKEND = os.environ.get("BABYVLLM_PREFILL_ATTN", "triton")


class Attention(nn.Module):
    """Paged attention over a flattened (varlen) token batch."""

    def __init__(self, num_heads: int, head_dim: int, num_kv_heads: int,
                 scale: float | None = None):
        super().__init__()
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.num_queries_per_kv = num_heads // num_kv_heads
        self.scale = scale if scale is not None else head_dim ** -0.5
        self.kv_cache = None

    def forward(self, q, k, v):
        ctx = get_forward_context()
        if self.kv_cache is None or ctx is None:
            raise RuntimeError(
                "Attention needs a KV cache and a forward context: the cache-less path "
                "(memory-sizing forward) is outside this build's hot path")
        if not q.is_cuda:
            raise RuntimeError(f"Attention runs only on a ROCm device, got {q.device}")
        md = ctx.attn_metadata
        if md.max_query_len == 1 and self.kv_cache.shape[2] >= 16:
            from babyvllm.kernels.paged_attn import paged_decode_attention
            return paged_decode_attention(q, self.kv_cache, md.block_tables, md.seq_lens,
                                          self.scale, max_seq_len=md.max_seq_len)
        if _PREFILL_BACKEND not in ("triton", "hip"):
            raise RuntimeError(
                f"BABYVLLM_PREFILL_ATTN={_PREFILL_BACKEND!r}: this build runs multi-token steps only on its "
                "HIP paged prefill kernel ('triton' or 'hip'); the reference's torch SDPA loop is not shipped")
        from babyvllm.kernels.paged_prefill import paged_prefill_attention
        return paged_prefill_attention(q, self.kv_cache, md, self.scale)
