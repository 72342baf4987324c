"""Attention metadata handed from the runner to the attention layer (babyvllm/worker/context.py:5-35).

Same fields and meaning as the reference: ``slot_mapping`` int64 ``[T]``,
``block_tables`` int32 ``[S, W]``, ``query_start_loc`` int32 ``[S+1]``,
``seq_lens`` / ``context_lens`` int32 ``[S]``, their host-side lists, and the
host ints ``max_query_len`` (1 for a pure decode step) and ``max_seq_len``
(the context bucket under a captured graph).
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass

import torch


@dataclass
class AttentionMetadata:
    slot_mapping: torch.Tensor
    block_tables: torch.Tensor
    query_start_loc: torch.Tensor
    seq_lens: torch.Tensor
    context_lens: torch.Tensor
    query_start_loc_cpu: list[int]
    seq_lens_cpu: list[int]
    context_lens_cpu: list[int]
    max_query_len: int
    max_seq_len: int


@dataclass
class ForwardContext:
    attn_metadata: AttentionMetadata


_FORWARD_CTX: ForwardContext | None = None


@contextmanager
def set_forward_context(attn_metadata: AttentionMetadata):
    """Make ``attn_metadata`` visible to every Attention layer inside the block."""
    global _FORWARD_CTX
    saved = _FORWARD_CTX
    _FORWARD_CTX = ForwardContext(attn_metadata)
    try:
        yield
    finally:
        _FORWARD_CTX = saved


def get_forward_context() -> ForwardContext | None:
    return _FORWARD_CTX
