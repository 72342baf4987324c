"""Greedy sampling on the HIP kernel (drop-in for babyvllm/kernels/argmax.py:41-56).

``greedy_argmax(logits, out, block=4096)`` keeps the reference's signature and
semantics: ``out[i] = argmax(logits[i])`` for a (rows, vocab) matrix with unit
column stride, ties to the lowest index (torch.argmax's order), written into
``out`` (int64, possibly a slice of a larger buffer) and returned. ``block`` is
the reference's chunk width; the HIP kernel chooses its own and ignores it.
No host sync, so the call can sit inside a captured decode graph.
"""

from __future__ import annotations

import torch

from babyvllm.kernels import _lib


def greedy_argmax(logits: torch.Tensor, out: torch.Tensor, block: int = 4096) -> torch.Tensor:
    """out[i] = argmax(logits[i]). logits is (rows, vocab) with unit column stride."""
    assert logits.dim() == 2 and logits.stride(1) == 1, "logits must be (rows, vocab), contiguous rows"
    del block
    _lib.require_rocm_tensor("logits", logits)
    _lib.require_rocm_tensor("out", out)
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"logits must be bfloat16 or float32, got {logits.dtype}")
    if out.dtype != torch.int64 or out.dim() != 1 or out.stride(0) != 1:
        raise TypeError("out must be a contiguous int64 vector")
    rows, vocab = logits.shape
    if out.shape[0] < rows:
        raise ValueError(f"out holds {out.shape[0]} rows, logits has {rows}")
    if rows == 0:
        return out
    h = _lib.lib()
    ws = torch.empty(h.bvllm_argmax_workspace_bytes(rows, vocab) // 4, device=logits.device, dtype=torch.int32)
    rc = h.bvllm_greedy_argmax(logits.data_ptr(), logits.stride(0), rows, vocab,
                               1 if logits.dtype == torch.float32 else 0, ws.data_ptr(), out.data_ptr(),
                               _lib.stream_handle(logits.device))
    _lib.check(rc, "bvllm_greedy_argmax")
    return out
