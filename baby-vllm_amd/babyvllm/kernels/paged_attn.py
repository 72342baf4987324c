"""Paged decode attention on the HIP kernel (drop-in for babyvllm/kernels/paged_attn.py:254-346).

``paged_decode_attention(q, kv_cache, block_tables, seq_lens, scale,
max_seq_len=None, partition_blocks=None)`` keeps the reference's signature:
one query token per sequence, GQA, pages read through the block table, and
the flash-decoding split chosen by ``decode_split_plan`` from the context
*bucket* (``max_seq_len``) and the batch's power-of-two bucket, never from the
live lengths, so the launch is identical on every replay of a captured graph.

The wrapper allocates the output and, for a split launch, the fp32 partial
scratch through torch (so both land in a graph's private pool under capture),
then makes one C-ABI call on the current stream: no host synchronisation and
no device-to-host read.
"""

from __future__ import annotations

import functools

import torch

from babyvllm.kernels import _lib
from babyvllm.kernels.decode_split import decode_split_plan


@functools.lru_cache(maxsize=None)
def _num_sms(device_index: int) -> int:
    return torch.cuda.get_device_properties(device_index).multi_processor_count


def _device_index(t: torch.Tensor) -> int:
    return t.device.index if t.device.index is not None else torch.cuda.current_device()


def paged_decode_attention(q, kv_cache, block_tables, seq_lens, scale,
                           max_seq_len=None, partition_blocks=None):
    """``[B, H, D]`` attention of one query token per row against its paged K/V.

    ``max_seq_len`` is the context bucket the step was sized for; it sets the
    split count. ``partition_blocks`` overrides BABYVLLM_DECODE_PARTITION.
    Rows with ``seq_len == 0`` return zeros.
    """
    for name, t in (("q", q), ("kv_cache", kv_cache), ("block_tables", block_tables),
                    ("seq_lens", seq_lens)):
        _lib.require_rocm_tensor(name, t)
    if q.dim() != 3 or q.stride(-1) != 1:
        raise ValueError("q must be [B, H, D] with a unit last stride")
    if q.dtype != torch.bfloat16 or kv_cache.dtype != torch.bfloat16:
        raise TypeError("q and kv_cache must be bfloat16")
    if block_tables.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise TypeError("block_tables and seq_lens must be int32")
    if kv_cache.dim() != 5 or kv_cache.shape[0] != 2:
        raise ValueError(f"kv_cache must be [2, NB, BS, Hkv, D], got {tuple(kv_cache.shape)}")
    B, n_heads, head_dim = q.shape
    _, num_blocks, block_size, n_kv_heads, cache_dim = kv_cache.shape
    if cache_dim != head_dim:
        raise ValueError("kv_cache head_dim differs from q")
    if block_tables.dim() != 2 or block_tables.shape[0] < B or block_tables.stride(1) != 1:
        raise ValueError("block_tables must be [B, W] with a unit last stride")
    if seq_lens.dim() != 1 or seq_lens.shape[0] < B or not seq_lens.is_contiguous():
        raise ValueError("seq_lens must be a contiguous [B] vector")
    k_cache, v_cache = kv_cache[0], kv_cache[1]
    if k_cache.stride() != v_cache.stride() or k_cache.stride(3) != 1:
        raise ValueError("K and V halves of kv_cache must share a layout with unit last stride")

    width = block_tables.shape[1]
    num_splits, blocks_per_split = decode_split_plan(
        B, n_kv_heads, block_size, width, max_seq_len, _num_sms(_device_index(q)), partition_blocks,
    )
    out = torch.empty(B, n_heads, head_dim, device=q.device, dtype=q.dtype)
    if B == 0:
        return out
    workspace = None
    nbytes = _lib.lib().bvllm_decode_workspace_bytes(B, n_heads, n_kv_heads, head_dim, num_splits,
                                                     blocks_per_split)
    if nbytes > 0:
        workspace = torch.empty(nbytes // 4, device=q.device, dtype=torch.float32)
    rc = _lib.lib().bvllm_paged_decode(
        q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        num_blocks,
        block_tables.data_ptr(), block_tables.stride(0), width,
        seq_lens.data_ptr(), float(scale),
        out.data_ptr(), out.stride(0), out.stride(1),
        None if workspace is None else workspace.data_ptr(), num_splits, blocks_per_split,
        B, n_heads, n_kv_heads, head_dim, block_size, 0,
        _lib.stream_handle(q.device),
    )
    _lib.check(rc, "bvllm_paged_decode")
    return out
