"""Varlen paged prefill attention on the HIP kernel (drop-in for babyvllm/kernels/paged_prefill.py:104-146).

``paged_prefill_attention(q, kv_cache, md, scale)`` keeps the reference's
signature and semantics: a flattened batch of sequences, each with
``context_lens[s]`` cached tokens plus ``q_len`` new query rows, causal, GQA,
with K/V (prefix and new tokens alike) read from the paged cache through
``md.block_tables``. Decode rows (query length 1) may be mixed into the step.
"""

from __future__ import annotations

import torch

from babyvllm.kernels import _lib


def _single_query_seqs(md, num_seqs):
    """Sequences with exactly one query token, from the host copy of query_start_loc.

    -1 (unknown) when the metadata carries no host copy of the right length;
    the library then checks every sequence on the device.
    """
    qsl = getattr(md, "query_start_loc_cpu", None)
    if qsl is None or len(qsl) != num_seqs + 1:
        return -1
    return sum(1 for i in range(num_seqs) if qsl[i + 1] - qsl[i] == 1)


def paged_prefill_attention(q, kv_cache, md, scale):
    """Causal attention for a flattened varlen batch, reading K/V from the paged cache.

    K/V of the step's tokens must already be in the cache (the RoPE + append
    kernel writes them first).
    """
    num_tokens, num_heads, head_dim = q.shape
    num_kv_heads = kv_cache.shape[3]
    page = kv_cache.shape[2]
    assert head_dim & (head_dim - 1) == 0, f"head_dim {head_dim} must be a power of two"
    assert num_heads % num_kv_heads == 0

    for name, t in (("q", q), ("kv_cache", kv_cache), ("block_tables", md.block_tables),
                    ("query_start_loc", md.query_start_loc), ("seq_lens", md.seq_lens),
                    ("context_lens", md.context_lens)):
        _lib.require_rocm_tensor(name, t)
    if q.dtype != torch.bfloat16 or kv_cache.dtype != torch.bfloat16:
        raise TypeError("q and kv_cache must be bfloat16")
    if q.stride(-1) != 1:
        raise ValueError("q must have a unit last stride")
    for name, t in (("block_tables", md.block_tables), ("query_start_loc", md.query_start_loc),
                    ("seq_lens", md.seq_lens), ("context_lens", md.context_lens)):
        if t.dtype != torch.int32:
            raise TypeError(f"{name} must be int32, got {t.dtype}")
    bt = md.block_tables
    if bt.dim() != 2 or bt.stride(1) != 1:
        raise ValueError("block_tables must be [S, W] with a unit last stride")
    qsl = md.query_start_loc.contiguous()
    seq_lens = md.seq_lens.contiguous()
    ctx_lens = md.context_lens.contiguous()

    out = torch.empty(num_tokens, num_heads, head_dim, device=q.device, dtype=q.dtype)
    if num_tokens == 0:
        return out
    k_cache, v_cache = kv_cache[0], kv_cache[1]
    if k_cache.stride() != v_cache.stride() or k_cache.stride(3) != 1:
        raise ValueError("K and V halves of kv_cache must share a layout with unit last stride")
    num_seqs = seq_lens.shape[0]
    rc = _lib.lib().bvllm_paged_prefill(
        q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        kv_cache.shape[1],
        bt.data_ptr(), bt.stride(0), bt.shape[1],
        qsl.data_ptr(), seq_lens.data_ptr(), ctx_lens.data_ptr(), float(scale),
        out.data_ptr(), out.stride(0), out.stride(1),
        num_seqs, num_tokens, int(md.max_query_len), _single_query_seqs(md, num_seqs),
        num_heads, num_kv_heads, head_dim, page,
        _lib.stream_handle(q.device),
    )
    _lib.check(rc, "bvllm_paged_prefill")
    return out
