"""CPU restatement of the reference's torch attention paths (test infrastructure only).

Follows:
  * ``gather_kv_batched``       <- babyvllm/layers/attention.py:71-95
  * ``make_decode_mask``        <- babyvllm/layers/attention.py:98-110
  * ``static_decode_attention`` <- babyvllm/layers/attention.py:113-134 (gather + SDPA decode)
  * ``paged_attention_torch``   <- babyvllm/layers/attention.py:137-175 (per-sequence SDPA loop)
  * ``causal_sdpa``             <- babyvllm/layers/attention.py:178-196
  * ``naive_causal_attention``  <- babyvllm/layers/attention.py:199-205
  * ``lse_merge``               <- paged_decode_attn_reduce_kernel, babyvllm/kernels/paged_attn.py:216-251
                                   and the split kernel's partial state, paged_attn.py:193-213

``brute_decode`` / ``brute_prefill`` are independent float64 loops over the
textbook definition softmax(q·kᵀ·scale)·v, used to pin the functions above; the
decode brute force mirrors the test reference in tests/test_paged_attn.py:93-107.

``md`` is any object with the fields of AttentionMetadata
(babyvllm/worker/context.py:5-17).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

_CAUSAL_SDPA_BACKENDS = (
    SDPBackend.FLASH_ATTENTION,
    SDPBackend.EFFICIENT_ATTENTION,
    SDPBackend.MATH,
)


def gather_kv_batched(kv_cache, block_tables, ctx_bucket: int, block_size: int):
    """Pages of every row gathered into ``[B, Hkv, ctx_bucket, D]`` K and V (attention.py:71-95)."""
    n_blocks_needed = (ctx_bucket + block_size - 1) // block_size
    n_blocks_needed = min(n_blocks_needed, block_tables.shape[1])
    B = block_tables.shape[0]
    n_kv_heads = kv_cache.shape[3]
    head_dim = kv_cache.shape[4]
    bt_flat = block_tables[:, :n_blocks_needed].reshape(-1).long()
    k_blocks = kv_cache[0][bt_flat]
    v_blocks = kv_cache[1][bt_flat]
    gathered = n_blocks_needed * block_size
    k = k_blocks.reshape(B, gathered, n_kv_heads, head_dim)
    v = v_blocks.reshape(B, gathered, n_kv_heads, head_dim)
    return k[:, :ctx_bucket].permute(0, 2, 1, 3), v[:, :ctx_bucket].permute(0, 2, 1, 3)


def make_decode_mask(seq_lens, ctx_bucket: int, dtype) -> torch.Tensor:
    """Additive ``[B, 1, 1, ctx]`` mask: 0 where position < seq_len, else −inf (attention.py:98-110)."""
    positions = torch.arange(ctx_bucket)
    valid = positions[None, :] < seq_lens.to(torch.int64)[:, None]
    additive = torch.zeros(seq_lens.shape[0], 1, 1, ctx_bucket, dtype=dtype)
    return additive.masked_fill(~valid[:, None, None, :], float("-inf"))


def static_decode_attention(q, kv_cache, block_tables, seq_lens, ctx_bucket: int, scale: float):
    """One query token per row: gather pages, then GQA SDPA with an additive mask (attention.py:113-134).

    A row with ``seq_len == 0`` has every key masked; SDPA then returns NaN for
    it, as the reference's torch path does. Callers compare only live rows.
    """
    B, num_heads, head_dim = q.shape
    num_kv_heads = kv_cache.shape[3]
    block_size = kv_cache.shape[2]
    K, V = gather_kv_batched(kv_cache, block_tables, ctx_bucket, block_size)
    Q = q.reshape(B, num_heads, 1, head_dim)
    mask = make_decode_mask(seq_lens, K.shape[2], q.dtype)
    group = num_heads // num_kv_heads
    if group > 1:
        Q = Q.reshape(B, num_kv_heads, group, head_dim)
    out = F.scaled_dot_product_attention(Q, K, V, attn_mask=mask, scale=scale)
    if group > 1:
        out = out.reshape(B, num_heads, 1, head_dim)
    return out.squeeze(2).reshape(-1, num_heads, head_dim)


def causal_sdpa(q, k, v, scale):
    """Causal attention for ``(seq, heads, dim)`` Q/K/V through 4-D SDPA with GQA (attention.py:178-196)."""
    q = q.transpose(0, 1).unsqueeze(0).contiguous()
    k = k.transpose(0, 1).unsqueeze(0).contiguous()
    v = v.transpose(0, 1).unsqueeze(0).contiguous()
    with sdpa_kernel(list(_CAUSAL_SDPA_BACKENDS)):
        out = F.scaled_dot_product_attention(
            q, k, v, is_causal=True, scale=scale, enable_gqa=q.shape[1] != k.shape[1],
        )
    return out.squeeze(0).transpose(0, 1).contiguous()


def naive_causal_attention(q, k, v, scale, num_queries_per_kv):
    """Single sequence, no cache (attention.py:199-205)."""
    if q.shape[1] != k.shape[1] * num_queries_per_kv:
        raise ValueError(
            f"query heads {q.shape[1]} != kv heads {k.shape[1]} × {num_queries_per_kv}"
        )
    return causal_sdpa(q, k, v, scale)


def paged_attention_torch(query, kv_cache, md, scale, num_queries_per_kv):
    """Per-sequence SDPA over each row's pages, causal with a cached prefix (attention.py:137-175).

    Query row i of sequence s sits at absolute position ``ctx_s + i`` and sees
    keys ``0 .. ctx_s + i``.
    """
    block_size = kv_cache.shape[2]
    num_kv_heads, head_dim = kv_cache.shape[3], kv_cache.shape[4]
    out = torch.empty_like(query)
    qsl = list(md.query_start_loc_cpu)
    for i, (start, end) in enumerate(zip(qsl[:-1], qsl[1:])):
        seq_len = md.seq_lens_cpu[i]
        ctx_len = md.context_lens_cpu[i]
        q_len = end - start
        if q_len == 0:
            continue
        num_blocks = (seq_len + block_size - 1) // block_size
        blocks = md.block_tables[i, :num_blocks].long()
        k_i = kv_cache[0][blocks].reshape(-1, num_kv_heads, head_dim)[:seq_len]
        v_i = kv_cache[1][blocks].reshape(-1, num_kv_heads, head_dim)[:seq_len]
        q_i = query[start:end]
        if ctx_len == 0 and q_len == seq_len:
            out[start:end] = causal_sdpa(q_i, k_i, v_i, scale)
        else:
            if num_queries_per_kv > 1:
                k_i = k_i.repeat_interleave(num_queries_per_kv, dim=1)
                v_i = v_i.repeat_interleave(num_queries_per_kv, dim=1)
            q_i = q_i.transpose(0, 1)
            k_i = k_i.transpose(0, 1)
            v_i = v_i.transpose(0, 1)
            mask = torch.tril(torch.ones(q_len, seq_len, dtype=torch.bool), diagonal=ctx_len)
            o = F.scaled_dot_product_attention(q_i, k_i, v_i, attn_mask=mask, scale=scale)
            out[start:end] = o.transpose(0, 1)
    return out


def lse_merge(part_out: torch.Tensor, part_lse: torch.Tensor) -> torch.Tensor:
    """Reweight normalised split outputs by their log-sum-exp (paged_attn.py:216-251).

    part_out ``[..., S, D]``, part_lse ``[..., S]`` (−inf marks an empty split).
    Accumulates in split order; an all-empty row gives exact zeros.
    """
    lse_max = part_lse.max(dim=-1, keepdim=True).values
    lse_max = torch.where(lse_max == float("-inf"), torch.zeros_like(lse_max), lse_max)
    num = torch.zeros(part_out.shape[:-2] + part_out.shape[-1:], dtype=torch.float32)
    den = torch.zeros(part_out.shape[:-2] + (1,), dtype=torch.float32)
    for n in range(part_out.shape[-2]):
        w = torch.exp(part_lse[..., n:n + 1] - lse_max)
        num = num + w * part_out[..., n, :]
        den = den + w
    return num / torch.where(den == 0, torch.ones_like(den), den)


def split_partials(q, kv_cache, block_tables, seq_lens, scale, num_splits, blocks_per_split):
    """Per-split normalised output and LSE, float64 (paged_attn.py:145-213 semantics).

    Split ``s`` covers pages ``[s·bps, (s+1)·bps)`` clipped to the row's pages; the
    last split runs to the row's last page. Empty splits give zeros and −inf.
    """
    B, H, D = q.shape
    bs = kv_cache.shape[2]
    hkv = kv_cache.shape[3]
    g = H // hkv
    width = block_tables.shape[1]
    out = torch.zeros(B, H, num_splits, D, dtype=torch.float64)
    lse = torch.full((B, H, num_splits), float("-inf"), dtype=torch.float64)
    for b in range(B):
        n = int(seq_lens[b])
        n_blocks = min(-(-n // bs), width)
        for s in range(num_splits):
            start = s * blocks_per_split
            end = n_blocks if s == num_splits - 1 else min(start + blocks_per_split, n_blocks)
            if start >= end:
                continue
            pages = block_tables[b, start:end].long()
            k = kv_cache[0][pages].reshape(-1, hkv, D).double()
            v = kv_cache[1][pages].reshape(-1, hkv, D).double()
            last = min(n, end * bs) - start * bs
            k, v = k[:last], v[:last]
            for h in range(H):
                sc = (k[:, h // g] @ q[b, h].double()) * scale
                m = sc.max()
                p = torch.exp(sc - m)
                l = p.sum()
                out[b, h, s] = (p @ v[:, h // g]) / l
                lse[b, h, s] = m + torch.log(l)
    return out, lse


# ---------------------------------------------------------------------------
# Independent float64 brute force (pins the SDPA-based functions above).
# ---------------------------------------------------------------------------

def _row_attention_f64(qv, keys, vals, scale):
    """softmax(q·kᵀ·scale)·v for one query vector, by explicit loops in float64."""
    scores = [scale * sum(float(a) * float(b) for a, b in zip(qv, kk)) for kk in keys]
    m = max(scores)
    w = [math.exp(s - m) for s in scores]
    z = sum(w)
    d = len(vals[0])
    return [sum(w[j] * float(vals[j][c]) for j in range(len(vals))) / z for c in range(d)]


def brute_decode(q, kv_cache, block_tables, lens, scale):
    """float64 loops: row b, head h attends keys 0..len-1 of KV head h // G. Padded rows are 0."""
    B, H, D = q.shape
    bs, hkv = kv_cache.shape[2], kv_cache.shape[3]
    g = H // hkv
    out = torch.zeros(B, H, D, dtype=torch.float64)
    for b, n in enumerate(lens):
        if n == 0:
            continue
        slots = [int(block_tables[b, p // bs]) * bs + p % bs for p in range(n)]
        kf = kv_cache[0].reshape(-1, hkv, D)
        vf = kv_cache[1].reshape(-1, hkv, D)
        for h in range(H):
            keys = [kf[s, h // g].tolist() for s in slots]
            vals = [vf[s, h // g].tolist() for s in slots]
            out[b, h] = torch.tensor(_row_attention_f64(q[b, h].tolist(), keys, vals, scale),
                                     dtype=torch.float64)
    return out


def brute_prefill(q, kv_cache, md, scale):
    """float64 loops over the varlen batch; row i of sequence s sees keys 0..ctx_s+i."""
    T, H, D = q.shape
    bs, hkv = kv_cache.shape[2], kv_cache.shape[3]
    g = H // hkv
    kf = kv_cache[0].reshape(-1, hkv, D)
    vf = kv_cache[1].reshape(-1, hkv, D)
    out = torch.zeros(T, H, D, dtype=torch.float64)
    qsl = list(md.query_start_loc_cpu)
    for s in range(len(qsl) - 1):
        ctx = md.context_lens_cpu[s]
        table = md.block_tables[s]
        for i, t in enumerate(range(qsl[s], qsl[s + 1])):
            visible = ctx + i + 1
            slots = [int(table[p // bs]) * bs + p % bs for p in range(visible)]
            for h in range(H):
                keys = [kf[x, h // g].tolist() for x in slots]
                vals = [vf[x, h // g].tolist() for x in slots]
                out[t, h] = torch.tensor(_row_attention_f64(q[t, h].tolist(), keys, vals, scale),
                                         dtype=torch.float64)
    return out
