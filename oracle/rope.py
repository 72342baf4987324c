"""CPU restatement of RoPE and the KV-store scatter (test infrastructure only).

Follows the reference's torch path:
  * ``rope_tables``      <- RotaryEmbedding.__init__/forward, babyvllm/layers/rotary.py:17-32
  * ``apply_rope``       <- apply_rope, babyvllm/layers/rotary.py:4-15
  * ``store_kvcache``    <- store_kvcache, babyvllm/layers/attention.py:24-32
  * ``slot_of``          <- KVCacheManager.get_slot_mapping, babyvllm/kv_cache_manager.py:62-76
                            and DecodeInputs.update, babyvllm/worker/decode_inputs.py:104
"""

from __future__ import annotations

import numpy as np
import torch


def rope_tables(dim: int, max_pos: int, base: float) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin tables ``[max_pos, dim]`` with duplicated halves (rotary.py:17-27)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))
    t = torch.arange(max_pos, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def gather_cos_sin(cos_t, sin_t, positions, dtype):
    """Per-token rows cast to the model dtype (rotary.py:29-32)."""
    return cos_t[positions].to(dtype), sin_t[positions].to(dtype)


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(q, k, cos, sin):
    """``x·cos + rotate_half(x)·sin`` with cos/sin ``[T, D]`` broadcast over heads (rotary.py:4-15).

    Evaluated op by op in the inputs' dtype, so bf16 inputs round after every
    multiply and after the add, exactly as torch's eager elementwise ops do.
    """
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)
    return (q * cos) + (_rotate_half(q) * sin), (k * cos) + (_rotate_half(k) * sin)


def store_kvcache(key, value, kv_cache, slot_mapping) -> None:
    """``index_copy_`` of k/v rows into the flat ``[NB·BS, Hkv, D]`` views (attention.py:24-32)."""
    _, _, _, num_kv_heads, head_dim = kv_cache.shape
    k_flat = kv_cache[0].view(-1, num_kv_heads, head_dim)
    v_flat = kv_cache[1].view(-1, num_kv_heads, head_dim)
    k_flat.index_copy_(0, slot_mapping, key.to(k_flat.dtype))
    v_flat.index_copy_(0, slot_mapping, value.to(v_flat.dtype))


def slot_of(table: list[int], pos: int, block_size: int) -> int:
    """``table[pos // bs] * bs + pos % bs`` (kv_cache_manager.py:62-76, decode_inputs.py:104)."""
    return table[pos // block_size] * block_size + pos % block_size


# ---------------------------------------------------------------------------
# Independent restatements used only to pin the functions above.
# ---------------------------------------------------------------------------

def bf16_round_np(x: np.ndarray) -> np.ndarray:
    """Round float32 -> bfloat16 (round to nearest, ties to even), returned as float32.

    Written from the IEEE-754 definition on the raw bits, independent of torch.
    NaN stays NaN.
    """
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def apply_rope_bf16_explicit(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Per-op-rounded bf16 RoPE from the closed form, in numpy.

    ``out1 = bf16(bf16(x1·c1) − bf16(x2·s1))``, ``out2 = bf16(bf16(x2·c2) + bf16(x1·s2))``.
    x ``[T, H, D]`` and cos/sin ``[T, D]`` hold bf16 values as float32. A product of
    two bf16 values is exact in float32, so each multiply rounds once.
    """
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    c1, c2 = cos[:, None, :half], cos[:, None, half:]
    s1, s2 = sin[:, None, :half], sin[:, None, half:]
    r = bf16_round_np
    o1 = r(r(x1 * c1) - r(x2 * s1))
    o2 = r(r(x2 * c2) + r(x1 * s2))
    return np.concatenate([o1, o2], axis=-1)
