"""Fused RoPE + KV-store append on the HIP kernel (drop-in for babyvllm/kernels/rope.py:101-153).

``fused_rope_and_cache`` keeps the reference's signature and semantics:
rotate-half RoPE on q and k *in place* (they are usually views into the fused
QKV projection output), and, when a cache and a slot mapping are given, the
rotated k and the raw v are written to ``kv_cache[0/1].view(-1, Hkv, D)[slot]``.
Returns ``(q, k)`` — the same tensors, mutated.
"""

from __future__ import annotations

import torch

from babyvllm.kernels import _lib


def _check_rows(name: str, t: torch.Tensor, ndim: int) -> None:
    if t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must have a unit stride on its last dimension")
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {t.dtype}")


def fused_rope_and_cache(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
    cos: torch.Tensor, sin: torch.Tensor,
    kv_cache: torch.Tensor | None = None, slot_mapping: torch.Tensor | None = None,
):
    """Rotate q ``[T, H, D]`` and k ``[T, Hkv, D]`` in place; optionally append k/v to the paged cache.

    cos/sin are ``[T, D]`` per-token rows (RotaryEmbedding output, duplicated halves).
    """
    for name, t in (("q", q), ("k", k), ("cos", cos), ("sin", sin)):
        _lib.require_rocm_tensor(name, t)
    _check_rows("q", q, 3)
    _check_rows("k", k, 3)
    _check_rows("cos", cos, 2)
    _check_rows("sin", sin, 2)
    num_tokens, num_heads, head_dim = q.shape
    num_kv_heads = k.shape[1]
    if k.shape[0] != num_tokens or k.shape[2] != head_dim:
        raise ValueError(f"k shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    if cos.shape[0] < num_tokens or cos.shape[1] != head_dim or sin.shape != cos.shape:
        raise ValueError("cos/sin must be [num_tokens, head_dim]")

    has_cache = kv_cache is not None and slot_mapping is not None
    if has_cache:
        _lib.require_rocm_tensor("v", v)
        _check_rows("v", v, 3)
        if v.shape != k.shape:
            raise ValueError(f"v shape {tuple(v.shape)} does not match k {tuple(k.shape)}")
        if kv_cache.dim() != 5 or kv_cache.shape[0] != 2 or kv_cache.shape[3] != num_kv_heads \
                or kv_cache.shape[4] != head_dim:
            raise ValueError(f"kv_cache must be [2, NB, BS, {num_kv_heads}, {head_dim}], "
                             f"got {tuple(kv_cache.shape)}")
        if kv_cache.dtype != torch.bfloat16:
            raise TypeError(f"kv_cache must be bfloat16, got {kv_cache.dtype}")
        if not kv_cache.is_contiguous():
            raise ValueError("kv_cache must be contiguous (its [NB·BS, Hkv, D] view is written)")
        if slot_mapping.dtype != torch.int64 or slot_mapping.dim() != 1 \
                or slot_mapping.shape[0] < num_tokens:
            raise TypeError("slot_mapping must be an int64 vector with one slot per token")
        if not slot_mapping.is_contiguous():
            slot_mapping = slot_mapping.contiguous()
        k_cache = kv_cache[0]
        v_cache = kv_cache[1]
        num_slots = kv_cache.shape[1] * kv_cache.shape[2]
        rc = _lib.lib().bvllm_rope_kv_append(
            q.data_ptr(), q.stride(0), q.stride(1),
            k.data_ptr(), k.stride(0), k.stride(1),
            v.data_ptr(), v.stride(0), v.stride(1),
            cos.data_ptr(), cos.stride(0),
            sin.data_ptr(), sin.stride(0),
            k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(1), k_cache.stride(2),
            num_slots, slot_mapping.data_ptr(),
            num_tokens, num_heads, num_kv_heads, head_dim,
            _lib.stream_handle(q.device),
        )
    else:
        rc = _lib.lib().bvllm_rope_kv_append(
            q.data_ptr(), q.stride(0), q.stride(1),
            k.data_ptr(), k.stride(0), k.stride(1),
            None, 0, 0,
            cos.data_ptr(), cos.stride(0),
            sin.data_ptr(), sin.stride(0),
            None, None, 0, 0, 0, None,
            num_tokens, num_heads, num_kv_heads, head_dim,
            _lib.stream_handle(q.device),
        )
    _lib.check(rc, "bvllm_rope_kv_append")
    return q, k
