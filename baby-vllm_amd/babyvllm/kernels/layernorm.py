"""Residual add + RMSNorm on the HIP kernel (drop-in for babyvllm/kernels/layernorm.py:46-83).

``fused_add_rms_norm(input, residual, weight, eps)`` keeps the reference's
signature and semantics: with a residual, ``residual += input`` in place (bf16)
and the normalised sum is returned; without one, ``input`` is normalised.
``out = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * weight)``; the output has the
input's shape and dtype. Inputs are viewed, never copied, so the in-place
residual update always lands in the caller's tensor.
"""

from __future__ import annotations

import torch

from babyvllm.kernels import _lib


def fused_add_rms_norm(input: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor, eps: float):
    original_shape = input.shape
    # .view (not .reshape): a non-contiguous input must fail loudly rather
    # than be copied, or the in-place residual update would land in a temporary.
    input_2d = input.view(-1, input.shape[-1])
    assert input_2d.stride(-1) == 1, "Last dimension must be contiguous"
    residual_2d = None
    if residual is not None:
        residual_2d = residual.view(-1, residual.shape[-1])
        assert residual_2d.stride(-1) == 1, "Residual last dimension must be contiguous"
    M, N = input_2d.shape
    for name, t in (("input", input_2d), ("weight", weight)):
        _lib.require_rocm_tensor(name, t)
    if input.dtype != torch.bfloat16:
        raise TypeError(f"input must be bfloat16, got {input.dtype}")
    if residual_2d is not None:
        _lib.require_rocm_tensor("residual", residual_2d)
        if residual_2d.dtype != torch.bfloat16 or residual_2d.shape != input_2d.shape:
            raise TypeError("residual must be a bfloat16 tensor of the input's shape")
    if weight.dtype not in (torch.bfloat16, torch.float32) or weight.numel() != N or not weight.is_contiguous():
        raise TypeError("weight must be a contiguous bfloat16 or float32 vector of the hidden size")
    output_2d = torch.empty_like(input_2d)
    rc = _lib.lib().bvllm_fused_add_rms_norm(
        input_2d.data_ptr(), input_2d.stride(0),
        None if residual_2d is None else residual_2d.data_ptr(),
        0 if residual_2d is None else residual_2d.stride(0),
        weight.data_ptr(), 1 if weight.dtype == torch.float32 else 0,
        output_2d.data_ptr(), output_2d.stride(0), M, N, float(eps),
        _lib.stream_handle(input.device),
    )
    _lib.check(rc, "bvllm_fused_add_rms_norm")
    return output_2d.view(original_shape)
