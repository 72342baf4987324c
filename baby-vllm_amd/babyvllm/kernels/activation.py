"""SiLU(gate) * up on the HIP kernel (drop-in for babyvllm/kernels/activation.py:44-65).

``fused_silu_mul(gate_up)`` keeps the reference's signature and semantics:
``gate_up`` is (..., 2·D) holding gate then up; returns (..., D) =
bf16(silu(gate) · up) with silu and the product in fp32.
"""

from __future__ import annotations

import torch

from babyvllm.kernels import _lib


def fused_silu_mul(gate_up: torch.Tensor):
    """Fuses F.silu(gate) * up where gate_up is a concatenated tensor (..., 2 * D)."""
    assert gate_up.is_contiguous(), "gate_up tensor must be contiguous"
    _lib.require_rocm_tensor("gate_up", gate_up)
    if gate_up.dtype != torch.bfloat16:
        raise TypeError(f"gate_up must be bfloat16, got {gate_up.dtype}")
    original_shape = gate_up.shape[:-1]
    D = gate_up.shape[-1] // 2
    M = gate_up.numel() // (2 * D) if D > 0 else 0
    output = torch.empty((M, D), device=gate_up.device, dtype=gate_up.dtype)
    if M == 0 or D == 0:
        return output.view(*original_shape, D)
    rc = _lib.lib().bvllm_silu_mul(gate_up.data_ptr(), M, D, output.data_ptr(), _lib.stream_handle(gate_up.device))
    _lib.check(rc, "bvllm_silu_mul")
    return output.view(*original_shape, D)
