"""CPU restatement of the decode step's other three kernels (test infrastructure only).

The reference computes these with Triton kernels whose math is the spec:
  * ``greedy_argmax``       <- _argmax_chunks_kernel + _argmax_rows_kernel,
                               babyvllm/kernels/argmax.py:14-56 (chunk winners,
                               then row winner; ties to the lowest index in both)
  * ``fused_add_rms_norm``  <- _fused_add_rms_norm_kernel, babyvllm/kernels/layernorm.py:5-43
                               (x + residual rounded to the input dtype and written
                               back; fp32 variance; bf16(x·rsqrt) · w rounded once more)
                               and the torch path it mirrors, babyvllm/layers/layernorm.py:27-37
  * ``silu_mul``            <- _silu_mul_kernel, babyvllm/kernels/activation.py:5-42
                               (silu and the product in fp32, one rounding at the end)
"""

from __future__ import annotations

import torch


def greedy_argmax(logits: torch.Tensor, block: int = 4096) -> torch.Tensor:
    """Row-wise argmax by the reference's two-stage reduction (argmax.py:14-38).

    Stage 1 takes each block-wide chunk's maximum and its first index, stage 2
    the first chunk holding the row maximum. NaN counts as the maximum (the
    first NaN wins), as in torch.argmax.
    """
    x = logits.float()
    rows, vocab = x.shape
    out = torch.empty(rows, dtype=torch.int64)
    for r in range(rows):
        best_v, best_i = None, None
        for lo in range(0, vocab, block):
            chunk = x[r, lo:lo + block]
            i = int(torch.argmax(chunk))
            v = float(chunk[i])
            if best_v is None or _before(v, lo + i, best_v, best_i):
                best_v, best_i = v, lo + i
        out[r] = best_i
    return out


def _before(v, i, w, j):
    vn, wn = v != v, w != w
    if vn or wn:
        return vn and (not wn or i < j)
    return v > w or (v == w and i < j)


def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor, eps: float):
    """Returns (out, new_residual) of the fused residual add + RMSNorm (layernorm.py:5-43)."""
    dt = x.dtype
    if residual is not None:
        x = (x.float() + residual.float()).to(dt)
        new_res = x
    else:
        new_res = None
    xf = x.float()
    var = (xf * xf).sum(-1, keepdim=True) / xf.shape[-1]
    normed = (xf * torch.rsqrt(var + eps)).to(dt)
    out = (normed.float() * weight.float()).to(dt)
    return out, new_res


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """bf16(silu(gate)·up) with the silu and product in fp32 (activation.py:30-41)."""
    d = gate_up.shape[-1] // 2
    g = gate_up[..., :d].float()
    u = gate_up[..., d:].float()
    sig = 1.0 / (1.0 + torch.exp(-g))
    return (g * sig * u).to(gate_up.dtype)
