"""RMSNorm module with the fused residual add (babyvllm/layers/layernorm.py:11-38).

``forward(x, residual=None)`` returns ``(normed, residual)``: with a residual
it adds ``x`` into it in place and normalises the sum; without one it
normalises ``x`` and returns ``x`` as the new residual. GPU only (the HIP
kernel); a CPU tensor raises.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from babyvllm.kernels.layernorm import fused_add_rms_norm


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        if residual is None:
            return fused_add_rms_norm(x, None, self.weight, self.eps), x
        return fused_add_rms_norm(x, residual, self.weight, self.eps), residual
