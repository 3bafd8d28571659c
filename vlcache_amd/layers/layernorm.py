"""RMSNorm with an optional fused residual add (layers/layernorm.py:5-50 of the reference).

One gfx950 kernel per call (vlc_rms_norm): fp32 statistics, the residual sum
rounded to bf16 for the next layer while the norm uses the fp32 sum, the
normalised value rounded to bf16 before the weight multiply, as the
reference's rms_forward / add_rms_forward compute.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import kernels


class RMSNorm(nn.Module):
    """(add +) RMSNorm with fp32 statistics (layers/layernorm.py:16-40)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x, residual=None):
        if residual is None:
            return kernels.rms_norm(x, self.weight, self.eps)
        # the new residual goes to a fresh tensor: callers may still hold the old one
        return kernels.rms_norm(x, self.weight, self.eps, residual, residual_out=torch.empty_like(residual))
