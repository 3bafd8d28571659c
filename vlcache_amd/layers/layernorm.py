"""RMSNorm with an optional fused residual add (layers/layernorm.py:5-50 of the reference)."""
from __future__ import annotations

import torch
from torch import nn


class RMSNorm(nn.Module):
    """(add +) RMSNorm with fp32 statistics (layers/layernorm.py:16-40)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x, residual=None):
        dtype = x.dtype
        xf = x.float()
        if residual is not None:
            xf = xf + residual.float()
            residual = xf.to(dtype)
        xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        out = xf.to(dtype) * self.weight
        return out if residual is None else (out, residual)
