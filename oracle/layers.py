"""RMSNorm and SiLU-and-multiply as the reference computes them, on the CPU (test-only).

rms_norm restates layers/layernorm.py:16-40 (rms_forward / add_rms_forward):
fp32 statistics; with a residual, the fp32 sum is both rounded to bf16 (the new
residual) and normalised unrounded; the normalised value is rounded to bf16
before the bf16 weight multiply, whose product is rounded again.

silu_mul restates layers/activation.py:8-14 (SiluAndMul, torch.compile'd:
silu(gate) * up in fp32, one rounding to bf16).

Pinned in tests/test_oracle_layers.py against transformers' Qwen2RMSNorm
(an independent implementation of the same formula) and torch's SiLU.
"""
from __future__ import annotations

import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None):
    """bf16 x [rows, dim] -> bf16 out, or (out, new residual) when residual is given."""
    s = x.float()
    new_res = None
    if residual is not None:
        s = s + residual.float()
        new_res = s.to(torch.bfloat16)
    r = torch.rsqrt(s.pow(2).mean(dim=-1, keepdim=True) + eps)
    out = (s * r).to(torch.bfloat16) * weight.to(torch.bfloat16)
    return out if residual is None else (out, new_res)


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    g, u = gate_up.float().chunk(2, dim=-1)
    return (torch.nn.functional.silu(g) * u).to(torch.bfloat16)
