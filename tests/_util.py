"""Shared test helpers: seeded inputs and the tolerance rule of this path.

Floating-point parity bar: max |out - ref| <= 2e-2 and cosine(out, ref) >= 0.9995
against the fp32 oracle; integer and byte work is bit-exact.
"""
from __future__ import annotations

import sys

import numpy as np
import torch

ATOL = 2e-2
COS_MIN = 0.9995


def gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def randn_bf16(shape, seed: int, scale: float = 1.0) -> torch.Tensor:
    return (torch.randn(shape, generator=gen(seed)) * scale).to(torch.bfloat16)


def compare(out: torch.Tensor, ref: torch.Tensor):
    o = out.detach().float().cpu().flatten()
    r = ref.detach().float().cpu().flatten()
    err = (o - r).abs().max().item() if o.numel() else 0.0
    cos = torch.nn.functional.cosine_similarity(o.double(), r.double(), dim=0).item() if o.numel() else 1.0
    return err, cos


def assert_close(out: torch.Tensor, ref: torch.Tensor, atol: float = ATOL, cos_min: float = COS_MIN,
                 what: str = ""):
    err, cos = compare(out, ref)
    assert err <= atol and (cos >= cos_min or ref.abs().max().item() == 0.0), (
        f"{what}: max-abs {err:.3e} (<= {atol}), cosine {cos:.6f} (>= {cos_min})")
    return err, cos


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bits of a bf16/fp16 tensor as uint16 (for bit-exact comparisons)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def say(msg: str) -> None:
    """Name the case before a GPU step, flushed so a failing box still shows it."""
    print(msg, flush=True)
    sys.stdout.flush()
