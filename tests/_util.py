"""Shared test helpers: seeded inputs and the tolerance rule of this path.

Floating-point parity bar: max |out - ref| <= 2e-2 and cosine(out, ref) >= 0.9995
against the fp32 oracle; integer and byte work is bit-exact.  Attention and
decode outputs also pass a bar per (row, head) vector: cosine >= 0.9999 with the
oracle's vector, and exact zeros where the oracle's row sees no key.  A whole-
tensor cosine cannot see an error confined to a few rows (one query tile that
loses one split of its keys moves the global cosine by ~1e-6); the per-vector
bar fails on it.
"""
from __future__ import annotations

import sys

import numpy as np
import torch

ATOL = 2e-2
COS_MIN = 0.9995
ROW_COS_MIN = 0.9999


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


def row_cosines(out: torch.Tensor, ref: torch.Tensor):
    """Cosine of every [..., head_dim] vector of out with ref's, float64.

    Returns (cos, ref_zero, out_zero): vectors where ref is all zero get cos 1.0
    and are reported in ref_zero so the caller can demand exact zeros there."""
    hd = ref.shape[-1]
    o = out.detach().float().cpu().reshape(-1, hd).double()
    r = ref.detach().float().cpu().reshape(-1, hd).double()
    on, rn = o.norm(dim=1), r.norm(dim=1)
    ref_zero = rn == 0
    cos = (o * r).sum(dim=1) / (on * rn).clamp_min(1e-300)
    cos = torch.where(ref_zero, torch.ones_like(cos), cos)
    return cos, ref_zero, on == 0


def assert_rows_close(out: torch.Tensor, ref: torch.Tensor, row_cos_min: float = ROW_COS_MIN,
                      what: str = ""):
    """The per-(row, head) bar: cosine >= row_cos_min everywhere, zeros where ref is zero."""
    cos, ref_zero, out_zero = row_cosines(out, ref)
    bad_zero = ref_zero & ~out_zero
    assert not bool(bad_zero.any()), (
        f"{what}: {int(bad_zero.sum())} vectors are non-zero where the oracle's row sees no key "
        f"(first flat vector index {int(bad_zero.nonzero()[0])})")
    if cos.numel():
        worst = int(torch.argmin(cos))
        hq = ref.shape[-2] if ref.dim() >= 3 else 1
        assert cos[worst].item() >= row_cos_min, (
            f"{what}: row {worst // hq} head {worst % hq} cosine {cos[worst].item():.6f} (>= {row_cos_min})")
    return float(cos.min()) if cos.numel() else 1.0


def assert_attn_close(out: torch.Tensor, ref: torch.Tensor, what: str = ""):
    """Attention/decode bar: the global bar of assert_close plus the per-vector bar."""
    err, cos = assert_close(out, ref, what=what)
    worst = assert_rows_close(out, ref, what=what)
    print(f"{what}: max-abs {err:.3e}, cosine {cos:.7f}, worst row cosine {worst:.7f}", flush=True)
    return err, cos, worst


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bits of a bf16/fp16 tensor as uint16 (for bit-exact comparisons)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def say(msg: str) -> None:
    """Name the case before a GPU step, flushed so a failing box still shows it."""
    print(msg, flush=True)
    sys.stdout.flush()
