"""Pins of the RMSNorm / SiLU-and-multiply oracle (CPU)."""
from __future__ import annotations

import pytest
import torch

from oracle import layers as ol
from tests._util import randn_bf16


@pytest.mark.parametrize("dim", [64, 1280, 2048])
def test_rms_norm_matches_transformers(dim):
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm
    x = randn_bf16((33, dim), 1, 3.0)
    w = randn_bf16((dim,), 2) * 0.1 + 1
    m = Qwen2RMSNorm(dim, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        m.weight.copy_(w)
        ref = m(x)
    assert torch.equal(ol.rms_norm(x, w, 1e-6).view(torch.int16), ref.view(torch.int16))


def test_rms_norm_residual_is_the_norm_of_the_sum():
    x, r = randn_bf16((17, 256), 3), randn_bf16((17, 256), 4)
    w = randn_bf16((256,), 5)
    out, new_res = ol.rms_norm(x, w, 1e-6, r)
    assert torch.equal(new_res, (x.float() + r.float()).to(torch.bfloat16))
    # the norm takes the unrounded sum: equal to a plain norm of the fp32 sum, not of new_res in general
    s = x.float() + r.float()
    ref = (s * torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16) * w
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    # a scaled row gives the same normalised row (scale invariance, eps aside)
    o2 = ol.rms_norm((x.float() * 4).to(torch.bfloat16), w, 0.0)
    assert torch.equal(o2.view(torch.int16), ol.rms_norm(x, w, 0.0).view(torch.int16))


def test_silu_mul_against_torch_silu():
    gu = randn_bf16((9, 2 * 96), 6, 4.0)
    got = ol.silu_mul(gu)
    g, u = gu.float()[:, :96], gu.float()[:, 96:]
    ref = g * torch.sigmoid(g) * u
    assert torch.allclose(got.float(), ref, rtol=2 ** -8, atol=1e-6)
    assert torch.equal(ol.silu_mul(torch.cat([torch.zeros(1, 96), torch.ones(1, 96)], 1).to(torch.bfloat16)),
                       torch.zeros(1, 96, dtype=torch.bfloat16))
