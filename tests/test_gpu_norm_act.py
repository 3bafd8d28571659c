"""GPU parity of vlc_rms_norm and vlc_silu_mul against the CPU oracle (oracle/layers.py).

The new residual (a bf16 rounding of an fp32 sum of two bf16 values) is bit-exact.
The normalised output may differ from the oracle's in rare elements: the row's
sum of squares is accumulated in another order, so rsqrt can move by an fp32 ulp,
a normalised value at a bf16 rounding boundary can round the other way (one bf16
ulp), and the weight multiply rounds that difference again (up to two ulps of the
output).  SiLU-and-multiply rounds once (the device exp differs from the host's
in the last fp32 bits: at most one ulp).  Bars: |out - ref| <= 2^-6 |ref| for
RMSNorm, 2^-7 |ref| for SiLU-and-multiply, and the fraction of bit-exact
elements is printed.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import layers as ol
from tests._util import randn_bf16, say
from vlcache_amd import kernels

pytestmark = pytest.mark.gpu


def _within_ulps(got, ref, what, ulps=1):
    g, r = got.float().cpu(), ref.float().cpu()
    bad = (g - r).abs() > r.abs() * (ulps * 2.0 ** -7)
    n = int(bad.sum())
    exact = float((g == r).float().mean())
    print(f"{what}: {exact:.6f} of elements bit-exact", flush=True)
    assert n == 0, f"{what}: {n} elements beyond {ulps} bf16 ulp(s)"


@pytest.mark.parametrize("rows,dim", [(1, 64), (7, 1280), (1247, 2048), (42196, 1280), (33, 3584), (5, 8192),
                                      (129, 5120)])
@pytest.mark.parametrize("with_residual", [False, True], ids=["plain", "residual"])
def test_rms_norm(dev, rows, dim, with_residual):
    say(f"rms_norm rows={rows} dim={dim} residual={with_residual}")
    x = randn_bf16((rows, dim), rows + dim, 2.0)
    w = (randn_bf16((dim,), 3) * 0.2 + 1).to(torch.bfloat16)
    xd, wd = x.to(dev), w.to(dev)
    if with_residual:
        r = randn_bf16((rows, dim), 7)
        out, new_res = kernels.rms_norm(xd, wd, 1e-6, r.to(dev), residual_out=torch.empty_like(xd))
        ref, ref_res = ol.rms_norm(x, w, 1e-6, r)
        assert torch.equal(new_res.cpu().view(torch.int16), ref_res.view(torch.int16))
    else:
        out = kernels.rms_norm(xd, wd, 1e-6)
        ref = ol.rms_norm(x, w, 1e-6)
    _within_ulps(out, ref, f"rms_norm {rows}x{dim}", 2)


def test_rms_norm_strided_rows_and_in_place_residual(dev):
    """x a strided view (row stride 3 * dim); the new residual written over the old one."""
    say("rms_norm: strided x, residual updated in place")
    rows, dim = 300, 2048
    big = randn_bf16((rows, 3 * dim), 11)
    x = big[:, dim:2 * dim]
    r = randn_bf16((rows, dim), 12)
    w = randn_bf16((dim,), 13)
    rd = r.to(dev)
    out, new_res = kernels.rms_norm(big.to(dev)[:, dim:2 * dim], w.to(dev), 1e-6, rd)
    assert new_res.data_ptr() == rd.data_ptr()
    ref, ref_res = ol.rms_norm(x, w, 1e-6, r)
    assert torch.equal(rd.cpu().view(torch.int16), ref_res.view(torch.int16))
    _within_ulps(out, ref, "rms_norm strided", 2)


def test_rms_norm_rejects_bad_shapes(dev):
    x = torch.zeros(4, 100, dtype=torch.bfloat16, device=dev)       # dim % 8 != 0
    with pytest.raises(Exception):
        kernels.rms_norm(x, torch.ones(100, dtype=torch.bfloat16, device=dev), 1e-6)
    x = torch.zeros(4, 64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        kernels.rms_norm(x, torch.ones(64, dtype=torch.float32, device=dev), 1e-6)


@pytest.mark.parametrize("rows,inter", [(1, 4), (1247, 11008), (4219, 3420), (3, 18944)])
def test_silu_mul(dev, rows, inter):
    say(f"silu_mul rows={rows} inter={inter}")
    gu = randn_bf16((rows, 2 * inter), rows + inter, 3.0)
    out = kernels.silu_mul(gu.to(dev))
    _within_ulps(out, ol.silu_mul(gu), f"silu_mul {rows}x{inter}")


def test_silu_mul_extremes(dev):
    """Large |gate|: silu(-100) * up = -0 (exp overflows to inf), silu(100) = 100; 0 -> 0."""
    g = torch.tensor([[-100.0, 100.0, 0.0, -1e30]]).to(torch.bfloat16)
    u = torch.tensor([[3.0, 2.0, 5.0, 1.0]]).to(torch.bfloat16)
    out = kernels.silu_mul(torch.cat([g, u], 1).to(dev)).float().cpu()
    assert out.tolist() == [[-0.0, 200.0, 0.0, -0.0]]


@pytest.mark.parametrize("m,k,n,bias", [(1, 32, 16, False), (3, 2048, 2560, True), (4, 3584, 4608, True),
                                        (4, 18944, 3584, False), (16, 3584, 37888, False), (7, 11008, 2048, False),
                                        (2, 2048, 151936, False)])
def test_linear_skinny(dev, m, k, n, bias):
    """vlc_linear_skinny against the fp32 product of the same bf16 operands, rounded once:
    within one bf16 ulp of the fp32 reference (the fp32 sums are accumulated in another
    order than the reference's, a relative change of about K * 2^-24)."""
    from vlcache_amd import kernels

    say(f"linear_skinny m={m} k={k} n={n} bias={bias}")
    x = randn_bf16((m, k), m + k)
    w = randn_bf16((n, k), n + k, 0.05)
    b = randn_bf16((n,), 9) if bias else None
    out = kernels.linear_skinny(x.to(dev), w.to(dev), b.to(dev) if bias else None).float().cpu()
    ref = x.float() @ w.float().t() + (b.float() if bias else 0.0)
    tol = ref.abs() * 2.0 ** -7 + ref.abs().max() * k * 2.0 ** -24
    bad = int(((out - ref).abs() > tol).sum())
    assert bad == 0, f"{bad} outputs beyond one bf16 ulp"
    exact = float((out == ref.to(torch.bfloat16).float()).float().mean())
    print(f"equal to the rounded fp32 reference: {exact:.4f}", flush=True)


def test_linear_skinny_strided_rows_and_refusals(dev):
    from vlcache_amd import kernels

    big = randn_bf16((4, 3 * 1024), 3)
    w = randn_bf16((256, 1024), 4)
    x = big.to(dev)[:, 1024:2048]              # row stride 3072
    out = kernels.linear_skinny(x, w.to(dev)).float().cpu()
    ref = big[:, 1024:2048].float() @ w.float().t()
    assert ((out - ref).abs() <= ref.abs() * 2.0 ** -7 + 1e-3).all()
    with pytest.raises(ValueError):
        kernels.linear_skinny(randn_bf16((17, 1024), 5).to(dev), w.to(dev))      # more than 16 rows
    with pytest.raises(ValueError):
        kernels.linear_skinny(randn_bf16((4, 1000), 5).to(dev), randn_bf16((256, 1000), 6).to(dev))  # K % 32


def test_linear_layer_routes_few_rows_to_the_skinny_kernel(dev):
    """layers.linear.Linear: <= 16 rows through vlc_linear_skinny, more through torch; both
    agree with the fp32 product within bf16 rounding."""
    from vlcache_amd.layers.linear import Linear

    torch.manual_seed(0)
    lin = Linear(2048, 512, bias=True).to(dev, torch.bfloat16)
    for rows in (1, 16, 17, 300):
        x = randn_bf16((rows, 2048), rows).to(dev)
        y = lin(x).float().cpu()
        ref = x.float().cpu() @ lin.weight.float().cpu().t() + lin.bias.float().cpu()
        assert ((y - ref).abs() <= ref.abs() * 2.0 ** -6 + 2e-3).all(), rows
    y3 = lin(randn_bf16((2, 3, 2048), 7).to(dev))
    assert y3.shape == (2, 3, 512)


@pytest.mark.parametrize("seed", range(6))
def test_random_shapes(dev, seed):
    """Seeded random shapes for the three kernels: RMSNorm (dims multiples of 8 up to
    8192, 1..3000 rows, with and without the residual), SiLU-and-multiply (inter multiples
    of 4), and the skinny linear layer (1..16 rows, K multiples of 32, N multiples of 16,
    with and without bias), each against the oracle / fp32 product to the bars above."""
    from vlcache_amd import kernels

    rng = np.random.default_rng(100 + seed)
    rows, dim = int(rng.integers(1, 3000)), 8 * int(rng.integers(1, 1025))
    say(f"random shapes seed {seed}: rms {rows}x{dim}")
    x = randn_bf16((rows, dim), seed, float(rng.uniform(0.1, 10)))
    w = randn_bf16((dim,), seed + 1)
    if rng.integers(2):
        r = randn_bf16((rows, dim), seed + 2)
        out, nr = kernels.rms_norm(x.to(dev), w.to(dev), 1e-6, r.to(dev), residual_out=torch.empty_like(x, device=dev))
        ref, ref_r = ol.rms_norm(x, w, 1e-6, r)
        assert torch.equal(nr.cpu().view(torch.int16), ref_r.view(torch.int16))
    else:
        out, ref = kernels.rms_norm(x.to(dev), w.to(dev), 1e-6), ol.rms_norm(x, w, 1e-6)
    _within_ulps(out, ref, f"rms {rows}x{dim}", 2)
    srows, inter = int(rng.integers(1, 2000)), 4 * int(rng.integers(1, 3000))
    gu = randn_bf16((srows, 2 * inter), seed + 3, 3.0)
    _within_ulps(kernels.silu_mul(gu.to(dev)), ol.silu_mul(gu), f"silu {srows}x{inter}")
    m, k, n = int(rng.integers(1, 17)), 32 * int(rng.integers(1, 400)), 16 * int(rng.integers(1, 2000))
    xs = randn_bf16((m, k), seed + 4)
    ws = randn_bf16((n, k), seed + 5, 0.05)
    b = randn_bf16((n,), seed + 6) if rng.integers(2) else None
    say(f"skinny {m}x{k}x{n} bias={b is not None}")
    y = kernels.linear_skinny(xs.to(dev), ws.to(dev), b.to(dev) if b is not None else None).float().cpu()
    ref = xs.float() @ ws.float().t() + (b.float() if b is not None else 0.0)
    tol = ref.abs() * 2.0 ** -7 + ref.abs().max() * k * 2.0 ** -24
    assert int(((y - ref).abs() > tol).sum()) == 0
