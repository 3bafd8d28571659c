"""GPU parity of the benchmarked workloads, built exactly as bench.py builds them.

Each test constructs the workload's device state with WarmPrefillHotPath (the
class bench.py times), runs the step, and checks against the CPU oracle:

* the 4K-image warm request (3B, 36 layers, 128 + 10549 + 64 tokens, ratio
  0.1): the one-launch re-rotation of all 36 layers and every layer's fused
  M-RoPE + KV store bit for bit, and the attention call behind the headline
  figure (cu_seqlens_q [0, 1183, 1247], cu_seqlens_k [0, 1183, 11924], planned
  for the device's compute units) under the per-(row, head) bar;
* the same image at ratio 0 (dense causal 10741 x 10741, contiguous K/V as the
  reference's prefill without block tables, layers/attention.py:64-70 and
  engine/model_runner.py:278-299);
* eight warm requests sharing one cached 4K image (16 virtual sub-sequences,
  ratio 0.05, negative rotary shifts for prefixes shorter than the cached one).

The attention kernel's plan depends on the whole problem (its split decisions
follow the total work), so these are the plans the benchmark runs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oattn
from oracle import rope as orope
from tests._util import assert_attn_close, say
from vlcache_amd import kernels, workloads
from vlcache_amd.hotpath import WarmPrefillHotPath

pytestmark = pytest.mark.gpu


def _expected_cache(hp, kv_before):
    """The cache after one step, on the CPU: re-rotation copy, then every layer's store of
    the rotated k and of v at the recomputed tokens' slots.  Returns (cache, q_ref, k_ref)."""
    m = hp.model
    ref = kv_before.clone()
    if hp.n_reused:
        cs = orope.rerotation_cos_sin(hp.deltas, m.head_dim, m.rope_theta, list(m.mrope_section))
        orope.rerotate_copy_kv(ref, hp.old_slots.cpu().tolist(), hp.new_slots.cpu().tolist(), cs, hp.seg.cpu())
    q_ref, k_ref = orope.rope_store_kvcache(hp.positions.cpu().numpy(), hp.q_in.cpu(), hp.k_in.cpu(), None,
                                            hp.rope.cos_sin_cache.cpu(), list(m.mrope_section))
    if hp.paged:
        slots = hp.slot_mapping.cpu().long()
        d = m.num_kv_heads * m.head_dim
        v = hp.v.cpu().reshape(-1, d)
        for layer in range(m.num_layers):
            ref[0, layer].view(-1, d)[slots] = k_ref.reshape(-1, d)
            ref[1, layer].view(-1, d)[slots] = v
    return ref, q_ref, k_ref


def _check_cache(got, ref, what):
    mism = (got.view(torch.int16) != ref.view(torch.int16))
    n = int(mism.sum())
    if n:
        plane, layer = [int(x) for x in mism.nonzero()[0][:2]]
        raise AssertionError(f"{what}: {n} cache elements differ (first in plane {plane}, layer {layer})")


def test_4k_warm_request_36_layers(dev):
    """The headline workload: re-rotation of 36 layers x 9494 reused tokens, 36 fused
    M-RoPE + KV stores, and the benchmarked attention call."""
    say("config: 3B 4K-image warm request, 36 layers, ratio 0.1 (the benchmarked step)")
    wl = workloads.cfg2()
    hp = WarmPrefillHotPath(wl, dev, seed=0)
    assert hp.cu_q_host == [0, 1183, 1247] and hp.cu_k_host == [0, 1183, 11924]
    assert hp.n_reused == 9494 and hp.deltas == [[88, 88, 88]] and hp.paged
    print(f"plan for {kernels._num_cus(dev)} CUs: items={hp.plan.num_items} combines={hp.plan.num_combine} "
          f"partial slots={hp.plan.num_slots}", flush=True)
    kv_before = hp.kv_cache.cpu()
    out = hp.step().cpu()
    torch.cuda.synchronize()
    got = hp.kv_cache.cpu()
    ref, q_ref, _ = _expected_cache(hp, kv_before)
    del kv_before
    assert torch.equal(hp.q.cpu().view(torch.int16), q_ref.view(torch.int16)), "rotated q"
    _check_cache(got, ref, "36-layer re-rotation + fused stores")
    del got
    last = wl.model.num_layers - 1
    o_ref = oattn.varlen_attention(q_ref, ref[0, last], ref[1, last], hp.cu_q_host, hp.cu_k_host, hp.scale,
                                   True, hp.block_tables.cpu().tolist(), 256)
    assert_attn_close(out, o_ref, what="4K warm request attention (last layer)")
    assert np.isfinite(out.float().numpy()).all()
    # The plan is reused by every layer: layer 0 through the same plan and workspace.
    say("config: 4K warm request, attention of layer 0 on the same plan")
    out0 = hp.attention(0).cpu()
    o_ref0 = oattn.varlen_attention(q_ref, ref[0, 0], ref[1, 0], hp.cu_q_host, hp.cu_k_host, hp.scale,
                                    True, hp.block_tables.cpu().tolist(), 256)
    assert_attn_close(out0, o_ref0, what="4K warm request attention (layer 0)")


def test_4k_full_recompute_dense_contiguous(dev):
    """Ratio 0: one dense causal 10741 x 10741 call on contiguous K/V (v strided inside the
    QKV rows), the call the benchmark times for the full-recompute baseline."""
    say("config: 3B 4K image at ratio 0, dense causal 10741 x 10741, contiguous K/V")
    wl = workloads.cfg3(num_layers=1)
    hp = WarmPrefillHotPath(wl, dev, seed=1)
    assert hp.cu_q_host == [0, 10741] and hp.cu_k_host == [0, 10741] and not hp.paged
    print(f"plan: items={hp.plan.num_items} combines={hp.plan.num_combine}", flush=True)
    out = hp.step().cpu()
    torch.cuda.synchronize()
    _, q_ref, k_ref = _expected_cache(hp, hp.kv_cache.cpu())
    assert torch.equal(hp.q.cpu().view(torch.int16), q_ref.view(torch.int16)), "rotated q"
    assert torch.equal(hp.k.cpu().view(torch.int16), k_ref.view(torch.int16)), "rotated k"
    o_ref = oattn.varlen_attention(q_ref, k_ref, hp.v.cpu(), hp.cu_q_host, hp.cu_k_host, hp.scale, True, None)
    assert_attn_close(out, o_ref, what="dense 10741^2 attention")


def test_eight_requests_sharing_one_image(dev):
    """Eight warm requests sharing one cached 4K image: prefixes U[16, 512], suffixes
    U[16, 256] (seed 0), ratio 0.05, 16 virtual sub-sequences, 2 layers."""
    say("config: 3B, 8 requests sharing one 4K image, ratio 0.05, 16 sub-sequences, 2 layers")
    wl = workloads.cfg4(num_layers=2)
    hp = WarmPrefillHotPath(wl, dev, seed=2)
    assert len(hp.cu_q_host) == 17 and hp.paged
    deltas = [d[0] for d in hp.deltas]
    assert min(deltas) < 0 < max(deltas), deltas  # prefixes on both sides of the cached 128
    print(f"cu_q={hp.cu_q_host}\ncu_k={hp.cu_k_host}\nplan: items={hp.plan.num_items} "
          f"combines={hp.plan.num_combine}", flush=True)
    kv_before = hp.kv_cache.cpu()
    out = hp.step().cpu()
    torch.cuda.synchronize()
    got = hp.kv_cache.cpu()
    ref, q_ref, _ = _expected_cache(hp, kv_before)
    assert torch.equal(hp.q.cpu().view(torch.int16), q_ref.view(torch.int16)), "rotated q"
    _check_cache(got, ref, "8-request re-rotation + fused stores")
    o_ref = oattn.varlen_attention(q_ref, ref[0, 1], ref[1, 1], hp.cu_q_host, hp.cu_k_host, hp.scale, True,
                                   hp.block_tables.cpu().tolist(), 256)
    assert_attn_close(out, o_ref, what="8-request attention")


def test_4k_warm_request_graph_replays_match_eager(dev):
    """The warm request's per-layer calls (fused M-RoPE + KV store, then attention with its
    split-KV merge) for four layers captured as one HIP graph, as bench.py replays them, and
    replayed three times with eager calls of other layers in between (they rewrite the shared
    rotated q and the plan's split workspace).  Every replay's outputs equal the eager outputs
    bit for bit; the outputs are cleared by a fill kernel before each replay."""
    say("graph: 4K warm request, 4 layers of rope_store + attention, 3 replays vs eager")
    hp = WarmPrefillHotPath(workloads.cfg2(), dev, seed=0)
    layers = [0, 7, 19, 35]

    def run(outs):
        for l, o in zip(layers, outs):
            hp.rope_store(l)
            kernels.varlen_attention(hp.q, hp.k_caches[l], hp.v_caches[l], hp.cu_q, hp.cu_k, hp.scale, True,
                                     hp.block_tables, plan=hp.plan, out=o)

    eager = [torch.empty_like(hp.out) for _ in layers]
    run(eager)
    torch.cuda.synchronize()
    ref = [e.clone() for e in eager]
    outs = [torch.empty_like(hp.out) for _ in layers]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(outs)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(outs)
    for rep in range(3):
        for o in outs:
            o.zero_()
        for l in (3, 11, 28):  # eager work on the same q, workspace and plan
            hp.rope_store(l)
            hp.attention(l)
        g.replay()
        torch.cuda.synchronize()
        for l, o, r in zip(layers, outs, ref):
            assert torch.equal(o, r), f"replay {rep}, layer {l}"
