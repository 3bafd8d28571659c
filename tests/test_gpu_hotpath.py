"""GPU parity of a whole warm prefill step at the batched two-image 7B shapes.

Four requests of 64 text + 2691-token image + 64 text + 10549-token image + 64 text
(13432 tokens), ratio 0.02, both images cached standalone after 64 text tokens, 7B
heads (28 q / 4 kv), 2 layers: the reuse copy with per-image re-rotation, the fused
M-RoPE + KV store of the 457 recomputed tokens per request, and the paged attention
of the 12 virtual sub-sequences, checked against the CPU oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oattn
from oracle import rope as orope
from tests._util import assert_attn_close, say
from vlcache_amd import workloads
from vlcache_amd.hotpath import WarmPrefillHotPath

pytestmark = pytest.mark.gpu


def test_two_image_batch_step_matches_oracle(dev):
    say("hot path: batch 4 x (64 + 2691 + 64 + 10549 + 64), ratio 0.02, 7B heads, 2 layers")
    wl = workloads.cfg5(num_layers=2)
    r = wl.requests[0]
    assert r.recompute() == [54, 211] and r.deltas() == [0, 133]
    hp = WarmPrefillHotPath(wl, dev, seed=3)
    assert hp.cu_q_host[:4] == [0, 118, 393, 457] and hp.cu_k_host[:4] == [0, 118, 3148, 16580]
    kv_before = hp.kv_cache.cpu()
    out = hp.step().cpu()
    torch.cuda.synchronize()
    got = hp.kv_cache.cpu()

    # reuse copy: both images of every request, image k re-rotated by its own delta
    ref = kv_before.clone()
    cs = orope.rerotation_cos_sin(hp.deltas, 128, 1e6, [16, 24, 24])
    orope.rerotate_copy_kv(ref, hp.old_slots.cpu().tolist(), hp.new_slots.cpu().tolist(), cs, hp.seg.cpu())
    # fused M-RoPE + store of the recomputed tokens, every layer
    q_ref, k_ref = orope.rope_store_kvcache(hp.positions.cpu().numpy(), hp.q_in.cpu(), hp.k_in.cpu(), None,
                                            hp.rope.cos_sin_cache.cpu(), [16, 24, 24])
    assert torch.equal(hp.q.cpu().view(torch.int16), q_ref.view(torch.int16)), "rotated q"
    slots = hp.slot_mapping.cpu().long()
    d = 4 * 128
    for layer in range(2):
        ref[0, layer].view(-1, d)[slots] = k_ref.reshape(-1, d)
        ref[1, layer].view(-1, d)[slots] = hp.v.cpu().reshape(-1, d)
    mism = (got.view(torch.int16) != ref.view(torch.int16)).sum().item()
    assert mism == 0, f"{mism} cache elements differ"

    # attention of the last layer through the block tables
    o_ref = oattn.varlen_attention(q_ref, ref[0, 1], ref[1, 1], hp.cu_q_host, hp.cu_k_host, hp.scale, True,
                                   hp.block_tables.cpu().tolist(), 256)
    assert_attn_close(out, o_ref, what="two-image batch attention")
    assert np.isfinite(out.float().numpy()).all()
