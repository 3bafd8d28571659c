"""The allocation-free decode entry point (vlc_decode_attn_noalloc) against vlc_decode_attn.

Both run the same kernels; the allocation-free one keeps its ticket counters and
split partials in the library's fixed per-device scratch.  Checked bit for bit
against the workspace entry point on calls in a row -- the second smaller than the
first (fewer sequences, shorter contexts, fewer chunks), then the first again (the
counters the first call left in the scratch must be back at zero) -- and once
against the fp32 oracle.
"""
from __future__ import annotations

import pytest
import torch

from oracle import attention as oattn
from tests._util import assert_attn_close, gen, say
from vlcache_amd import _lib, kernels

pytestmark = pytest.mark.gpu


def _problem(lens, hq, hkv, seed, page=256):
    g = gen(seed)
    B = len(lens)
    nbs = [max(1, -(-n // page)) for n in lens]
    nb = sum(nbs) + 2
    ids = torch.randperm(nb, generator=g).tolist()
    bt = torch.full((B, max(nbs)), -1, dtype=torch.int32)
    p = 0
    for b, n in enumerate(nbs):
        bt[b, :n] = torch.tensor(ids[p:p + n], dtype=torch.int32)
        p += n
    q = torch.randn(B, hq, 128, generator=g).to(torch.bfloat16)
    kc = torch.randn(nb, page, hkv, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, page, hkv, 128, generator=g).to(torch.bfloat16)
    return q, kc, vc, bt


def _both(dev, lens, hq, hkv, seed, num_splits=0, check_oracle=False):
    q, kc, vc, bt = _problem(lens, hq, hkv, seed)
    B = len(lens)
    args = (q.to(dev), kc.to(dev), vc.to(dev), torch.tensor(lens, dtype=torch.int32, device=dev), bt.to(dev))
    plan = kernels.plan_decode(B, hq, hkv, 128, 256, max(lens), dev, num_splits=num_splits)
    plan_na = kernels.plan_decode(B, hq, hkv, 128, 256, max(lens), dev, num_splits=num_splits, workspace=False)
    assert (plan_na.key_chunk, plan_na.grid_splits, plan_na.pipeline) == (plan.key_chunk, plan.grid_splits,
                                                                           plan.pipeline)
    say(f"decode noalloc: lens={lens} heads={hq}/{hkv} chunks={plan.grid_splits} "
        f"scratch bytes={plan_na.workspace_bytes if plan.grid_splits > 1 else 0}")
    ref = kernels.decode_attention(*args, 128 ** -0.5, plan=plan, max_seqlen_k=max(lens))
    out = torch.empty(B, hq, 128, dtype=torch.bfloat16, device=dev)
    got = kernels.decode_attention_noalloc(*args, 128 ** -0.5, plan=plan_na, out=out, max_seqlen_k=max(lens))
    torch.cuda.synchronize()
    assert got.data_ptr() == out.data_ptr()
    assert torch.equal(got.cpu().view(torch.int16), ref.cpu().view(torch.int16)), "noalloc != workspace entry"
    if check_oracle:
        cu_k = [0]
        for n in lens:
            cu_k.append(cu_k[-1] + n)
        o_ref = oattn.varlen_attention(q, kc, vc, list(range(B + 1)), cu_k, 128 ** -0.5, True, bt.tolist(), 256)
        assert_attn_close(got.cpu(), o_ref, what="decode noalloc vs oracle")
    return got.cpu()


def test_noalloc_decode_matches_workspace_entry_on_calls_in_a_row(dev):
    first = _both(dev, [13432, 13433, 13434, 13435], 28, 4, seed=90, check_oracle=True)  # 7B, 15 chunks
    _both(dev, [5000, 700], 16, 2, seed=91)                                              # smaller
    again = _both(dev, [13432, 13433, 13434, 13435], 28, 4, seed=90)
    assert torch.equal(first.view(torch.int16), again.view(torch.int16))


def test_noalloc_decode_single_chunk_and_ragged(dev):
    _both(dev, [1, 95, 2500, 6000, 0], 28, 4, seed=92, num_splits=1)  # one chunk: no scratch use
    _both(dev, [33, 4000, 257], 16, 2, seed=93, num_splits=7)


def test_noalloc_decode_refuses_oversized_call(dev):
    say("decode noalloc: a call needing more than the fixed scratch is refused")
    B, hq, hkv = 600, 28, 4
    q = torch.zeros(B, hq, 128, dtype=torch.bfloat16)
    kc = vc = torch.zeros(4, 256, hkv, 128, dtype=torch.bfloat16)
    bt = torch.zeros(B, 2, dtype=torch.int32)
    plan = kernels.plan_decode(B, hq, hkv, 128, 256, 300, dev, num_splits=2, workspace=False)
    assert plan.grid_splits == 2 and plan.workspace_bytes > _lib.DECODE_NOALLOC_MAX_BYTES
    out = torch.empty(B, hq, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="scratch"):
        kernels.decode_attention_noalloc(q.to(dev), kc.to(dev), vc.to(dev),
                                         torch.full((B,), 300, dtype=torch.int32, device=dev), bt.to(dev),
                                         128 ** -0.5, plan=plan, out=out)
