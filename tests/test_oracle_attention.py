"""Pins the attention and scatter oracles on the CPU.

Attention: the fp32 SDPA restatement (oracle/attention.py) against a float64
element loop on tiny shapes, torch SDPA's is_causal for sq == sk, and layout
invariances.  Scatter / image-KV copy: element loops, the -1 skip and canary rows.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oattn
from oracle import scatter as oscat


def _case(seed, subs, hq, hkv, page=16, nb_extra=2):
    g = torch.Generator().manual_seed(seed)
    cu_q, cu_k = [0], [0]
    for sq, sk in subs:
        cu_q.append(cu_q[-1] + sq)
        cu_k.append(cu_k[-1] + sk)
    nbs = [-(-sk // page) for _, sk in subs]
    nb = sum(nbs) + nb_extra
    ids = torch.randperm(nb, generator=g).tolist()
    bt, p = [], 0
    for n in nbs:
        bt.append(ids[p:p + n] + [-1] * (max(nbs) - n))
        p += n
    q = torch.randn(cu_q[-1], hq, 128, generator=g)
    kc = torch.randn(nb, page, hkv, 128, generator=g)
    vc = torch.randn(nb, page, hkv, 128, generator=g)
    return q, kc, vc, bt, cu_q, cu_k


@pytest.mark.parametrize("causal", [True, False])
def test_varlen_matches_float64_loop(causal):
    subs = [(3, 3), (2, 9), (5, 20), (4, 2)]  # includes sk < sq: rows with no key are zero
    q, kc, vc, bt, cu_q, cu_k = _case(0, subs, hq=4, hkv=2)
    got = oattn.varlen_attention(q, kc, vc, cu_q, cu_k, 0.1, causal, bt, 16)
    ref = oattn.brute_force_attention(q.numpy(), kc.numpy(), vc.numpy(), cu_q, cu_k, 0.1, causal, bt, 16)
    assert np.abs(got.numpy() - ref).max() < 1e-5
    if causal:
        assert float(got[cu_q[3]:cu_q[3] + 2].abs().max()) == 0.0


def test_bottom_right_alignment_known_answer():
    # one query (sq = 1) against sk = 5 keys sees all 5 keys; with sq = sk = 5 the first row sees 1 key
    g = torch.Generator().manual_seed(1)
    k = torch.randn(5, 1, 128, generator=g)
    v = torch.randn(5, 1, 128, generator=g)
    q = torch.randn(1, 1, 128, generator=g)
    o = oattn.varlen_attention(q, k, v, [0, 1], [0, 5], 1.0, True)
    w = torch.softmax((k[:, 0] @ q[0, 0]), dim=0)
    assert torch.allclose(o[0, 0], w @ v[:, 0], atol=1e-5)
    q5 = torch.randn(5, 1, 128, generator=g)
    o5 = oattn.varlen_attention(q5, k, v, [0, 5], [0, 5], 1.0, True)
    assert torch.allclose(o5[0, 0], v[0, 0], atol=1e-6)


def test_equal_lengths_reduce_to_sdpa_is_causal():
    g = torch.Generator().manual_seed(2)
    n, hq = 37, 4
    q = torch.randn(n, hq, 128, generator=g)
    k = torch.randn(n, hq, 128, generator=g)
    v = torch.randn(n, hq, 128, generator=g)
    got = oattn.varlen_attention(q, k, v, [0, n], [0, n], 0.088, True)
    ref = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), is_causal=True,
                                         scale=0.088).transpose(0, 1)
    assert torch.allclose(got, ref, atol=1e-5)


def test_paged_equals_contiguous_and_gqa_equals_mha():
    q, kc, vc, bt, cu_q, cu_k = _case(3, [(6, 6), (3, 40)], hq=8, hkv=2)
    paged = oattn.varlen_attention(q, kc, vc, cu_q, cu_k, 0.1, True, bt, 16)
    ks = torch.cat([oattn.gather_keys(kc, bt[b], cu_k[b + 1] - cu_k[b], 16) for b in range(2)])
    vs = torch.cat([oattn.gather_keys(vc, bt[b], cu_k[b + 1] - cu_k[b], 16) for b in range(2)])
    contig = oattn.varlen_attention(q, ks, vs, cu_q, cu_k, 0.1, True)
    assert torch.equal(paged, contig)
    mha = oattn.varlen_attention(q, ks.repeat_interleave(4, dim=1), vs.repeat_interleave(4, dim=1), cu_q, cu_k, 0.1,
                                 True)
    assert torch.allclose(mha, contig, atol=1e-6)


def test_store_kvcache_element_loop_and_skip():
    g = torch.Generator().manual_seed(4)
    n, d = 9, 6
    key = torch.randint(0, 1 << 15, (n, 2, 3), generator=g, dtype=torch.int16).numpy()
    val = torch.randint(0, 1 << 15, (n, 2, 3), generator=g, dtype=torch.int16).numpy()
    kc = np.full((4, 4, 2, 3), 7, dtype=np.int16)  # canary
    vc = np.full((4, 4, 2, 3), 7, dtype=np.int16)
    slots = np.array([3, -1, 0, 15, 8, -1, 1, 2, 9], dtype=np.int32)
    oscat.store_kvcache(key, val, kc, vc, slots)
    kf, vf = kc.reshape(-1, d), vc.reshape(-1, d)
    for i, s in enumerate(slots):
        if s == -1:
            continue
        assert (kf[s] == key[i].reshape(-1)).all() and (vf[s] == val[i].reshape(-1)).all()
    untouched = sorted(set(range(16)) - set(int(s) for s in slots if s >= 0))
    assert (kf[untouched] == 7).all() and (vf[untouched] == 7).all()


def test_copy_image_kv_gathers_before_writing():
    kv = np.arange(2 * 3 * 2 * 4 * 1 * 2, dtype=np.int16).reshape(2, 3, 2, 4, 1, 2)
    before = kv.copy()
    old, new = [0, 1, 2], [5, 6, 0]  # slot 0 is both read and overwritten: the gather comes first
    oscat.copy_image_kv(kv, old, new)
    f0, f1 = before.reshape(2, 3, 8, 2), kv.reshape(2, 3, 8, 2)
    for o, nw in zip(old, new):
        assert (f1[:, :, nw] == f0[:, :, o]).all()
    assert (f1[:, :, [3, 4, 7]] == f0[:, :, [3, 4, 7]]).all()


def test_per_row_bar_catches_a_dropped_split():
    """A planted mistake on the CPU: one 8-position query tile of the 64 x 10741 suffix
    loses one 384-key split (keys [384, 768) of its 8 q heads of kv head 0).  The global
    bar (max-abs 2e-2, cosine 0.9995) passes it; the per-(row, head) bar must not."""
    from tests._util import assert_close, assert_rows_close

    g = torch.Generator().manual_seed(7)
    sq, sk, hq, hkv = 64, 10741, 16, 2
    q = torch.randn(sq + 300, hq, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(sk + 300, hkv, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(sk + 300, hkv, 128, generator=g).to(torch.bfloat16)
    cu_q, cu_k = [0, sq, sq + 300], [0, sk, sk + 300]
    ref = oattn.varlen_attention(q, k, v, cu_q, cu_k, 128 ** -0.5, True, None)
    bad = ref.clone()
    rows = torch.arange(8, 16)
    for h in range(8):  # q heads of kv head 0
        qi = q[rows, h].float()
        kk, vv = k[:sk, 0].float(), v[:sk, 0].float()
        keep = torch.ones(rows.numel(), sk, dtype=torch.bool)
        keep[:, 384:768] = False
        keep &= torch.arange(sk)[None, :] <= rows[:, None] + sk - sq
        bad[rows, h] = F.scaled_dot_product_attention(qi[None], kk[None], vv[None], attn_mask=keep[None],
                                                      scale=128 ** -0.5)[0]
    assert_close(bad, ref, what="planted dropped split (global bar)")
    with pytest.raises(AssertionError, match="cosine"):
        assert_rows_close(bad, ref, what="planted dropped split")
    # and the bar passes what it should: the oracle against its own bf16 rounding
    assert_rows_close(ref.to(torch.bfloat16), ref, what="bf16 rounding of the oracle")


def test_per_row_bar_demands_zero_rows():
    from tests._util import assert_rows_close

    ref = torch.zeros(4, 2, 128)
    ref[2:] = torch.randn(2, 2, 128)
    out = ref.clone()
    out[0, 1, 5] = 1e-3  # a row that sees no key must stay exactly zero
    with pytest.raises(AssertionError, match="non-zero"):
        assert_rows_close(out, ref)
