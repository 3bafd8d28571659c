"""GPU parity of the three gfx950 kernels against the CPU oracle.

Scatter and the K/V reuse copy are bit-exact; attention and re-rotated K are
held to max-abs <= 2e-2 and cosine >= 0.9995 against fp32 (tests/_util.py).
Every case prints its name before touching the GPU.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as oattn
from oracle import prefill as opre
from oracle import rope as orope
from oracle import scatter as oscat
from tests._util import assert_attn_close, assert_close, bits, gen, randn_bf16, say
from vlcache_amd import kernels

pytestmark = pytest.mark.gpu


# ----------------------------------------------------------------------------- scatter
def _scatter_case(dev, n, hkv, hd, nb, bs, seed, dtype=torch.bfloat16, neg_every=7, v_row=None):
    g = gen(seed)
    d = hkv * hd
    v_row = v_row or d
    k = torch.randn(n, hkv, hd, generator=g).to(dtype)
    vbuf = torch.randn(n, v_row, generator=g).to(dtype)
    v = vbuf[:, v_row - d:].reshape(n, hkv, hd) if v_row == d else vbuf[:, v_row - d:].view(n, hkv, hd)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    if neg_every:
        slots[::neg_every] = -1
    kc = torch.randn(nb, bs, hkv, hd, generator=g).to(dtype)  # canary contents
    vc = torch.randn(nb, bs, hkv, hd, generator=g).to(dtype)
    # oracle on raw bits
    view = torch.int16 if dtype.itemsize == 2 else torch.int32
    kc_ref, vc_ref = kc.clone(), vc.clone()
    oscat.store_kvcache(k.view(view).numpy(), v.contiguous().view(view).numpy(), kc_ref.view(view).numpy(),
                        vc_ref.view(view).numpy(), slots.numpy())
    # device
    vbuf_d = vbuf.to(dev)
    v_d = vbuf_d[:, v_row - d:].view(n, hkv, hd)
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    kernels.store_kvcache_raw(k.to(dev), v_d, kc_d, vc_d, slots.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(kc_d.cpu().view(view), kc_ref.view(view))
    assert torch.equal(vc_d.cpu().view(view), vc_ref.view(view))


def test_scatter_cfg1_strided_value(dev):
    say("scatter: 199 tokens, 2x128 bf16, value row stride 2560, slot -1 every 7th")
    _scatter_case(dev, 199, 2, 128, 6, 256, seed=1, v_row=2560)


def test_scatter_cfg2_shape(dev):
    say("scatter: 1247 tokens, 2x128 bf16, value row stride 2560")
    _scatter_case(dev, 1247, 2, 128, 84, 256, seed=2, v_row=2560, neg_every=0)


def test_scatter_7b_rows_fp32_and_unaligned(dev):
    say("scatter: 7B rows 4x128 bf16; fp32 rows; unaligned 3x2 bf16 rows (element path)")
    _scatter_case(dev, 300, 4, 128, 4, 256, seed=3, v_row=28 * 128 + 2 * 512)
    _scatter_case(dev, 64, 2, 64, 2, 256, seed=4, dtype=torch.float32)
    _scatter_case(dev, 50, 3, 2, 2, 64, seed=5)


def test_scatter_out_of_range_slot_skipped(dev):
    say("scatter: slot beyond the cache is skipped, not written")
    n, hkv, hd, nb, bs = 8, 2, 128, 1, 16
    k = randn_bf16((n, hkv, hd), 6)
    v = randn_bf16((n, hkv, hd), 7)
    slots = torch.tensor([0, 1, 16, 2, 1 << 30, -1, 3, 4], dtype=torch.int32)
    kc = torch.zeros(nb, bs, hkv, hd, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    kernels.store_kvcache_raw(k.to(dev), v.to(dev), kc_d, vc_d, slots.to(dev))
    torch.cuda.synchronize()
    keep = [i for i, s in enumerate(slots.tolist()) if 0 <= s < nb * bs]
    ref = kc.view(-1, hkv, hd).clone()
    ref[slots[keep].long()] = k[keep]
    assert torch.equal(kc_d.cpu().view(-1, hkv, hd), ref)


@pytest.mark.parametrize("seed", range(6))
def test_scatter_random_shapes(dev, seed):
    """Seeded random scatters: token counts, kv heads, head dims, strided V rows, skip rates,
    bf16 and fp32 rows; bit for bit."""
    r = np.random.default_rng(4000 + seed)
    hkv, hd = int(r.choice([1, 2, 4, 8])), int(r.choice([64, 128]))
    n = int(r.integers(1, 3000))
    nb, bs = int(r.integers(-(-n // 256) + 1, 40)), 256
    dtype = torch.bfloat16 if r.random() < 0.75 else torch.float32
    v_row = None if r.random() < 0.5 else hkv * hd * 3
    neg = int(r.choice([0, 3, 11]))
    say(f"scatter random seed={seed}: n={n} hkv={hkv} hd={hd} blocks={nb} dtype={dtype} v_row={v_row} neg_every={neg}")
    _scatter_case(dev, n, hkv, hd, nb, bs, seed=500 + seed, dtype=dtype, neg_every=neg, v_row=v_row)


def test_scatter_call_above_the_nontemporal_limit(dev):
    """A scatter that writes more than 256 MB (65600 tokens x 8 kv heads x 128 dims, K and V:
    269 MB) takes the plain-store kernel; bit for bit, with skipped slots."""
    say("scatter: 65600 tokens x 8 x 128 (269 MB written, plain stores), slot -1 every 13th")
    _scatter_case(dev, 65600, 8, 128, 258, 256, seed=77, neg_every=13)


def test_scatter_call_between_the_store_limits(dev):
    """A scatter that writes between 64 and 256 MB (24000 tokens x 8 kv heads x 128 dims: 98 MB)
    takes the nontemporal-store kernel (smaller calls store at agent scope); bit for bit."""
    say("scatter: 24000 tokens x 8 x 128 (98 MB written, nontemporal stores), slot -1 every 11th")
    _scatter_case(dev, 24000, 8, 128, 95, 256, seed=78, neg_every=11)


# ----------------------------------------------------------------------------- rerotate
def _rerotate_setup(L, nb, seed, hkv=2, hd=128):
    g = gen(seed)
    kv = torch.randn(2, L, nb, 256, hkv, hd, generator=g).to(torch.bfloat16)
    return kv


def _cfg1_slots(nb_entry=6):
    # cached entry: image at [16, 1040) in blocks 0..5; new sequence: image at [64, 1088) in blocks 11..6
    entry_bt = list(range(nb_entry))
    seq_bt = list(range(2 * nb_entry - 1, nb_entry - 1, -1))
    R = opre.recompute_count(0.1, 1024)
    old, new = opre.image_kv_copy_slots(entry_bt, 16, seq_bt, 64, 64 + 1024, R)
    return old, new


def test_rerotate_zero_delta_is_bit_copy(dev):
    say("rerotate: delta 0 over 3 layers is a bit copy of K and V")
    kv = _rerotate_setup(3, 12, seed=10)
    old, new = _cfg1_slots()
    ref = kv.clone()
    oscat.copy_image_kv(ref.view(torch.int16).numpy(), old, new)
    kv_d = kv.to(dev)
    cs = kernels.rerotation_table([[0, 0, 0]], 128, 1e6, (16, 24, 24), device=dev)
    kernels.rerotate_copy_kv(kv_d, torch.tensor(old, device=dev), torch.tensor(new, device=dev), cs)
    torch.cuda.synchronize()
    assert np.array_equal(bits(kv_d), bits(ref))


def test_rerotate_plain_copy_matches_reference_copy(dev):
    say("rerotate: rotate_k=False is the reference's copy_image_kv, bit for bit")
    kv = _rerotate_setup(2, 12, seed=11)
    old, new = _cfg1_slots()
    ref = kv.clone()
    oscat.copy_image_kv(ref.view(torch.int16).numpy(), old, new)
    kv_d = kv.to(dev)
    kernels.rerotate_copy_kv(kv_d, torch.tensor(old, device=dev), torch.tensor(new, device=dev), rotate_k=False)
    torch.cuda.synchronize()
    assert np.array_equal(bits(kv_d), bits(ref))


def test_rerotate_cfg1_delta48(dev):
    say("rerotate: cfg1 slots, 921 reused tokens, delta (48,48,48), 2 layers")
    kv = _rerotate_setup(2, 12, seed=12)
    old, new = _cfg1_slots()
    cs = orope.rerotation_cos_sin([[48, 48, 48]], 128, 1e6, [16, 24, 24])
    ref = kv.clone()
    orope.rerotate_copy_kv(ref, old, new, cs)
    kv_d = kv.to(dev)
    kernels.rerotate_copy_kv(kv_d, torch.tensor(old, device=dev), torch.tensor(new, device=dev), cs.to(dev))
    torch.cuda.synchronize()
    out = kv_d.cpu()
    # V and every untouched row: bit-exact; rotated K: the fp32 tolerance, and in practice bit-exact.
    assert torch.equal(out[1].view(torch.int16), ref[1].view(torch.int16))
    flat_o = out[0].view(2, -1, 2, 128)
    flat_r = ref[0].view(2, -1, 2, 128)
    assert_close(flat_o[:, new], flat_r[:, new], what="rerotated K")
    mism = (flat_o.view(torch.int16) != flat_r.view(torch.int16)).sum().item()
    print(f"rerotated K bf16 mismatches vs oracle: {mism}")
    assert mism == 0


def test_rerotate_segments_negative_and_sectioned_deltas(dev):
    say("rerotate: 3 segments, deltas (-40,-40,-40), (5,17,-3), (0,0,0); 3 layers, 4 kv heads")
    L, nb, hkv = 3, 16, 4
    kv = _rerotate_setup(L, nb, seed=13, hkv=hkv)
    g = gen(14)
    perm = torch.randperm(8 * 256, generator=g)
    old = perm[:700].tolist()
    new = (perm[700:1400] + 8 * 256).tolist()
    seg = torch.randint(0, 3, (700,), generator=g, dtype=torch.int32)
    deltas = [[-40, -40, -40], [5, 17, -3], [0, 0, 0]]
    cs = orope.rerotation_cos_sin(deltas, 128, 1e6, [16, 24, 24])
    ref = kv.clone()
    orope.rerotate_copy_kv(ref, old, new, cs, seg)
    kv_d = kv.to(dev)
    kernels.rerotate_copy_kv(kv_d, torch.tensor(old, device=dev), torch.tensor(new, device=dev), cs.to(dev),
                             seg.to(dev))
    torch.cuda.synchronize()
    out = kv_d.cpu()
    assert torch.equal(out[1].view(torch.int16), ref[1].view(torch.int16))
    assert_close(out[0], ref[0], what="rerotated K (segments)")
    assert (out[0].view(torch.int16) != ref[0].view(torch.int16)).sum().item() == 0


@pytest.mark.parametrize("seed", range(6))
def test_rerotate_random_shapes(dev, seed):
    """Seeded random re-rotations: layers, kv heads, token counts, 1-3 segments with
    random (dt, dh, dw) deltas, M-RoPE or 1-D sections; V and K bit for bit."""
    r = np.random.default_rng(2000 + seed)
    L, hkv = int(r.integers(1, 5)), int(r.choice([1, 2, 4]))
    nb = 12
    kv = _rerotate_setup(L, nb, seed=60 + seed, hkv=hkv)
    n = int(r.integers(1, 6 * 256 // 2))
    perm = r.permutation(nb * 256)
    old, new = perm[:n].tolist(), perm[n:2 * n].tolist()
    nseg = int(r.integers(1, 4))
    seg = torch.from_numpy(r.integers(0, nseg, n).astype(np.int32))
    deltas = r.integers(-300, 300, (nseg, 3)).tolist()
    section = [16, 24, 24] if r.random() < 0.7 else None
    if section is None:
        deltas = [[d[0]] * 3 for d in deltas]
    say(f"rerotate random seed={seed}: L={L} hkv={hkv} n={n} deltas={deltas} section={section}")
    cs = orope.rerotation_cos_sin(deltas, 128, 1e6, section)
    ref = kv.clone()
    orope.rerotate_copy_kv(ref, old, new, cs, seg)
    kv_d = kv.to(dev)
    kernels.rerotate_copy_kv(kv_d, torch.tensor(old, device=dev), torch.tensor(new, device=dev), cs.to(dev),
                             seg.to(dev))
    torch.cuda.synchronize()
    out = kv_d.cpu()
    assert torch.equal(out[1].view(torch.int16), ref[1].view(torch.int16)), "V"
    assert torch.equal(out[0].view(torch.int16), ref[0].view(torch.int16)), "K"


# ----------------------------------------------------------------------------- fused RoPE + scatter
def _recomputed_mrope_positions():
    """M-RoPE positions of the 1247 recomputed tokens of the 4K-image request (ratio 0.1)."""
    pos, _ = orope.mrope_positions([("text", 128), ("image", (1, 154, 274)), ("text", 64)])
    R = opre.recompute_count(0.1, 10549)
    cols = np.concatenate([np.arange(0, 128 + R), np.arange(128 + 10549, 128 + 10549 + 64)])
    return np.ascontiguousarray(pos[:, cols])


def _rope_case(dev, positions, hq, hkv, section, seed, nb=8, bs=256, neg_every=5, store=True,
               in_place=False, want_k=False, max_pos=16384, cache_offset=0, clamp_to=None):
    """Fused kernel vs oracle (RotaryEmbedding then store_kvcache), all outputs bit for bit."""
    hd = 128
    positions = np.asarray(positions, dtype=np.int64)
    n = positions.shape[-1]
    g = gen(seed)
    qkv = torch.randn(n, (hq + 2 * hkv) * hd, generator=g).to(torch.bfloat16)
    q = qkv[:, :hq * hd].view(n, hq, hd)
    k = qkv[:, hq * hd:(hq + hkv) * hd].view(n, hkv, hd)
    v = qkv[:, (hq + hkv) * hd:].view(n, hkv, hd)
    cache = orope.rope_cache(max_pos, hd, 1e6)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    if neg_every:
        slots[::neg_every] = -1
    kc = torch.randn(nb, bs, hkv, hd, generator=g).to(torch.bfloat16)  # canary contents
    vc = torch.randn(nb, bs, hkv, hd, generator=g).to(torch.bfloat16)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    pos_ref = positions if clamp_to is None else np.clip(positions, 0, clamp_to - 1)
    q_ref, k_ref = orope.rope_store_kvcache(pos_ref, q, k, v, cache, section,
                                            kc_ref if store else None, vc_ref if store else None, slots.numpy())
    qkv_d = qkv.to(dev)
    q_d = qkv_d[:, :hq * hd].view(n, hq, hd)
    k_d = qkv_d[:, hq * hd:(hq + hkv) * hd].view(n, hkv, hd)
    v_d = qkv_d[:, (hq + hkv) * hd:].view(n, hkv, hd)
    if cache_offset:  # rows at an address that is not 16-byte aligned: per-pair loads
        buf = torch.zeros(cache.numel() + cache_offset, dtype=torch.float32, device=dev)
        cache_d = buf[cache_offset:].view(cache.shape)
        cache_d.copy_(cache.to(dev))
    else:
        cache_d = cache.to(dev)
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    q_out, k_out = kernels.rope_store_kvcache(
        torch.from_numpy(positions).to(dev), q_d, k_d, v_d, cache_d, section,
        kc_d if store else None, vc_d if store else None, slots.to(dev) if store else None,
        q_out=q_d if in_place else None, return_k=want_k)
    torch.cuda.synchronize()
    assert np.array_equal(bits(q_out), bits(q_ref)), "rotated q"
    if in_place:
        assert np.array_equal(bits(qkv_d[:, :hq * hd]), bits(q_ref.reshape(n, -1)))
    # k and v inputs are read only
    assert np.array_equal(bits(qkv_d[:, hq * hd:]), bits(qkv[:, hq * hd:]))
    if want_k:
        assert np.array_equal(bits(k_out), bits(k_ref)), "rotated k (k_out)"
    else:
        assert k_out is None
    if store:
        assert np.array_equal(bits(kc_d), bits(kc_ref)), "k_cache"
        assert np.array_equal(bits(vc_d), bits(vc_ref)), "v_cache"


@pytest.mark.parametrize("seed", range(6))
def test_rope_store_random_shapes(dev, seed):
    """Seeded random fused RoPE + store calls: token counts, head layouts, 1-D or M-RoPE
    positions with random sections, skipped slots, q in place or not, k_out or not."""
    r = np.random.default_rng(5000 + seed)
    n = int(r.integers(1, 2500))
    hq, hkv = [(16, 2), (28, 4), (8, 1), (32, 2), (12, 12)][int(r.integers(0, 5))]
    if r.random() < 0.6:
        cut = sorted(r.choice(np.arange(1, 64), 2, replace=False).tolist())
        section = [cut[0], cut[1] - cut[0], 64 - cut[1]]
        pos = r.integers(0, 16000, (3, n))
    else:
        section, pos = None, r.integers(0, 16000, n)
    nb = -(-n // 256) + 2
    kw = dict(in_place=bool(r.random() < 0.5), want_k=bool(r.random() < 0.5), neg_every=int(r.choice([0, 5])))
    say(f"rope_store random seed={seed}: n={n} heads={hq}/{hkv} section={section} {kw}")
    _rope_case(dev, pos, hq, hkv, section, seed=600 + seed, nb=nb, **kw)


def test_rope_store_call_above_the_nontemporal_limit(dev):
    """A fused RoPE + store call that writes more than 256 MB (53000 tokens of 16/2 heads: q_out
    and the cache's k and v, 271 MB) takes the plain-store kernel; bit for bit, M-RoPE."""
    say("rope_store: 53000 tokens, 16/2 heads, M-RoPE [16,24,24] (271 MB written, plain stores)")
    pos = np.random.default_rng(46).integers(0, 16000, (3, 53000))
    _rope_case(dev, pos, 16, 2, [16, 24, 24], seed=46, nb=-(-53000 // 256) + 1, neg_every=0)


def test_rope_store_call_between_the_store_limits(dev):
    """A fused RoPE + store call that writes between 64 and 256 MB (20000 tokens of 16/2 heads:
    102 MB) takes the nontemporal-store kernel (smaller calls store at agent scope); bit for bit."""
    say("rope_store: 20000 tokens, 16/2 heads, M-RoPE [16,24,24] (102 MB written, nontemporal stores)")
    pos = np.random.default_rng(47).integers(0, 16000, (3, 20000))
    _rope_case(dev, pos, 16, 2, [16, 24, 24], seed=47, nb=-(-20000 // 256) + 1, neg_every=0)


def test_rope_store_4k_image_recomputed_mrope(dev):
    say("rope_store: 1247 recomputed tokens of the 4K-image request, M-RoPE [16,24,24], 16/2 heads, q in place")
    pos = _recomputed_mrope_positions()
    assert pos.shape == (3, 1247)
    _rope_case(dev, pos, 16, 2, [16, 24, 24], seed=40, nb=84, in_place=True, neg_every=0)


def test_rope_store_1d_7b_heads_k_out_and_skips(dev):
    say("rope_store: 1-D positions, 28/4 heads, slot -1 every 5th, k_out, separate q_out")
    _rope_case(dev, np.arange(300, 300 + 700), 28, 4, None, seed=41, nb=4, want_k=True)


def test_rope_store_unaligned_sections_and_cache(dev):
    say("rope_store: sections [10,27,27] and unaligned cache rows (per-pair path), distinct t/h/w")
    g = np.random.default_rng(42)
    pos = g.integers(0, 4000, size=(3, 333))
    _rope_case(dev, pos, 16, 2, [10, 27, 27], seed=42, nb=2, cache_offset=1, max_pos=4096)
    _rope_case(dev, pos, 16, 2, [16, 24, 24], seed=43, nb=2, cache_offset=1, max_pos=4096)


def test_rope_store_rotate_only_and_clamped_positions(dev):
    say("rope_store: no cache (rotation only) with k_out; positions outside the cache are clamped")
    pos = np.array([0, 5, -3, 4095, 4096, 1 << 40, 17], dtype=np.int64)
    _rope_case(dev, pos, 16, 2, None, seed=44, store=False, want_k=True, max_pos=4096, clamp_to=4096)
    pos3 = np.stack([pos, pos[::-1].copy(), pos])
    _rope_case(dev, pos3, 16, 2, [16, 24, 24], seed=45, nb=1, max_pos=4096, clamp_to=4096)


def test_rope_store_out_of_range_slot_skipped(dev):
    say("rope_store: slots beyond the cache are skipped, not written")
    hq, hkv, hd, n = 4, 2, 128, 6
    q = randn_bf16((n, hq, hd), 46)
    k = randn_bf16((n, hkv, hd), 47)
    v = randn_bf16((n, hkv, hd), 48)
    cache = orope.rope_cache(64, hd, 1e6)
    pos = np.arange(n)
    slots = torch.tensor([0, 16, 3, 1 << 30, -1, 5], dtype=torch.int32)
    kc = torch.zeros(1, 16, hkv, hd, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    keep = torch.tensor([0 <= s < 16 for s in slots.tolist()])
    _, k_ref = orope.rope_store_kvcache(pos, q, k, v, cache)
    kc_d, vc_d = kc.to(dev), vc.to(dev)
    kernels.rope_store_kvcache(torch.from_numpy(pos).to(dev), q.to(dev), k.to(dev), v.to(dev), cache.to(dev),
                               None, kc_d, vc_d, slots.to(dev))
    torch.cuda.synchronize()
    kr, vr = kc.view(16, hkv, hd).clone(), vc.view(16, hkv, hd).clone()
    idx = slots[keep].long()
    kr[idx] = k_ref[keep]
    vr[idx] = v[keep]
    assert np.array_equal(bits(kc_d.view(16, hkv, hd)), bits(kr))
    assert np.array_equal(bits(vc_d.view(16, hkv, hd)), bits(vr))


# ----------------------------------------------------------------------------- attention
def _paged_case(seed, hq, hkv, subseqs, page=256, extra_blocks=3, causal=True, shuffle=True):
    """Random q and a paged cache holding each virtual sequence's keys."""
    g = gen(seed)
    cu_q, cu_k = [0], [0]
    for sq, sk in subseqs:
        cu_q.append(cu_q[-1] + sq)
        cu_k.append(cu_k[-1] + sk)
    nbs = [-(-sk // page) for _, sk in subseqs]
    nb = sum(nbs) + extra_blocks
    ids = torch.randperm(nb, generator=g).tolist() if shuffle else list(range(nb))
    width = max(nbs) if nbs else 1
    bt = torch.full((len(subseqs), max(width, 1)), -1, dtype=torch.int32)
    p = 0
    for b, n in enumerate(nbs):
        bt[b, :n] = torch.tensor(ids[p:p + n], dtype=torch.int32)
        p += n
    q = torch.randn(cu_q[-1], hq, 128, generator=g).to(torch.bfloat16)
    kc = torch.randn(nb, page, hkv, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, page, hkv, 128, generator=g).to(torch.bfloat16)
    return q, kc, vc, bt, cu_q, cu_k


def _run_paged(dev, q, kc, vc, bt, cu_q, cu_k, hq, hkv, causal=True, num_cus=None):
    plan = kernels.plan_attention(cu_q, cu_k, hq, hkv, 128, causal, dev, num_cus=num_cus)
    out = kernels.varlen_attention(q.to(dev), kc.to(dev), vc.to(dev),
                                   torch.tensor(cu_q, dtype=torch.int32, device=dev),
                                   torch.tensor(cu_k, dtype=torch.int32, device=dev),
                                   128 ** -0.5, causal, bt.to(dev), plan=plan)
    torch.cuda.synchronize()
    return out.cpu(), plan


@pytest.mark.parametrize("num_cus", [None, 8, 4096])
def test_attention_cfg1_paged(dev, num_cus):
    say(f"attention: cfg1 paged (167,167),(32,1120) 16/2 heads, num_cus={num_cus}")
    hq, hkv = 16, 2
    q, kc, vc, bt, cu_q, cu_k = _paged_case(20, hq, hkv, [(167, 167), (32, 1120)])
    out, plan = _run_paged(dev, q, kc, vc, bt, cu_q, cu_k, hq, hkv, num_cus=num_cus)
    print(f"plan items={plan.num_items} combines={plan.num_combine}")
    ref = oattn.varlen_attention(q, kc, vc, cu_q, cu_k, 128 ** -0.5, True, bt.tolist(), 256)
    assert_attn_close(out, ref, what="cfg1 attention")


@pytest.mark.parametrize("subs,num_cus,min_splits", [([(64, 10741), (300, 300)], 256, 28),
                                                     ([(16, 20000)], 4096, 33),
                                                     ([(16, 60000)], 4096, 193),
                                                     ([(32, 3000)], 4096, 9)])
def test_attention_many_splits_repeat(dev, subs, num_cus, min_splits):
    """Long key ranges split into many partials (28, 63, 235 and 12 per query tile: the
    combine's (m, l) loads cover 64 splits per round, so 235 take four rounds; 12 take one
    16-deep batch) and merged by the combine pass: three calls on one plan and workspace
    give the same bits and match the oracle."""
    say(f"attention: many splits, subs={subs} num_cus={num_cus}, 3 calls on one plan")
    hq, hkv = 16, 2
    q, kc, vc, bt, cu_q, cu_k = _paged_case(24, hq, hkv, subs)
    plan = kernels.plan_attention(cu_q, cu_k, hq, hkv, 128, True, dev, num_cus=num_cus)
    comb = plan.host[16 + 16 * plan.num_items:16 + 16 * (plan.num_items + plan.num_combine)].reshape(-1, 16)
    print(f"plan items={plan.num_items} combines={plan.num_combine} max splits={int(comb[:, 5].max())}")
    assert int(comb[:, 5].max()) >= min_splits
    assert min_splits > 16 or int(comb[:, 5].max()) <= 16
    args = (q.to(dev), kc.to(dev), vc.to(dev), torch.tensor(cu_q, dtype=torch.int32, device=dev),
            torch.tensor(cu_k, dtype=torch.int32, device=dev), 128 ** -0.5, True, bt.to(dev))
    outs = [kernels.varlen_attention(*args, plan=plan).cpu() for _ in range(3)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    ref = oattn.varlen_attention(q, kc, vc, cu_q, cu_k, 128 ** -0.5, True, bt.tolist(), 256)
    assert_attn_close(outs[0], ref, what="many-split attention")


def test_attention_7b_group7_multi_run(dev):
    say("attention: 7B heads 28/4, runs (118,118),(275,3030),(64,3200) paged")
    hq, hkv = 28, 4
    q, kc, vc, bt, cu_q, cu_k = _paged_case(21, hq, hkv, [(118, 118), (275, 3030), (64, 3200)])
    out, _ = _run_paged(dev, q, kc, vc, bt, cu_q, cu_k, hq, hkv)
    ref = oattn.varlen_attention(q, kc, vc, cu_q, cu_k, 128 ** -0.5, True, bt.tolist(), 256)
    assert_attn_close(out, ref, what="7B attention")


def test_attention_batched_ragged(dev):
    say("attention: 6 ragged sequences incl. sq=1, sq=sk, long suffix; 16/2 heads")
    subs = [(1, 1), (1, 700), (17, 17), (300, 300), (45, 2000), (129, 513)]
    hq, hkv = 16, 2
    q, kc, vc, bt, cu_q, cu_k = _paged_case(22, hq, hkv, subs)
    out, _ = _run_paged(dev, q, kc, vc, bt, cu_q, cu_k, hq, hkv)
    ref = oattn.varlen_attention(q, kc, vc, cu_q, cu_k, 128 ** -0.5, True, bt.tolist(), 256)
    assert_attn_close(out, ref, what="ragged attention")


@pytest.mark.parametrize("seed", range(12))
def test_attention_random_shapes(dev, seed):
    """Seeded random varlen problems: sequence count, lengths (empty and short ones
    included), head layouts, page sizes, causal or not, and planner CU counts."""
    r = np.random.default_rng(1000 + seed)
    n = int(r.integers(1, 5))
    subs = []
    for _ in range(n):
        sq = int(r.choice([0, 1, int(r.integers(2, 200))]))
        sk = sq + int(r.integers(0, 1200)) if r.random() < 0.9 else max(0, sq - int(r.integers(1, 20)))
        subs.append((sq, sk))
    hq, hkv = [(16, 2), (28, 4), (8, 1), (32, 2), (12, 12)][int(r.integers(0, 5))]
    page = int(r.choice([16, 64, 256]))
    causal = bool(r.random() < 0.7)
    num_cus = [None, 8, 300][int(r.integers(0, 3))]
    say(f"attention random seed={seed}: subs={subs} heads={hq}/{hkv} page={page} causal={causal} "
        f"num_cus={num_cus}")
    q, kc, vc, bt, cu_q, cu_k = _paged_case(300 + seed, hq, hkv, subs, page=page)
    out, _ = _run_paged(dev, q, kc, vc, bt, cu_q, cu_k, hq, hkv, causal=causal, num_cus=num_cus)
    ref = oattn.varlen_attention(q, kc, vc, cu_q, cu_k, 128 ** -0.5, causal, bt.tolist(), page)
    assert_attn_close(out, ref, what=f"random attention seed {seed}")


@pytest.mark.parametrize("seed", range(24))
def test_attention_random_wide(dev, seed):
    """A wider random space: up to 5 sequences of up to 1300 queries and 4300 keys, page sizes
    16-256 (page boundaries inside tiles included), contiguous K/V, 16:1 and 1:1 head
    groupings, plans without splits (num_cus < 0) and with many (num_cus 4096)."""
    r = np.random.default_rng(50000 + seed)
    n = int(r.integers(1, 6))
    subs = []
    for _ in range(n):
        sq = int(r.choice([0, 1, int(r.integers(2, 300)), int(r.integers(300, 1300))]))
        sk = sq + int(r.integers(0, 3000)) if r.random() < 0.85 else max(0, sq - int(r.integers(1, 40)))
        subs.append((sq, sk))
    hq, hkv = [(16, 2), (28, 4), (8, 1), (32, 2), (12, 12), (16, 1), (4, 4)][int(r.integers(0, 7))]
    contiguous = r.random() < 0.2
    page = int(r.choice([16, 32, 48, 64, 80, 128, 256]))
    causal = bool(r.random() < 0.7)
    num_cus = [None, 8, 300, 4096, -1][int(r.integers(0, 5))]
    say(f"attention wide seed={seed}: subs={subs} heads={hq}/{hkv} page={'contiguous' if contiguous else page} "
        f"causal={causal} num_cus={num_cus}")
    q, kc, vc, bt, cu_q, cu_k = _paged_case(70000 + seed, hq, hkv, subs, page=page)
    if contiguous:
        rows = [bt[b, j // page].item() * page + j % page for b, (_, sk) in enumerate(subs) for j in range(sk)]
        k = torch.cat([kc.view(-1, hkv, 128)[rows], torch.zeros(1, hkv, 128, dtype=torch.bfloat16)])
        v = torch.cat([vc.view(-1, hkv, 128)[rows], torch.zeros(1, hkv, 128, dtype=torch.bfloat16)])
        plan = kernels.plan_attention(cu_q, cu_k, hq, hkv, 128, causal, dev, num_cus=num_cus)
        out = kernels.varlen_attention(q.to(dev), k.to(dev), v.to(dev),
                                       torch.tensor(cu_q, dtype=torch.int32, device=dev),
                                       torch.tensor(cu_k, dtype=torch.int32, device=dev), 128 ** -0.5, causal,
                                       None, plan=plan).cpu()
    else:
        out, _ = _run_paged(dev, q, kc, vc, bt, cu_q, cu_k, hq, hkv, causal=causal, num_cus=num_cus)
    ref = oattn.varlen_attention(q, kc, vc, cu_q, cu_k, 128 ** -0.5, causal, bt.tolist(), page)
    assert_attn_close(out, ref, what=f"wide random attention seed {seed}")


@pytest.mark.parametrize("page", [16, 32, 48, 80])
def test_attention_small_pages_and_non_causal(dev, page):
    """Pages that are multiples of 16 but not of 64: each wave's 16 rows of a tile lie in
    one page (48 and 80 put page boundaries inside tiles), causal and non-causal."""
    say(f"attention: page size {page} (per-wave page lookup), causal and non-causal")
    subs = [(40, 100), (7, 7), (64, 64), (130, 700)]
    hq, hkv = 8, 1
    q, kc, vc, bt, cu_q, cu_k = _paged_case(23, hq, hkv, subs, page=page)
    for causal in (True, False):
        out, _ = _run_paged(dev, q, kc, vc, bt, cu_q, cu_k, hq, hkv, causal=causal)
        ref = oattn.varlen_attention(q, kc, vc, cu_q, cu_k, 128 ** -0.5, causal, bt.tolist(), page)
        assert_attn_close(out, ref, what=f"page-{page} causal={causal}")


@pytest.mark.parametrize("page", [64, 192, 320])
def test_attention_block_ids_read_ahead(dev, page):
    """Paged plans of several waves read each step's block ids one step early and carry the
    tile's row within its page from step to step.  Pages of 64 keys (a new page every tile)
    and sizes that are multiples of 64 but not powers of two, with splits that start inside
    a page: against the oracle, and bit-identical to the same plan run by the kernel that
    reads the block ids in the step (the one-wave kernel, chosen by the plan's priority
    word 11 = 2)."""
    say(f"attention: block ids read a step ahead, page size {page}, multi-wave plan (num_cus 48)")
    subs = [(300, 2900), (64, 1500), (700, 700), (5, 4100)]
    hq, hkv = 16, 2
    q, kc, vc, bt, cu_q, cu_k = _paged_case(31 + page, hq, hkv, subs, page=page)
    host, ws = kernels.plan_attention_host(cu_q, cu_k, hq, hkv, 128, True, num_cus=48)
    items = host[16:16 + 16 * int(host[1])].reshape(-1, 16)
    assert int(host[1]) > 2 * 48 and int(host[11]) != 2  # several waves: the read-ahead kernel
    if page != 64:
        assert ((items[:, 6] >= 0) & (items[:, 4] % page != 0)).any()  # a split starts inside a page
    cq = torch.tensor(cu_q, dtype=torch.int32, device=dev)
    ck = torch.tensor(cu_k, dtype=torch.int32, device=dev)
    outs = []
    for prio in (int(host[11]), 2):
        h = host.copy()
        h[11] = prio
        plan = kernels.attn_plan_on_device(h, ws, torch.from_numpy(h).to(dev), cu_q, cu_k, hq, hkv, True)
        out = kernels.varlen_attention(q.to(dev), kc.to(dev), vc.to(dev), cq, ck, 128 ** -0.5, True, bt.to(dev),
                                       plan=plan)
        torch.cuda.synchronize()
        outs.append(out.cpu())
    assert torch.equal(outs[0], outs[1]), "read-ahead and in-step block ids differ"
    ref = oattn.varlen_attention(q, kc, vc, cu_q, cu_k, 128 ** -0.5, True, bt.tolist(), page)
    assert_attn_close(outs[0], ref, what=f"page-{page} read-ahead block ids")


def test_attention_rows_without_keys_are_zero(dev):
    say("attention: causal with sk < sq: the first sq-sk rows see no key and are zero")
    subs = [(50, 20)]
    hq, hkv = 4, 2
    q, kc, vc, bt, cu_q, cu_k = _paged_case(24, hq, hkv, subs)
    out, _ = _run_paged(dev, q, kc, vc, bt, cu_q, cu_k, hq, hkv)
    ref = oattn.varlen_attention(q, kc, vc, cu_q, cu_k, 128 ** -0.5, True, bt.tolist(), 256)
    assert torch.count_nonzero(out[:30].float()) == 0
    assert_attn_close(out, ref, what="sk<sq")


def test_attention_block_permutation_bit_identical(dev):
    say("attention: same keys under two block layouts give bit-identical output")
    hq, hkv = 16, 2
    q, kc, vc, bt, cu_q, cu_k = _paged_case(25, hq, hkv, [(100, 100), (20, 900)], shuffle=False)
    out1, _ = _run_paged(dev, q, kc, vc, bt, cu_q, cu_k, hq, hkv)
    perm = torch.randperm(kc.shape[0], generator=gen(26))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    kc2, vc2 = kc[perm], vc[perm]  # block i of the new cache is old block perm[i]
    bt2 = torch.where(bt >= 0, inv[bt.clamp(min=0).long()].to(torch.int32), bt)
    out2, _ = _run_paged(dev, q, kc2, vc2, bt2, cu_q, cu_k, hq, hkv)
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))


def test_attention_contiguous_dense_strided_v(dev):
    say("attention: contiguous mode, dense causal 1500 tokens, v strided inside qkv rows")
    hq, hkv, n = 16, 2, 1500
    g = gen(27)
    qkv = torch.randn(n, (hq + 2 * hkv) * 128, generator=g).to(torch.bfloat16)
    q = qkv[:, :hq * 128].reshape(n, hq, 128).contiguous()
    k = qkv[:, hq * 128:(hq + hkv) * 128].reshape(n, hkv, 128).contiguous()
    cu = [0, n]
    qkv_d = qkv.to(dev)
    v_d = qkv_d[:, (hq + hkv) * 128:].view(n, hkv, 128)
    plan = kernels.plan_attention(cu, cu, hq, hkv, 128, True, dev)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=dev)
    out = kernels.varlen_attention(q.to(dev), k.to(dev), v_d, cu_d, cu_d, 128 ** -0.5, True, None, plan=plan)
    torch.cuda.synchronize()
    v = qkv[:, (hq + hkv) * 128:].reshape(n, hkv, 128)
    ref = oattn.varlen_attention(q, k, v, cu, cu, 128 ** -0.5, True, None)
    assert_attn_close(out.cpu(), ref, what="dense contiguous")


@pytest.mark.parametrize("causal", [True, False])
def test_attention_score_gap_between_lane_halves(dev, causal):
    """Keys 4..7 of every 8 score ~1000 above the others: the column max must cover both
    half-waves (each holds half of a tile's keys), or exp2 of the gap overflows."""
    say(f"attention: score gap of ~1000 between the key halves of each tile, causal={causal}")
    hq, hkv, n = 16, 2, 300
    g = gen(28)
    q = torch.ones(n, hq, 128).to(torch.bfloat16)
    k = torch.zeros(n, hkv, 128)
    k[(torch.arange(n) % 8) >= 4] = 8.0
    k = k.to(torch.bfloat16)
    v = torch.randn(n, hkv, 128, generator=g).to(torch.bfloat16)
    cu = [0, n]
    plan = kernels.plan_attention(cu, cu, hq, hkv, 128, causal, dev)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=dev)
    out = kernels.varlen_attention(q.to(dev), k.to(dev), v.to(dev), cu_d, cu_d, 128 ** -0.5, causal, None,
                                   plan=plan)
    torch.cuda.synchronize()
    ref = oattn.varlen_attention(q, k, v, cu, cu, 128 ** -0.5, causal, None)
    assert torch.isfinite(out.cpu().float()).all(), "non-finite output"
    assert_attn_close(out.cpu(), ref, what="score gap")


# ----------------------------------------------------------------------------- decode attention
def _decode_case(dev, lens, hq, hkv, seed, page=256, num_splits=0, extra_blocks=2, reps=1, pipeline=0):
    """Paged decode (one query per sequence) vs the fp32 oracle; returns the outputs of every rep."""
    g = gen(seed)
    B = len(lens)
    nbs = [max(1, -(-n // page)) for n in lens]
    nb = sum(nbs) + extra_blocks
    ids = torch.randperm(nb, generator=g).tolist()
    bt = torch.full((B, max(nbs)), -1, dtype=torch.int32)
    p = 0
    for b, n in enumerate(nbs):
        bt[b, :n] = torch.tensor(ids[p:p + n], dtype=torch.int32)
        p += n
    q = torch.randn(B, hq, 128, generator=g).to(torch.bfloat16)
    kc = torch.randn(nb, page, hkv, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, page, hkv, 128, generator=g).to(torch.bfloat16)
    cu_q = list(range(B + 1))
    cu_k = [0]
    for n in lens:
        cu_k.append(cu_k[-1] + n)
    ref = oattn.varlen_attention(q, kc, vc, cu_q, cu_k, 128 ** -0.5, True, bt.tolist(), page)
    plan = kernels.plan_decode(B, hq, hkv, 128, page, max(lens), dev, num_splits=num_splits, pipeline=pipeline)
    qd, kd, vd = q.to(dev), kc.to(dev), vc.to(dev)
    sl, btd = torch.tensor(lens, dtype=torch.int32, device=dev), bt.to(dev)
    outs = []
    for _ in range(reps):
        o = kernels.decode_attention(qd, kd, vd, sl, btd, 128 ** -0.5, plan=plan)
        torch.cuda.synchronize()
        outs.append(o.cpu())
    for o in outs:
        assert_attn_close(o, ref, what=f"decode {lens} hq={hq} hkv={hkv} splits={num_splits}")
    return outs, plan


def test_decode_7b_batch4_13k_context(dev):
    say("decode: 7B heads 28/4, batch 4, contexts 13432..13435, page 256")
    _, plan = _decode_case(dev, [13432, 13433, 13434, 13435], 28, 4, seed=60)
    assert plan.grid_splits > 1  # split-KV with the in-kernel merge


def test_decode_3b_ragged_lengths_and_empty(dev):
    say("decode: 3B heads 16/2, lengths 0, 1, 31, 32, 33, 700, 10741")
    lens = [0, 1, 31, 32, 33, 700, 10741]
    outs, _ = _decode_case(dev, lens, 16, 2, seed=61)
    assert torch.count_nonzero(outs[0][0]) == 0  # no key: zeros


@pytest.mark.parametrize("seed", range(8))
def test_decode_random_shapes(dev, seed):
    """Seeded random decode batches: batch size, context lengths (1 token to 5000), head
    layouts, page sizes and forced split counts."""
    r = np.random.default_rng(3000 + seed)
    B = int(r.integers(1, 7))
    lens = [int(x) for x in r.integers(1, 5000, B)]
    hq, hkv = [(16, 2), (28, 4), (8, 1), (32, 2), (12, 12)][int(r.integers(0, 5))]
    page = int(r.choice([16, 64, 256]))
    splits = [0, 1, int(r.integers(2, 40))][int(r.integers(0, 3))]
    say(f"decode random seed={seed}: lens={lens} heads={hq}/{hkv} page={page} splits={splits}")
    _decode_case(dev, lens, hq, hkv, seed=400 + seed, page=page, num_splits=splits)


@pytest.mark.parametrize("seed", range(12))
def test_decode_random_wide(dev, seed):
    """Up to 8 sequences of up to 9000 tokens, 16:1 and 1:1 head groupings, pages 16-256 and
    forced split counts up to 63."""
    r = np.random.default_rng(60000 + seed)
    B = int(r.integers(1, 9))
    lens = [int(x) for x in r.integers(1, 9000, B)]
    hq, hkv = [(16, 2), (28, 4), (8, 1), (32, 2), (12, 12), (16, 1)][int(r.integers(0, 6))]
    page = int(r.choice([16, 32, 64, 128, 256]))
    splits = [0, 1, int(r.integers(2, 64))][int(r.integers(0, 3))]
    say(f"decode wide seed={seed}: lens={lens} heads={hq}/{hkv} page={page} splits={splits}")
    _decode_case(dev, lens, hq, hkv, seed=80000 + seed, page=page, num_splits=splits)


@pytest.mark.parametrize("splits", [1, 3, 32])
def test_decode_forced_splits_repeatable(dev, splits):
    say(f"decode: forced {splits} chunks, 3 calls in a row (ticket counters reset), bit-identical")
    outs, plan = _decode_case(dev, [5000, 777, 3001], 16, 2, seed=62, num_splits=splits, reps=3)
    assert all(torch.equal(outs[0].view(torch.int16), o.view(torch.int16)) for o in outs[1:])
    assert int(plan.workspace[:4 * 3 * 2].view(torch.int32).count_nonzero()) == 0  # counters back at zero


@pytest.mark.parametrize("pipeline", [0x42, 0x22, 0x23, 0x24, 0x14, 0x142, 0x144, 0x182, 0x124])
def test_decode_pipeline_shapes(dev, pipeline):
    say(f"decode: kernel shape {pipeline:#x} (waves x stages), ragged lengths, 3 and 1 chunks")
    _decode_case(dev, [1, 95, 2500, 6000], 28, 4, seed=64, pipeline=pipeline, num_splits=3)
    _decode_case(dev, [33, 4000], 16, 2, seed=65, pipeline=pipeline, num_splits=1)


def test_decode_score_gap_between_lane_groups(dev):
    say("decode: keys 4..7 of every 8 score ~1000 above the others (column max over all lane groups)")
    B, hq, hkv, page, n = 2, 16, 2, 256, 700
    q = torch.ones(B, hq, 128).to(torch.bfloat16)
    kc = torch.zeros(3, page, hkv, 128)
    kc.view(-1, hkv, 128)[(torch.arange(3 * page) % 8) >= 4] = 8.0
    kc = kc.to(torch.bfloat16)
    vc = torch.randn(3, page, hkv, 128, generator=gen(67)).to(torch.bfloat16)
    bt = torch.tensor([[0, 1, 2], [2, 1, 0]], dtype=torch.int32)
    lens = [n, 517]
    ref = oattn.varlen_attention(q, kc, vc, [0, 1, 2], [0, n, n + 517], 128 ** -0.5, True, bt.tolist(), page)
    plan = kernels.plan_decode(B, hq, hkv, 128, page, n, dev, num_splits=3)
    out = kernels.decode_attention(q.to(dev), kc.to(dev), vc.to(dev), torch.tensor(lens, dtype=torch.int32,
                                   device=dev), bt.to(dev), 128 ** -0.5, plan=plan)
    torch.cuda.synchronize()
    assert torch.isfinite(out.cpu().float()).all()
    assert_attn_close(out.cpu(), ref, what="decode score gap")


def test_decode_small_pages_group7(dev):
    say("decode: page 32, 7 q heads per kv head, lengths 95, 96, 97, 4000; page 16 (16-key tiles)")
    _decode_case(dev, [95, 96, 97, 4000], 28, 4, seed=63, page=32)
    _decode_case(dev, [15, 16, 17, 900], 16, 2, seed=66, page=16)
