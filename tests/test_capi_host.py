"""CPU tests of the C-ABI library: it loads, exports every declared symbol, and
the host-side attention planner produces a work list that covers the problem.

No kernel is launched here (no GPU in this environment).
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from vlcache_amd import _lib, kernels, workloads

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from vlcache_amd import build

        build.build()
    return _lib.load()


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "vlc_capi.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vlc_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(lib):
    names = _declared_symbols()
    assert {"vlc_store_kvcache", "vlc_rerotate_copy_kv", "vlc_attn_plan", "vlc_varlen_attn_fwd"} <= set(names)
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_status_strings(lib):
    assert lib.vlc_abi_version() == _lib.ABI_VERSION
    assert lib.vlc_status_string(0) == b"ok"
    assert b"unsupported" in lib.vlc_status_string(-2)


def _items(plan):
    h = plan.host
    n_items, n_comb = int(h[1]), int(h[2])
    items = h[16:16 + 16 * n_items].reshape(-1, 16)
    comb = h[16 + 16 * n_items:16 + 16 * (n_items + n_comb)].reshape(-1, 16)
    return items, comb


def _check_plan_covers(cu_q, cu_k, hq, hkv, causal, num_cus):
    plan = kernels.plan_attention(cu_q, cu_k, hq, hkv, 128, causal, "cpu", num_cus=num_cus)
    items, comb = _items(plan)
    group = hq // hkv
    ppt = 128 // group
    assert int(plan.host[5]) == ppt
    # every (seq, kv head, query tile) is covered; split ranges partition [0, kmax) in 64-key steps
    expect = {}
    for b in range(len(cu_q) - 1):
        sq, sk = cu_q[b + 1] - cu_q[b], cu_k[b + 1] - cu_k[b]
        for qs in range(0, sq, ppt):
            qc = min(ppt, sq - qs)
            kmax = max(0, min(sk, qs + qc + sk - sq)) if causal else sk
            for g in range(hkv):
                expect[(b, g, qs)] = (qc, kmax)
    got = {}
    slots_seen = []
    for it in items:
        b, g, qs, qc, kb, ke, slot = (int(x) for x in it[:7])
        assert tuple(int(x) for x in it[7:11]) == (cu_q[b], cu_q[b + 1] - cu_q[b], cu_k[b], cu_k[b + 1] - cu_k[b])
        assert expect[(b, g, qs)][0] == qc
        got.setdefault((b, g, qs), []).append((kb, ke, slot))
        assert kb % 64 == 0 and kb <= ke
        if slot >= 0:
            slots_seen.append(slot)
    assert set(got) == set(expect)
    comb_of = {(int(c[0]), int(c[1]), int(c[2])): (int(c[4]), int(c[5])) for c in comb}
    for key, ranges in got.items():
        kmax = expect[key][1]
        ranges.sort()
        if len(ranges) == 1:
            assert ranges[0] == (0, kmax, -1)
            assert key not in comb_of
        else:
            first, n = comb_of[key]
            assert n == len(ranges)
            assert [r[2] for r in ranges] == list(range(first, first + n))
            assert ranges[0][0] == 0 and ranges[-1][1] == kmax
            for a, c in zip(ranges, ranges[1:]):
                assert a[1] == c[0]
    assert sorted(slots_seen) == list(range(int(plan.host[3])))
    # order: longest first, except a plan of one wave of workgroups (more items than CUs,
    # at most two per CU), where workgroup c + k shares a CU with workgroup k: the c - m
    # largest run alone (slots m .. c-1) and the others pair large with small
    cost = [max(1, -(-(int(i[5]) - int(i[4])) // 64)) for i in items]
    d = sorted(cost, reverse=True)
    n, c = len(cost), max(1, num_cus)
    if c < n <= 2 * c:
        m = n - c
        expect_cost = d[c - m:c] + d[:c - m] + d[c:][::-1]
        assert cost == expect_cost
    else:
        assert cost == d
    return plan


@pytest.mark.parametrize("num_cus", [1, 8, 256, 4096])
def test_plan_covers_warm_request(lib, num_cus):
    _check_plan_covers([0, 1183, 1247], [0, 1183, 11924], 16, 2, True, num_cus)


def test_plan_covers_ragged_and_group7(lib):
    rng = np.random.default_rng(0)
    for _ in range(20):
        n = int(rng.integers(1, 6))
        sq = rng.integers(0, 400, n)
        sk = sq + rng.integers(-20, 3000, n)
        sk = np.maximum(sk, 0)
        cu_q = [0] + list(np.cumsum(sq).astype(int))
        cu_k = [0] + list(np.cumsum(sk).astype(int))
        hq, hkv = [(16, 2), (28, 4), (8, 8), (32, 2)][int(rng.integers(0, 4))]
        _check_plan_covers(cu_q, cu_k, hq, hkv, bool(rng.integers(0, 2)), int(rng.integers(1, 512)))


def test_plan_rejects_bad_shapes(lib):
    with pytest.raises(_lib.VLCError) as e:
        kernels.plan_attention([0, 4], [0, 4], 16, 2, 64, True, "cpu")
    assert e.value.status == -2
    with pytest.raises(_lib.VLCError) as e:
        kernels.plan_attention([0, 4], [0, 4], 15, 2, 128, True, "cpu")
    assert e.value.status == -1
    # capacity protocol: a too-small buffer reports the needed length
    cu = np.array([0, 300], dtype=np.int32)
    n = ctypes.c_int64(0)
    ws = ctypes.c_int64(0)
    ip = ctypes.POINTER(ctypes.c_int32)
    buf = np.zeros(4, dtype=np.int32)
    st = lib.vlc_attn_plan(cu.ctypes.data_as(ip), cu.ctypes.data_as(ip), 1, 16, 2, 128, 1, 256,
                           buf.ctypes.data_as(ip), buf.size, ctypes.byref(n), ctypes.byref(ws))
    assert st == _lib.VLC_ERR_CAPACITY and n.value > 4


def test_kernel_wrappers_refuse_cpu_tensors(lib):
    q = torch.zeros(4, 16, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 256, 2, 128, dtype=torch.bfloat16)
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="HIP device"):
        kernels.varlen_attention(q, k, k, cu, cu, 0.1, True, torch.zeros(1, 1, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="HIP device"):
        kernels.store_kvcache_raw(torch.zeros(4, 2, 128), torch.zeros(4, 2, 128), k, k,
                                  torch.zeros(4, dtype=torch.int32))


def test_copy_entry_points_validate_before_launching(lib):
    """Argument errors come back as status codes before any launch: these calls pass
    placeholder (aligned, never dereferenced) device addresses and run without a GPU."""
    A = 1 << 20  # a 16-byte aligned placeholder address
    # empty work is a no-op
    assert lib.vlc_store_kvcache(A, 256, A, 256, A, A, 16, A, 0, 256, 2, None) == 0
    assert lib.vlc_store_kvcache(A, 256, A, 256, A, A, 16, A, -1, 256, 2, None) == _lib.VLC_ERR_INVALID
    # a row stride shorter than the row
    assert lib.vlc_store_kvcache(A, 128, A, 256, A, A, 16, A, 4, 256, 2, None) == _lib.VLC_ERR_INVALID
    # 2^28 tokens x 32 chunks of 16 bytes: beyond the kernel's 32-bit chunk index
    assert lib.vlc_store_kvcache(A, 256, A, 256, A, A, 16, A, 1 << 28, 256, 2, None) == _lib.VLC_ERR_UNSUPPORTED
    # re-rotation: 2^28 tokens x 16 units per token (2 kv heads x 128 dims) > 2^32 - 1
    row = 2 * 128
    slots = 1 << 29
    layer_stride = slots * row
    args = dict(plane_stride=36 * layer_stride, layer_stride=layer_stride, num_layers=36)
    st = lib.vlc_rerotate_copy_kv(A, args["plane_stride"], args["layer_stride"], args["num_layers"], A, A,
                                  1 << 28, slots, 2, 128, None, A, 1, 1, None)
    assert st == _lib.VLC_ERR_UNSUPPORTED
    st = lib.vlc_rerotate_copy_kv(A, args["plane_stride"], args["layer_stride"], args["num_layers"], A, A,
                                  0, slots, 2, 128, None, A, 1, 1, None)
    assert st == 0
    # head_dim not a multiple of 16; a layer stride shorter than the slots it must hold
    assert lib.vlc_rerotate_copy_kv(A, 0, 0, 1, A, A, 4, 16, 2, 120, None, A, 1, 1, None) == _lib.VLC_ERR_UNSUPPORTED
    assert lib.vlc_rerotate_copy_kv(A, 2 * 16 * row, 16 * row - 8, 1, A, A, 4, 16, 2, 128, None, A, 1, 1,
                                    None) == _lib.VLC_ERR_INVALID


def test_workload_counts_match_hand_derivation():
    # unmasked (query, key) pairs x 4 * hd * Hq: cfg1 49,372 pairs; cfg2 1,385,744; cfg3 57,689,911
    for wl, pairs in ((workloads.cfg1(), 49372), (workloads.cfg2(), 1385744), (workloads.cfg3(), 57689911)):
        cu_q, cu_k = wl.cu_seqlens()
        assert workloads.attention_flops(cu_q, cu_k, 16, 128) == 4 * 128 * 16 * pairs
    assert workloads.merged_grid(3840, 2160) == (77, 137)
    assert workloads.merged_grid(1920, 1080) == (39, 69)
    r = workloads.cfg2().requests[0]
    assert (r.R, r.n_reused, r.n_computed, r.delta) == (1055, 9494, 1247, 88)


def test_decode_noalloc_refuses_calls_beyond_its_scratch(lib):
    """600 sequences x 4 kv heads in 2 chunks each need ~40 MB of split partials, more
    than the fixed 16 MiB scratch: refused before any device call (the fake device
    addresses below are never touched)."""
    fake = 1 << 20
    B, hq, hkv = 600, 28, 4
    st = lib.vlc_decode_attn_noalloc(fake, hq * 128, fake, fake, hkv * 128, 256, 1000, fake, 64, 64, fake, B, hq,
                                     hkv, 128, 0.088, 1024, 2, 0x42, fake, hq * 128, None)
    assert st == _lib.VLC_ERR_SCRATCH
    assert b"scratch" in lib.vlc_status_string(st)
    # the same call through the torch wrapper's plan check
    plan = kernels.plan_decode(B, hq, hkv, 128, 256, 2048, "cpu", num_splits=2, workspace=False)
    assert plan.grid_splits == 2 and plan.workspace is None
    assert plan.workspace_bytes > _lib.DECODE_NOALLOC_MAX_BYTES


def test_plan_priority_policy():
    """Header word 11 (kPPrio): 2 (by remaining key tiles) when the plan's items fit in one
    wave of workgroups (two per CU), else 1 (alternating) when some sub-sequence has more
    keys than queries (reused context), else 0 (equal)."""
    def prio(cu_q, cu_k, hq=16, hkv=2):
        plan = kernels.plan_attention(cu_q, cu_k, hq, hkv, 128, True, "cpu", num_cus=256)
        n_items = int(plan.host[1])
        return int(plan.host[11]), n_items
    assert prio([0, 1183, 1247], [0, 1183, 11924]) == (2, 492)           # warm 4K request
    assert prio([0, 10, 30, 40], [0, 10, 30, 40], 28, 4)[0] == 2          # small square batch
    assert prio([0, 10, 30], [0, 10, 31], 28, 4)[0] == 2                 # small, reused context
    p, n = prio([0, 4096], [0, 4096])                                    # dense 4096^2: several waves
    assert p == 0 and n > 512
    p, n = prio([0, 10741], [0, 10741])
    assert p == 0 and n > 512
    cq, ck = workloads.cfg4().cu_seqlens()                               # 8 requests sharing an image
    p, n = prio(list(cq), list(ck))
    assert p == 1 and n > 512


def test_paged_attention_refuses_pages_not_multiple_of_16(lib):
    """Paged attention loads 16 consecutive keys per wave and tile from one page, so a
    page size that is not a multiple of 16 is refused before any device work (the
    reference's pages are multiples of 256, config.py:24)."""
    cu_q, cu_k = [0, 40], [0, 100]
    plan = kernels.plan_attention(cu_q, cu_k, 16, 2, 128, True, "cpu")
    ip = ctypes.POINTER(ctypes.c_int32)
    fake = 1 << 20  # 16-byte aligned stand-in addresses: the call must return before using them
    for page, want in ((8, -2), (24, -2), (100, -2)):
        st = lib.vlc_varlen_attn_fwd(fake, 16 * 128, fake, 2 * 128 * 1, fake, 2 * 128, fake, 8, page, 64,
                                     fake, fake, 1, 16, 2, 128, 128 ** -0.5, 1,
                                     plan.host.ctypes.data_as(ip), fake, plan.host.size,
                                     fake, 16 * 128, fake, 1 << 30, None)
        assert st == want, (page, st)
