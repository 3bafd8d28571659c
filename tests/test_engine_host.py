"""CPU tests of the host engine logic against the oracle and hand-derived answers."""
from __future__ import annotations

import numpy as np
import torch
import pytest

from oracle import prefill as op
from oracle import rope as orope
from vlcache_amd.config import QWEN25_VL_3B, Config, load_model_config
from vlcache_amd.engine.block_manager import BlockManager
from vlcache_amd.engine.positions import image_runs, mrope_positions
from vlcache_amd.engine.sequence import Sequence

IMG = 151655


def test_mrope_positions_match_oracle():
    # text 5, image (1, 6, 10) -> 15 tokens, text 3, image (1, 4, 4) -> 4 tokens, text 2
    toks = [1] * 5 + [IMG] * 15 + [2] * 3 + [IMG] * 4 + [3] * 2
    pos, starts, delta = mrope_positions(toks, [(1, 6, 10), (1, 4, 4)], IMG)
    ref, ref_starts = orope.mrope_positions([("text", 5), ("image", (1, 6, 10)), ("text", 3), ("image", (1, 4, 4)),
                                             ("text", 2)])
    assert np.array_equal(pos, ref)
    assert [s[0] for s in starts] == ref_starts
    assert delta == int(ref.max()) + 1 - len(toks)


def test_mrope_positions_reject_mismatched_grid():
    with pytest.raises(ValueError):
        mrope_positions([IMG] * 5, [(1, 4, 4)], IMG)
    with pytest.raises(ValueError):
        mrope_positions([IMG] * 4, [(1, 4, 4), (1, 2, 2)], IMG)


def test_image_runs():
    assert image_runs(np.array([1, IMG, IMG, 2, IMG]), IMG) == [(1, 3), (4, 5)]
    assert image_runs(np.array([1, 2]), IMG) == []


def test_sequence_image_range_matches_oracle():
    toks = [3, IMG, 4, IMG, IMG, 9]
    s = Sequence(toks)
    s.find_image_token_range(IMG)
    assert s.image_token_range == op.find_image_token_range(toks)


def _seq(prefix, n, suffix, hashes=(7,)):
    s = Sequence([1] * prefix + [IMG] * n + [2] * suffix, image_hashes=list(hashes))
    return s


def test_block_manager_partial_decision_and_refcounts():
    bm = BlockManager(num_blocks=64, block_size=256, recompute_ratio=0.1)
    a = _seq(40, 1024, 10)
    assert not bm.try_partial_recompute(a)            # registry miss
    bm.allocate(a)
    a.find_image_token_range(IMG)
    a.set_rope_starts([(40, 40, 40)])
    bm.store_image_kv(a)
    img_blocks = a.block_table[40 // 256:(40 + 1024 - 1) // 256 + 1]
    assert all(bm.ref_count(b) == 2 for b in img_blocks)
    b = _seq(128, 1024, 64)
    assert bm.try_partial_recompute(b)
    assert b.num_recompute_tokens == op.recompute_count(0.1, 1024) == 103
    entry = bm.get_image_kv_entry(7)
    assert (entry.img_start, entry.img_end, entry.rope_start) == (40, 1064, (40, 40, 40))
    c = _seq(10, 1000, 5)                               # different image size: no reuse
    assert not bm.try_partial_recompute(c)
    # the image blocks outlive the source sequence
    bm.deallocate(a)
    assert all(bm.ref_count(x) == 1 for x in img_blocks)
    free_before = bm.num_free_blocks
    assert bm.release_image(7) and not bm.release_image(7)
    assert bm.num_free_blocks == free_before + len(img_blocks)
    assert bm.free_block_ids()[-len(img_blocks):] == img_blocks


def test_config_from_dict_and_directory(tmp_path):
    import json

    cfg = Config(dict(QWEN25_VL_3B), recompute_ratio=0.1)
    assert cfg.use_mrope and cfg.hf_config.head_dim == 128 and cfg.eos == 151645
    nested = {"architectures": ["Qwen2_5_VLForConditionalGeneration"], "image_token_id": 151655,
              "vision_config": {"spatial_merge_size": 2},
              "text_config": {k: v for k, v in QWEN25_VL_3B.items() if k not in ("architectures", "image_token_id")}}
    (tmp_path / "config.json").write_text(json.dumps(nested))
    hf = load_model_config(str(tmp_path))
    assert hf.num_hidden_layers == 36 and hf.num_key_value_heads == 2 and hf.spatial_merge_size == 2
    flat = Config(str(tmp_path), use_mrope=False)
    assert flat.use_mrope is False and flat.hf_config.rope_scaling is None
    with pytest.raises(AssertionError):
        Config(dict(QWEN25_VL_3B), tensor_parallel_size=2)


# ----------------------------------------------------------------------------- several images per prompt
def _multi(parts, hashes):
    """Prompt of ("text", n) / ("image", n) parts; returns (Sequence, image token ranges)."""
    toks, ranges, p = [], [], 0
    for kind, n in parts:
        toks += ([IMG] if kind == "image" else [1]) * n
        if kind == "image":
            ranges.append((p, p + n))
        p += n
    return Sequence(toks, image_hashes=list(hashes)), ranges


def test_sequence_image_ranges_and_runs_match_oracle():
    rng = np.random.default_rng(5)
    for _ in range(50):
        k = int(rng.integers(1, 4))
        parts = [("text", int(rng.integers(1, 40)))]
        for _ in range(k):
            parts += [("image", int(rng.integers(1, 300))), ("text", int(rng.integers(0, 40)))]
        parts = [x for x in parts if x[1] > 0]
        seq, ranges = _multi(parts, range(k))
        seq.find_image_token_range(IMG)
        # adjacent images with no text between form one run
        merged = []
        for s, e in ranges:
            if merged and merged[-1][1] == s:
                merged[-1] = (merged[-1][0], e)
            else:
                merged.append((s, e))
        assert seq.image_ranges == merged
        rec = [None if rng.random() < 0.3 else op.recompute_count(0.1, e - s) for s, e in merged]
        seq.image_recompute = rec
        runs = op.computed_runs(len(seq), [r for r, x in zip(merged, rec) if x is not None],
                                [x for x in rec if x is not None])
        assert seq.computed_runs() == runs
        assert seq.num_reused_tokens == len(seq) - sum(b - a for a, b in runs)


def test_two_images_known_answer_runs():
    # 7B two-image request: 64 text + 2691 image + 64 text + 10549 image + 64 text
    seq, ranges = _multi([("text", 64), ("image", 2691), ("text", 64), ("image", 10549), ("text", 64)], [1, 2])
    seq.find_image_token_range(IMG)
    seq.image_recompute = [op.recompute_count(0.02, 2691), op.recompute_count(0.02, 10549)]
    assert seq.image_recompute == [54, 211]
    assert seq.computed_runs() == [(0, 118), (2755, 3030), (13368, 13432)]


def test_block_manager_per_image_decision_registry_and_budget():
    bm = BlockManager(num_blocks=128, block_size=256, recompute_ratio=0.1)
    a, _ = _multi([("text", 40), ("image", 1024), ("text", 10), ("image", 300), ("text", 5)], [7, 8])
    assert not bm.try_partial_recompute(a)            # registry miss for both
    bm.allocate(a)
    a.find_image_token_range(IMG)
    a.set_rope_starts([(40, 40, 40), (90, 90, 90)])
    bm.store_image_kv(a)
    e7, e8 = bm.get_image_kv_entry(7), bm.get_image_kv_entry(8)
    assert (e7.img_start, e7.img_end, e7.rope_start) == (40, 1064, (40, 40, 40))
    assert (e8.img_start, e8.img_end, e8.rope_start) == (1074, 1374, (90, 90, 90))
    # a new prompt: image 8 (same size) first, an unknown image 9 second
    b, _ = _multi([("text", 7), ("image", 300), ("text", 3), ("image", 50), ("text", 2)], [8, 9])
    assert bm.try_partial_recompute(b)
    assert b.image_recompute == [op.recompute_count(0.1, 300), None]
    assert b.num_reused_tokens == 300 - 30
    assert b.computed_runs() == [(0, 37), (307, len(b))]
    # image 7 with another token count is not reused
    c, _ = _multi([("text", 3), ("image", 1000)], [7])
    assert not bm.try_partial_recompute(c)
    # the scheduler charges only the computed tokens
    from vlcache_amd.engine.scheduler import Scheduler

    budget = len(b) - b.num_reused_tokens
    cfg = Config(dict(QWEN25_VL_3B, image_token_id=IMG), recompute_ratio=0.1, num_kvcache_blocks=128,
                 max_num_batched_tokens=budget, max_model_len=budget)
    sch = Scheduler(cfg)
    sch.block_manager = bm
    sch.image_token_id = IMG
    b.reset_partial_recompute()
    sch.add(b)
    seqs, is_prefill = sch.schedule()
    assert is_prefill and seqs == [b] and b.is_partial_recompute


def test_image_kv_copy_plan_matches_oracle_slots():
    from vlcache_amd.engine.llm_engine import image_kv_copy_plan

    bm = BlockManager(num_blocks=128, block_size=256, recompute_ratio=0.05)
    src, _ = _multi([("text", 64), ("image", 2691), ("text", 64), ("image", 700), ("text", 9)], [11, 12])
    bm.allocate(src)
    src.find_image_token_range(IMG)
    src.set_rope_starts([(64, 64, 64), (200, 200, 200)])
    bm.store_image_kv(src)
    dst, ranges = _multi([("text", 100), ("image", 700), ("text", 30), ("image", 2691), ("text", 64)], [12, 11])
    assert bm.try_partial_recompute(dst)
    bm.allocate(dst)
    dst.set_rope_starts([(100, 100, 100), (180, 180, 180)])
    old, new, deltas, seg = image_kv_copy_plan([dst], bm)
    exp_old, exp_new, exp_seg = [], [], []
    for k, ((s, e), h) in enumerate(zip(ranges, [12, 11])):
        entry = bm.get_image_kv_entry(h)
        R = op.recompute_count(0.05, e - s)
        o, n = op.image_kv_copy_slots(entry.block_table, entry.img_start, dst.block_table, s, e, R)
        exp_old += list(o)
        exp_new += list(n)
        exp_seg += [k] * len(o)
    assert old.tolist() == exp_old and new.tolist() == exp_new and seg.tolist() == exp_seg
    assert deltas == [[100 - 200] * 3, [180 - 64] * 3]


# ----------------------------------------------------------------------------- pool and scheduler vs the oracle
def _run_oracle(reqs, num_blocks, max_seqs, budget):
    from oracle import engine as oe

    sch = oe.Scheduler(num_blocks, 256, max_seqs, budget)
    seqs = [oe.Seq(i, p, m) for i, (p, m) in enumerate(reqs)]
    sch.waiting.extend(seqs)
    steps = []
    while sch.waiting or sch.running:
        batch, prefill = sch.schedule()
        steps.append(([s.seq_id for s in batch], prefill, [list(s.block_table) for s in batch]))
        sch.postprocess(batch)
        assert len(steps) < 10000
    return steps


def _run_product(reqs, num_blocks, max_seqs, budget):
    from vlcache_amd import SamplingParams
    from vlcache_amd.engine.scheduler import Scheduler

    cfg = Config(dict(QWEN25_VL_3B), num_kvcache_blocks=num_blocks, max_num_seqs=max_seqs,
                 max_num_batched_tokens=budget, max_model_len=budget)
    sch = Scheduler(cfg)
    seqs = [Sequence([5] * p, SamplingParams(max_tokens=m, ignore_eos=True)) for p, m in reqs]
    index = {s.seq_id: i for i, s in enumerate(seqs)}
    for s in seqs:
        sch.add(s)
    steps = []
    while not sch.is_finished():
        batch, prefill = sch.schedule()
        steps.append(([index[s.seq_id] for s in batch], prefill, [list(s.block_table) for s in batch]))
        sch.postprocess(batch, [7] * len(batch))
        assert len(steps) < 10000
    assert sch.block_manager.num_free_blocks == num_blocks and not sch.block_manager.ref_counts.any()
    return steps


def test_oracle_scheduler_known_answer():
    # 3 blocks; A and B: 256-token prompts, 3 new tokens each.  Hand-derived:
    # prefill [A, B] (1 block each); decode: A opens a block, B finds none and, being the
    # last left, preempts itself; decode [A]; A finishes; B is prefilled again (257
    # tokens, 2 blocks); decode [B] finishes it.
    steps = _run_oracle([(256, 3), (256, 3)], 3, 8, 4096)
    assert [(ids, pf) for ids, pf, _ in steps] == [([0, 1], True), ([0], False), ([0], False), ([1], True),
                                                  ([1], False)]
    assert steps[0][2] == [[0], [1]] and steps[1][2] == [[0, 2]]
    # freed blocks come back in release order: B's 1, then A's table last to first (2, 0)
    assert steps[3][2] == [[1, 2]]


def test_scheduler_matches_oracle_known_answer():
    assert _run_product([(256, 3), (256, 3)], 3, 8, 4096) == _run_oracle([(256, 3), (256, 3)], 3, 8, 4096)


@pytest.mark.parametrize("seed", range(25))
def test_scheduler_matches_oracle_random(seed):
    """Random request mixes under tight pools (preemption), small batch caps and budgets:
    every step's batch, kind and block tables equal the reference's loop."""
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 9))
    reqs = [(int(rng.integers(1, 900)), int(rng.integers(1, 300))) for _ in range(n)]
    need = max(-(-(p + m) // 256) for p, m in reqs)
    num_blocks = int(rng.integers(need, need + 8))
    max_seqs = int(rng.integers(1, 6))
    budget = int(rng.integers(max(p for p, _ in reqs) + 300, 4096))
    o = _run_oracle(reqs, num_blocks, max_seqs, budget)
    p = _run_product(reqs, num_blocks, max_seqs, budget)
    assert p == o


def test_pool_ring_wraps_and_refuses_overdraw():
    bm = BlockManager(num_blocks=4, block_size=256)
    s1, s2 = Sequence([1] * 700), Sequence([1] * 200)
    bm.allocate(s1)
    bm.allocate(s2)
    assert s1.block_table == [0, 1, 2] and s2.block_table == [3] and bm.num_free_blocks == 0
    bm.deallocate(s1)
    assert bm.free_block_ids() == [2, 1, 0]
    s3 = Sequence([1] * 300)
    bm.allocate(s3)
    assert s3.block_table == [2, 1] and bm.free_block_ids() == [0]
    with pytest.raises(RuntimeError):
        bm.allocate(Sequence([1] * 600))
    bm.deallocate(s2)
    bm.deallocate(s3)
    assert bm.free_block_ids() == [0, 3, 1, 2] and not bm.ref_counts.any()


# ----------------------------------------------------------------------------- positions after preemption
def test_positions_continue_past_the_prompt_after_preemption():
    """A prompt with an image, 5 generated tokens, then a preemption: the prefill of all
    len(seq) tokens gets one position column per token; past the prompt index p sits at
    p + rope_delta on every row (the decode rule), so the columns continue the prompt's."""
    toks = [1] * 5 + [IMG] * 15 + [2] * 3
    seq = Sequence(toks)
    pos, starts, delta = mrope_positions(toks, [(1, 6, 10)], IMG)
    seq.rope_positions, seq.rope_delta = pos, delta
    for t in range(5):
        seq.append_token(100 + t)
    got = seq.positions(0, len(seq), True)
    assert got.shape == (3, len(seq))
    assert np.array_equal(got[:, :len(toks)], pos)
    tail = np.arange(len(toks), len(seq)) + delta
    assert np.array_equal(got[:, len(toks):], np.tile(tail, (3, 1)))
    assert tail[0] == pos.max() + 1  # the first generated token follows the prompt's last position
    assert np.array_equal(seq.positions(20, 26, False), np.concatenate([pos[0, 20:23], tail[:3]]))
    # through the scheduler: prefill, 5 decode tokens, preemption, prefill again
    from vlcache_amd import SamplingParams
    from vlcache_amd.engine.scheduler import Scheduler

    cfg = Config(dict(QWEN25_VL_3B, image_token_id=IMG), num_kvcache_blocks=4, max_model_len=4096)
    sch = Scheduler(cfg)
    s = Sequence(toks, SamplingParams(max_tokens=50, ignore_eos=True))
    s.rope_positions, s.rope_delta = pos, delta
    sch.add(s)
    sch.schedule()
    sch.postprocess([s], [9])
    for _ in range(4):
        batch, prefill = sch.schedule()
        assert not prefill
        sch.postprocess(batch, [9])
    sch.preempt(s)
    batch, prefill = sch.schedule()
    assert prefill and batch == [s] and s.computed_runs() == [(0, len(s))]
    assert s.positions(0, len(s), True).shape == (3, len(toks) + 5)


# ----------------------------------------------------------------------------- encoder cache
def test_encoder_cache_lru_views_and_limits():
    import torch

    from vlcache_amd.engine.encoder_cache import EncoderCache

    ec = EncoderCache(num_pages=6, page_rows=4, hidden=3, dtype=torch.float32, device="cpu")
    a = torch.arange(10 * 3, dtype=torch.float32).view(10, 3)  # 3 pages
    b = -torch.arange(5 * 3, dtype=torch.float32).view(5, 3)   # 2 pages
    assert ec.put(1, a) and ec.put(2, b) and ec.free_pages == 1
    got = ec.get(1, 6)
    assert torch.equal(got, a[:6]) and got.data_ptr() == ec.pool.data_ptr()  # a view, no gather
    assert torch.equal(ec.get(2), b)
    c = torch.ones(7, 3)                                       # 2 pages: evicts the least recent (1)
    assert ec.put(3, c) and 1 not in ec and 2 in ec and ec.evictions == 1
    assert ec.get(1) is None and ec.misses == 1
    d = torch.full((4, 3), 5.0)                                # 1 page, fits without eviction
    assert ec.put(4, d)
    # entry 3 took pages 0, 1 (freed by 1) and entry 4 page 2: a read of 3 is a view again
    assert torch.equal(ec.get(3), c)
    ec2 = EncoderCache(num_pages=4, page_rows=2, hidden=1, dtype=torch.float32, device="cpu")
    ec2.put(1, torch.zeros(2, 1))
    ec2.put(2, torch.ones(2, 1))
    ec2.put(3, torch.full((2, 1), 2.0))
    ec2.get(1)
    ec2.put(4, torch.full((4, 1), 3.0))   # needs 2 pages, 1 free: evicts 2, the least recent
    assert sorted(k for k in (1, 2, 3, 4) if k in ec2) == [1, 3, 4] and ec2.evictions == 1
    ec2._free[:] = True
    ec2._entries.clear()
    ec2._last_use.clear()
    ec2.put(5, torch.zeros(2, 1))         # page 0
    ec2.put(6, torch.zeros(2, 1))         # page 1
    ec2.put(7, torch.zeros(2, 1))         # page 2
    ec2._free[1] = True                   # a hole: 8 lands on pages 1 and 3 (a gather to read)
    del ec2._entries[6], ec2._last_use[6]
    e = torch.tensor([[1.0], [2.0], [3.0], [4.0]])
    assert ec2.put(8, e) and torch.equal(ec2.get(8), e) and torch.equal(ec2.get(8, 3), e[:3])
    assert not ec2.put(9, torch.zeros(9, 1))  # larger than the pool: not cached


def test_process_visual_hits_survive_evictions_by_the_same_step():
    """A step reads image A from the cache (a view of the pool) and then stores the
    miss B, which evicts A and reuses its pages.  A's rows in the step's embeddings
    must still be A's: the reference's read gathers a copy
    (engine/encoder_cache_manager.py:59-62)."""
    from types import SimpleNamespace

    from vlcache_amd.engine.encoder_cache import EncoderCache
    from vlcache_amd.engine.model_runner import ModelRunner

    hidden = 3
    ec = EncoderCache(num_pages=2, page_rows=2, hidden=hidden, dtype=torch.float32, device="cpu")
    a = torch.arange(4 * hidden, dtype=torch.float32).view(4, hidden) + 1.0  # grid (1, 4, 4): 4 rows
    b = torch.full((4, hidden), -7.0)
    assert ec.put(11, a)
    cfg = SimpleNamespace(hf_config=SimpleNamespace(hidden_size=hidden, spatial_merge_size=2),
                          synthetic_vision=False)
    stub = SimpleNamespace(encoder_cache=ec, config=cfg, dtype=torch.float32, device=torch.device("cpu"),
                           model=SimpleNamespace(visual=None))
    stub._num_units = lambda grid: ModelRunner._num_units(stub, grid)
    mm = dict(image_hashes=[11, 22], image_grid_thw=[(1, 4, 4), (1, 4, 4)], image_embeds=[None, b],
              pixel_values=[None, None], recompute=[3, 0])
    out, vit = ModelRunner._process_visual(stub, mm)
    assert vit == 0.0 and ec.hits == 1 and 11 not in ec and 22 in ec and ec.evictions == 1
    assert torch.equal(out[:3], a[:3]), "the hit's rows were overwritten by the same step's put"
    assert torch.equal(out[3:], b)
    # the evicted image's pages now hold B
    assert torch.equal(ec.get(22), b)


def test_runner_refuses_token_ids_outside_the_vocabulary():
    from types import SimpleNamespace

    from vlcache_amd.engine.model_runner import ModelRunner

    stub = SimpleNamespace(config=SimpleNamespace(hf_config=SimpleNamespace(vocab_size=1000)))
    assert ModelRunner._checked_ids(stub, np.array([0, 5, 999])).tolist() == [0, 5, 999]
    for bad in ([1, 151655], [-1, 3]):
        with pytest.raises(ValueError, match="outside the vocabulary"):
            ModelRunner._checked_ids(stub, np.array(bad))


def test_image_hash_is_the_reference_digest():
    """xxh64 over the grid's bytes then the pixel values' bytes, as
    EncoderCacheManager.compute_hash (engine/encoder_cache_manager.py:25-29) computes it
    from numpy's tobytes(); bf16 pixels hash their raw bytes."""
    import xxhash

    from vlcache_amd.engine.llm_engine import image_hash

    pv = torch.randn(96, 1176, generator=torch.Generator().manual_seed(1))
    grid = torch.tensor([1, 8, 12])
    h = xxhash.xxh64()
    h.update(grid.numpy().tobytes())
    h.update(pv.numpy().tobytes())
    assert image_hash(pv, grid) == h.intdigest()
    assert image_hash(pv[:48], grid) != image_hash(pv[48:], grid)
    b = pv.to(torch.bfloat16)
    h2 = xxhash.xxh64()
    h2.update(grid.numpy().tobytes())
    h2.update(b.view(torch.int16).numpy().tobytes())
    assert image_hash(b, grid) == h2.intdigest()


def test_packed_host_to_device_copy_keeps_every_array():
    """One buffer, one copy: each array comes back with its values, dtype and shape,
    at a 16-byte aligned offset, whatever the mix of sizes (empty ones included)."""
    from vlcache_amd.engine.model_runner import _h2d_many

    rng = np.random.default_rng(3)
    arrays = [
        (rng.integers(-2**40, 2**40, 9494), np.int64),
        (rng.integers(0, 2**31 - 1, (3, 7)), np.int64),
        (np.array([0, 1183, 1247]), np.int32),
        (np.zeros(0), np.int32),
        (np.full((2, 5), -1), np.int32),
        (rng.standard_normal((1, 64, 2)).astype(np.float32), np.float32),
        (rng.integers(0, 100, 3), np.int32),
    ]
    out = _h2d_many("cpu", *arrays)
    assert len(out) == len(arrays)
    base = out[0].untyped_storage().data_ptr()
    for (a, dt), t in zip(arrays, out):
        want = np.asarray(a, dtype=dt)
        assert t.dtype == {np.int64: torch.int64, np.int32: torch.int32, np.float32: torch.float32}[dt]
        assert tuple(t.shape) == want.shape and t.is_contiguous()
        assert np.array_equal(t.numpy(), want)
        assert (t.data_ptr() - base) % 16 == 0


def test_registry_releases_least_recently_used_images_when_a_request_does_not_fit():
    """A request that does not fit the free blocks releases registered images, oldest use
    first, but never one that a request of the same step copies from."""
    from vlcache_amd.engine.scheduler import Scheduler

    cfg = Config(dict(QWEN25_VL_3B, image_token_id=IMG), recompute_ratio=0.1, num_kvcache_blocks=8,
                 max_num_batched_tokens=4096, max_model_len=4096)
    sch = Scheduler(cfg)
    sch.image_token_id = IMG
    bm = sch.block_manager
    for h in (1, 2):  # two prefilled, finished requests: their images pin 2 blocks each
        s, _ = _multi([("text", 10), ("image", 500)], [h])
        bm.allocate(s)
        s.find_image_token_range(IMG)
        bm.store_image_kv(s)
        bm.deallocate(s)
    assert bm.num_free_blocks == 4
    probe, _ = _multi([("text", 5), ("image", 500)], [1])
    assert bm.try_partial_recompute(probe, IMG)  # image 1 is now the most recently used
    # 1210 tokens need 5 blocks: the least recently used image (2) is released, image 1 stays
    c, _ = _multi([("text", 10), ("image", 1200)], [3])
    sch.add(c)
    seqs, is_prefill = sch.schedule()
    assert is_prefill and seqs == [c]
    assert bm.get_image_kv_entry(2) is None and bm.get_image_kv_entry(1) is not None
    assert bm.num_free_blocks == 1
    # a request that reuses image 1 needs 2 blocks; the only entry left is the one it copies
    # from, so nothing is released and it waits (the step decodes c instead)
    d, _ = _multi([("text", 10), ("image", 500)], [1])
    sch.add(d)
    seqs, is_prefill = sch.schedule()
    assert not is_prefill and seqs == [c]
    assert bm.get_image_kv_entry(1) is not None and not d.is_partial_recompute
    assert bm.evict_images(100) == 1 and bm.num_free_blocks == 3 and not bm.image_kv_cache


def test_visual_rows_count_is_checked_on_the_host():
    """With image_rows the model places the visual embeddings with index_copy_ (no
    device-to-host sync); a count mismatch raises before any kernel runs."""
    from vlcache_amd.qwen_vl import Qwen2_5_VLForConditionalGeneration

    tiny = dict(hidden_size=64, intermediate_size=128, num_hidden_layers=1, num_attention_heads=4,
                num_key_value_heads=2, vocab_size=100, rms_norm_eps=1e-6, rope_theta=1e6, head_dim=16,
                max_position_embeddings=256, tie_word_embeddings=True, image_token_id=7, torch_dtype="float32")
    model = Qwen2_5_VLForConditionalGeneration(load_model_config(tiny))
    ids = torch.tensor([1, 7, 7, 2])
    with pytest.raises(ValueError, match="2 image tokens, 3 visual rows"):
        model(ids, torch.arange(4), torch.zeros(3, 64), torch.tensor([1, 2]))
