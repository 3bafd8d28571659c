"""CPU tests of the host engine logic against the oracle and hand-derived answers."""
from __future__ import annotations

import numpy as np
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
    a.image_rope_start = (40, 40, 40)
    bm.store_image_kv(a)
    img_blocks = a.block_table[40 // 256:(40 + 1024 - 1) // 256 + 1]
    assert all(bm.blocks[b].ref_count == 2 for b in img_blocks)
    b = _seq(128, 1024, 64)
    assert bm.try_partial_recompute(b)
    assert b.num_recompute_tokens == op.recompute_count(0.1, 1024) == 103
    entry = bm.get_image_kv_entry(7)
    assert (entry.img_start, entry.img_end, entry.rope_start) == (40, 1064, (40, 40, 40))
    c = _seq(10, 1000, 5)                               # different image size: no reuse
    assert not bm.try_partial_recompute(c)
    # the image blocks outlive the source sequence
    bm.deallocate(a)
    assert all(bm.blocks[x].ref_count == 1 for x in img_blocks)
    free_before = len(bm.free_block_ids)
    bm._release_image_blocks(entry)
    assert len(bm.free_block_ids) == free_before + len(img_blocks)


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
    a.image_rope_starts = [(40, 40, 40), (90, 90, 90)]
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
    src.image_rope_starts = [(64, 64, 64), (200, 200, 200)]
    bm.store_image_kv(src)
    dst, ranges = _multi([("text", 100), ("image", 700), ("text", 30), ("image", 2691), ("text", 64)], [12, 11])
    assert bm.try_partial_recompute(dst)
    bm.allocate(dst)
    dst.image_rope_starts = [(100, 100, 100), (180, 180, 180)]
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
