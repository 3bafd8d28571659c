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
