"""Pins the integer oracle (oracle/prefill.py) with hand-derived known answers and invariants.

Known answers are derived by hand from the reference lines each function cites
(engine/block_manager.py:72, engine/sequence.py:91-100,
engine/model_runner.py:160-168,194-320, engine/llm_engine.py:70-88); none is
computed by the function under test.
"""
from __future__ import annotations

import math

import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import prefill as op

IMG = op.IMAGE_TOKEN_ID


def test_recompute_count_known_answers():
    assert op.recompute_count(0.1, 1024) == 103      # ceil(102.4)
    assert op.recompute_count(0.1, 10549) == 1055    # ceil(1054.9)
    assert op.recompute_count(0.05, 10549) == 528    # ceil(527.45)
    assert op.recompute_count(0.02, 2691) == 54      # ceil(53.82)
    assert op.recompute_count(0.02, 10549) == 211    # ceil(210.98)
    assert op.recompute_count(0.0, 10549) == 0
    assert op.recompute_count(1.0, 10549) == 10549
    # IEEE double: 0.07 * 100 = 7.000000000000001, so the reference recomputes 8 tokens
    assert 0.07 * 100 > 7 and op.recompute_count(0.07, 100) == 8


def test_find_image_token_range():
    assert op.find_image_token_range([1, 2, 3]) is None
    assert op.find_image_token_range([IMG]) == (0, 1)
    assert op.find_image_token_range([5, IMG, IMG, 7]) == (1, 3)
    # spans first to last image token, gaps included (single-image assumption)
    assert op.find_image_token_range([IMG, 1, IMG, 2]) == (0, 3)


def test_compute_slots_known_answer():
    bt = [5, 2, 9]
    assert op.compute_slots(bt, 0, 1) == [5 * 256]
    assert op.compute_slots(bt, 255, 257) == [5 * 256 + 255, 2 * 256]
    assert op.compute_slots(bt, 600, 601) == [9 * 256 + 88]
    assert op.compute_slots([3], 0, 2, block_size=2) == [6, 7]
    with pytest.raises(IndexError):  # position 2 needs a second block
        op.compute_slots([3], 0, 3, block_size=2)


def test_image_kv_copy_slots_cfg1():
    # cached entry: image [16, 1040) in blocks [10..14]; new seq: image [64, 1088) in blocks [0..4]
    entry_bt = [10, 11, 12, 13, 14]
    seq_bt = [0, 1, 2, 3, 4]
    R = 103
    old, new = op.image_kv_copy_slots(entry_bt, 16, seq_bt, 64, 1088, R)
    assert len(old) == len(new) == 1024 - 103 == 921
    # first reused token p = 167: old_p = 16 + 103 = 119 -> block 10, offset 119
    assert old[0] == 10 * 256 + 119 and new[0] == 167
    # last reused token p = 1087: old_p = 16 + 1023 = 1039 -> block index 4 (14), offset 15
    assert old[-1] == 14 * 256 + 15 and new[-1] == 4 * 256 + 63


def _warm_seq(prefix, n_img, suffix, ratio, bt):
    toks = [1] * prefix + [IMG] * n_img + [2] * suffix
    rng = op.find_image_token_range(toks)
    return op.SeqSpec(toks, bt, True, rng, op.recompute_count(ratio, n_img))


def test_prepare_prefill_cfg1_known_answer():
    seq = _warm_seq(64, 1024, 32, 0.1, [7, 3, 9, 1, 4])
    pl = op.prepare_prefill([seq])
    assert pl.cu_seqlens_q == [0, 167, 199]
    assert pl.cu_seqlens_k == [0, 167, 1287]
    assert (pl.max_seqlen_q, pl.max_seqlen_k) == (167, 1120)
    assert len(pl.slot_mapping) == 199
    assert pl.slot_mapping[0] == 7 * 256 and pl.slot_mapping[166] == 7 * 256 + 166
    assert pl.slot_mapping[167] == 4 * 256 + (1088 - 1024)  # suffix token 1088 -> block 4, offset 64
    assert pl.positions[:3] == [0, 1, 2] and pl.positions[167] == 1088 and pl.positions[-1] == 1119
    assert pl.block_tables == [[7, 3, 9, 1, 4]] * 2
    assert pl.logit_indices == [1]
    assert len(pl.input_ids) == 199 and pl.input_ids.count(IMG) == 103


def test_prepare_prefill_cfg2_known_answer():
    seq = _warm_seq(128, 10549, 64, 0.1, list(range(42)))
    pl = op.prepare_prefill([seq])
    assert pl.cu_seqlens_q == [0, 1183, 1247]
    assert pl.cu_seqlens_k == [0, 1183, 11924]
    assert (pl.max_seqlen_q, pl.max_seqlen_k) == (1183, 10741)
    assert len(pl.block_tables[0]) == 42 == math.ceil(10741 / 256)


def test_prepare_prefill_mixed_and_plain_batches():
    warm = _warm_seq(10, 40, 5, 0.25, [3])
    plain = op.SeqSpec([1] * 300, [8, 6])
    pl = op.prepare_prefill([warm, plain])
    assert pl.cu_seqlens_q == [0, 20, 25, 325]
    assert pl.cu_seqlens_k == [0, 20, 75, 375]
    assert pl.block_tables == [[3, -1], [3, -1], [8, 6]]
    assert pl.logit_indices == [1, 2]
    only_plain = op.prepare_prefill([plain])
    assert only_plain.block_tables is None and only_plain.logit_indices is None
    assert only_plain.cu_seqlens_q == only_plain.cu_seqlens_k == [0, 300]


@settings(max_examples=60, deadline=None)
@given(st.lists(st.tuples(st.integers(0, 300), st.integers(1, 600), st.integers(1, 200),
                          st.sampled_from([0.0, 0.02, 0.1, 0.5, 1.0])), min_size=1, max_size=4),
       st.integers(0, 2**31 - 1))
def test_prepare_prefill_invariants(specs, seed):
    import random

    rnd = random.Random(seed)
    pool = list(range(4096))
    rnd.shuffle(pool)
    seqs = []
    for pre, n, suf, ratio in specs:
        length = pre + n + suf
        nb = -(-length // 256)
        bt = [pool.pop() for _ in range(nb)]
        s = _warm_seq(pre, n, suf, ratio, bt)
        if ratio == 0.0:
            s = op.SeqSpec(s.token_ids, bt)
        seqs.append(s)
    pl = op.prepare_prefill(seqs)
    assert len(pl.slot_mapping) == pl.cu_seqlens_q[-1] == len(pl.input_ids) == len(pl.positions)
    assert len(set(pl.slot_mapping)) == len(pl.slot_mapping)
    for b in range(len(pl.cu_seqlens_q) - 1):
        sq = pl.cu_seqlens_q[b + 1] - pl.cu_seqlens_q[b]
        sk = pl.cu_seqlens_k[b + 1] - pl.cu_seqlens_k[b]
        assert sk >= sq >= 0
    # every slot lies in its own sequence's blocks; computed + reused = all tokens
    q = 0
    for s in seqs:
        own = set(s.block_table)
        if s.is_partial_recompute:
            a, e = s.image_token_range
            n_comp = a + s.num_recompute_tokens + len(s.token_ids) - e
            reused = e - a - s.num_recompute_tokens
            assert n_comp + reused == len(s.token_ids)
        else:
            n_comp = len(s.token_ids)
        assert all(x // 256 in own for x in pl.slot_mapping[q:q + n_comp])
        q += n_comp


def test_computed_runs_reduces_to_reference_subsequences():
    # one image: runs are exactly (sub1, sub2) of prepare_prefill
    runs = op.computed_runs(1120, [(64, 1088)], [103])
    assert runs == [(0, 167), (1088, 1120)]
    # two images (Qwen2.5-VL-7B request): 64 + 2691 + 64 + 10549 + 64 tokens, R = 54 and 211
    runs = op.computed_runs(13432, [(64, 2755), (2819, 13368)], [54, 211])
    assert runs == [(0, 118), (2755, 3030), (13368, 13432)]
