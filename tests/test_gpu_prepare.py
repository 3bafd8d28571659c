"""ModelRunner.prepare_prefill's integer outputs, element by element, against the oracle.

The oracle (oracle/prefill.py::prepare_prefill) restates engine/model_runner.py:194-320
of the reference.  Sequences are scheduled by the engine's own scheduler and
block manager (a cold request registers the image KV without running the model;
the warm requests then reuse it), in the reference's 1-D positions mode:

* the small warm request (64 text + 1024 image + 32 text, ratio 0.1);
* the 4K-image warm request (128 + 10549 + 64, ratio 0.1);
* a mixed batch: two warm requests with different prefixes and a text-only prompt.

Compared: input_ids, positions, cu_seqlens_q/k, max_seqlen_q/k, slot_mapping,
block_tables and the logit indices.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import prefill as op
from tests._util import say
from vlcache_amd import SamplingParams
from vlcache_amd.utils.context import get_context, reset_context

pytestmark = pytest.mark.gpu

IMG = 151655
# vocab_size covers the image token id: the model embeds every prompt id before the image
# rows are replaced by visual embeddings.
SMALL = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=1, num_attention_heads=2,
             num_key_value_heads=1, vocab_size=151936, rms_norm_eps=1e-6, rope_theta=1e6,
             rope_scaling={"type": "mrope", "mrope_section": [16, 24, 24]}, max_position_embeddings=32768,
             tie_word_embeddings=True, image_token_id=IMG, spatial_merge_size=2, eos_token_id=0,
             torch_dtype="bfloat16", head_dim=128)


def _engine(ratio, blocks):
    from vlcache_amd import LLM

    return LLM(dict(SMALL), recompute_ratio=ratio, num_kvcache_blocks=blocks, max_model_len=16384,
               max_num_batched_tokens=65536, use_mrope=False, enforce_eager=True)


def _prompt(prefix, grid, suffix, seed):
    t, h, w = grid
    rng = np.random.default_rng(seed)
    toks = ([int(x) for x in rng.integers(1, 900, prefix)] + [IMG] * (t * (h // 2) * (w // 2))
            + [int(x) for x in rng.integers(1, 900, suffix)])
    pv = torch.linspace(0, 1, t * h * w)[:, None]  # stands in for pixel patches; only hashed
    return toks, {"pixel_values": pv, "image_grid_thw": torch.tensor([list(grid)])}


def _register_image(engine, prefix, grid, seed):
    """A cold request scheduled and registered as the image-KV source (no model run)."""
    toks, mm = _prompt(prefix, grid, 8, seed)
    seq = engine.add_request(toks, SamplingParams(max_tokens=1), mm)
    seqs, is_prefill = engine.scheduler.schedule()
    assert is_prefill and seqs == [seq]
    engine._store_image_kv(seqs)
    engine.scheduler.running.remove(seq)  # its blocks stay allocated, as mid-generation
    return mm


def _spec(seq):
    return op.SeqSpec(list(seq.token_ids), list(seq.block_table), seq.is_partial_recompute,
                      seq.image_token_range if seq.is_partial_recompute else None, seq.num_recompute_tokens)


def _check(engine, seqs):
    runner = engine.model_runner
    ids, pos, _ = runner.prepare_prefill(seqs)
    ctx = get_context()
    exp = op.prepare_prefill([_spec(s) for s in seqs])
    try:
        assert ids.dtype == torch.int64 and ids.cpu().tolist() == exp.input_ids
        assert pos.dtype == torch.int64 and pos.dim() == 1 and pos.cpu().tolist() == exp.positions
        assert ctx.cu_seqlens_q.dtype == torch.int32 and ctx.cu_seqlens_q.cpu().tolist() == exp.cu_seqlens_q
        assert ctx.cu_seqlens_k.dtype == torch.int32 and ctx.cu_seqlens_k.cpu().tolist() == exp.cu_seqlens_k
        assert (ctx.max_seqlen_q, ctx.max_seqlen_k) == (exp.max_seqlen_q, exp.max_seqlen_k)
        assert ctx.slot_mapping.dtype == torch.int32 and ctx.slot_mapping.cpu().tolist() == exp.slot_mapping
        if exp.block_tables is None:
            assert ctx.block_tables is None
        else:
            assert ctx.block_tables.dtype == torch.int32 and ctx.block_tables.cpu().tolist() == exp.block_tables
        assert runner._logit_indices == exp.logit_indices
        assert list(ctx.cu_seqlens_q_host) == exp.cu_seqlens_q and list(ctx.cu_seqlens_k_host) == exp.cu_seqlens_k
    finally:
        reset_context()
    return exp


def test_prepare_prefill_small_warm_request(dev):
    say("prepare_prefill: 64 + 1024 + 32 warm request, ratio 0.1, 1-D positions, vs oracle")
    eng = _engine(0.1, 32)
    mm = _register_image(eng, 16, (1, 64, 64), seed=0)
    toks, _ = _prompt(64, (1, 64, 64), 32, seed=1)
    seq = eng.add_request(toks, SamplingParams(max_tokens=1), mm)
    seqs, _ = eng.scheduler.schedule()
    assert seqs == [seq] and seq.is_partial_recompute and seq.num_recompute_tokens == 103
    exp = _check(eng, seqs)
    assert exp.cu_seqlens_q == [0, 167, 199] and exp.cu_seqlens_k == [0, 167, 1287]
    assert exp.logit_indices == [1]


def test_prepare_prefill_4k_warm_request(dev):
    say("prepare_prefill: 128 + 10549 + 64 warm request, ratio 0.1, vs oracle")
    eng = _engine(0.1, 100)
    mm = _register_image(eng, 40, (1, 154, 274), seed=2)
    toks, _ = _prompt(128, (1, 154, 274), 64, seed=3)
    seq = eng.add_request(toks, SamplingParams(max_tokens=1), mm)
    seqs, _ = eng.scheduler.schedule()
    assert seq.is_partial_recompute and seq.num_recompute_tokens == 1055
    exp = _check(eng, seqs)
    assert exp.cu_seqlens_q == [0, 1183, 1247] and exp.cu_seqlens_k == [0, 1183, 11924]
    assert len(exp.block_tables) == 2 and len(exp.block_tables[0]) == 42


def test_prepare_prefill_mixed_batch(dev):
    say("prepare_prefill: mixed batch (warm, text-only, warm with another prefix), vs oracle")
    eng = _engine(0.07, 64)
    mm = _register_image(eng, 30, (1, 40, 40), seed=4)  # 400 image tokens
    # R = ceil(0.07 * 400) in IEEE double: 0.07 * 400 = 28.000000000000004, so R = 29
    seqs_in = []
    t1, _ = _prompt(50, (1, 40, 40), 20, seed=5)
    seqs_in.append(eng.add_request(t1, SamplingParams(max_tokens=1), mm))
    t2 = [int(x) for x in np.random.default_rng(6).integers(1, 900, 300)]
    seqs_in.append(eng.add_request(t2, SamplingParams(max_tokens=1)))
    t3, _ = _prompt(7, (1, 40, 40), 3, seed=7)
    seqs_in.append(eng.add_request(t3, SamplingParams(max_tokens=1), mm))
    seqs, _ = eng.scheduler.schedule()
    assert seqs == seqs_in
    assert [s.is_partial_recompute for s in seqs] == [True, False, True]
    assert seqs[0].num_recompute_tokens == op.recompute_count(0.07, 400) == 29
    exp = _check(eng, seqs)
    assert exp.logit_indices == [1, 2, 4]
    assert len(exp.block_tables) == 5  # the text-only prompt reads the paged cache too


def test_prepare_prefill_after_preemption_mrope(dev):
    """An image prompt in M-RoPE mode, five decoded tokens, a preemption, then the prefill
    of all its tokens again: one position column per token, the prompt's rows followed by
    index + rope_delta on every row."""
    from vlcache_amd import LLM
    from vlcache_amd.engine.positions import mrope_positions

    say("prepare_prefill: M-RoPE prompt with an image, preempted after 5 decode steps, prefilled again")
    eng = LLM(dict(SMALL), recompute_ratio=0.0, num_kvcache_blocks=8, max_model_len=4096, enforce_eager=True)
    toks, mm = _prompt(20, (1, 12, 16), 9, seed=8)
    seq = eng.add_request(toks, SamplingParams(max_tokens=50, ignore_eos=True), mm)
    sch = eng.scheduler
    sch.schedule()
    sch.postprocess([seq], [11])
    for _ in range(4):
        batch, prefill = sch.schedule()
        assert not prefill
        sch.postprocess(batch, [11])
    sch.preempt(seq)
    seqs, prefill = sch.schedule()
    assert prefill and seqs == [seq] and len(seq) == len(toks) + 5
    _, pos, _ = eng.model_runner.prepare_prefill(seqs)
    reset_context()
    pos = pos.cpu().numpy()
    ref, _, delta = mrope_positions(toks, [(1, 12, 16)], IMG, 2)
    assert pos.shape == (3, len(seq))
    assert (pos[:, :len(toks)] == ref).all()
    assert (pos[:, len(toks):] == np.arange(len(toks), len(seq)) + delta).all()


def test_encoder_cache_miss_without_embeddings_raises(dev):
    """The vision tower is not part of this path: a cold image with no image_embeds and no
    synthetic opt-in is an error, not silently made-up embeddings."""
    say("engine: encoder-cache miss without image_embeds raises")
    from vlcache_amd import LLM

    eng = LLM(dict(SMALL), recompute_ratio=0.1, num_kvcache_blocks=8, max_model_len=4096, enforce_eager=True)
    toks, mm = _prompt(10, (1, 8, 8), 4, seed=9)
    eng.add_request(toks, SamplingParams(max_tokens=1), mm)
    with pytest.raises(RuntimeError, match="encoder cache"):
        eng.step()
    reset_context()
    # with the caller's embeddings the same request runs and fills the cache
    eng2 = LLM(dict(SMALL), recompute_ratio=0.1, num_kvcache_blocks=8, max_model_len=4096, enforce_eager=True)
    emb = torch.randn(16, SMALL["hidden_size"]).to(torch.bfloat16)
    mm2 = dict(mm, image_embeds=[emb])
    out = eng2.generate([toks], SamplingParams(max_tokens=1), [mm2])
    assert len(out) == 1 and len(eng2.model_runner.encoder_cache) == 1
    cached = eng2.model_runner.encoder_cache.get(next(iter(eng2.model_runner.encoder_cache._entries)))
    assert torch.equal(cached.cpu(), emb)


def test_token_ids_outside_the_vocabulary_are_refused(dev):
    """An id the embedding table does not have is a host-side error, raised before any
    device work."""
    say("engine: token id outside the vocabulary is refused on the host")
    from vlcache_amd import LLM

    eng = LLM(dict(SMALL, vocab_size=1000), num_kvcache_blocks=4, max_model_len=4096, enforce_eager=True)
    eng.add_request([1, 2, 5000, 3], SamplingParams(max_tokens=1))
    with pytest.raises(ValueError, match="outside the vocabulary"):
        eng.step()
    reset_context()
