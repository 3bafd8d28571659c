"""Request loop (engine/llm_engine.py of the reference), one GPU.

Same flow: add_request hashes each image (xxhash of grid + pixel values,
engine/encoder_cache_manager.py:24-29) before the Sequence - and with it the
TTFT clock - starts; step() schedules, copies the reused image KV of partial
sequences, runs the model, stamps TTFT after a prefill and registers the
image KV for reuse (:58-120); generate() returns
[{text, token_ids, vit_time, ttft}] (:125-167).

The reused-KV copy also re-rotates K from the cached image's rotary start to
the new one (the reference copies the keys unchanged, :75-89).  A prompt may
hold several images; each is reused or computed on its own.
"""
from __future__ import annotations

import os
from dataclasses import fields
from time import time

import numpy as np
import torch
import xxhash

from ..config import Config
from ..sampling_params import SamplingParams
from .model_runner import ModelRunner
from .positions import mrope_positions
from .scheduler import Scheduler
from .sequence import Sequence


def image_hash(pixel_values: torch.Tensor, grid_thw: torch.Tensor) -> int:
    h = xxhash.xxh64()
    h.update(grid_thw.cpu().numpy().tobytes())
    h.update(pixel_values.cpu().numpy().tobytes())
    return h.intdigest()


def image_kv_copy_plan(seqs: list[Sequence], block_manager):
    """Slots of the reused image KV of a prefill step (engine/llm_engine.py:58-89).

    For image k of a partially recomputed sequence with a registry hit, positions
    p in [start_k + R_k, end_k) take the rows of the cached entry's positions
    entry.img_start + (p - start_k).  Returns (old_slots, new_slots, deltas,
    seg_of_token) for ModelRunner.copy_image_kv - one launch for every image of
    every sequence, image k being rotation segment k with delta = its new rotary
    start - the cached one (deltas None when a rotary start is unknown) - or None
    when nothing is reused.
    """
    bs = block_manager.block_size
    olds, news, segs, deltas = [], [], [], []
    have_rope = True
    for seq in seqs:
        if not seq.is_partial_recompute:
            continue
        sbt = np.asarray(seq.block_table, dtype=np.int64)
        starts = seq.image_rope_starts or [seq.image_rope_start] * len(seq.image_ranges)
        for (img_start, img_end), r, h, rope in zip(seq.image_ranges, seq.image_recompute, seq.image_hashes, starts):
            if r is None:
                continue
            entry = block_manager.get_image_kv_entry(h)
            if entry is None:
                continue
            p = np.arange(img_start + r, img_end, dtype=np.int64)
            if p.size == 0:
                continue
            old_p = entry.img_start + (p - img_start)
            ebt = np.asarray(entry.block_table, dtype=np.int64)
            olds.append(ebt[old_p // bs] * bs + old_p % bs)
            news.append(sbt[p // bs] * bs + p % bs)
            segs.append(np.full(p.size, len(deltas), dtype=np.int32))
            if entry.rope_start is None or rope is None:
                have_rope = False
                deltas.append([0, 0, 0])
            else:
                deltas.append([a - b for a, b in zip(rope, entry.rope_start)])
    if not olds:
        return None
    return np.concatenate(olds), np.concatenate(news), (deltas if have_rope else None), np.concatenate(segs)


class LLMEngine:

    def __init__(self, model, **kwargs):
        names = {f.name for f in fields(Config)}
        config = Config(model, **{k: v for k, v in kwargs.items() if k in names})
        self.config = config
        self.model_runner = ModelRunner(config, 0)
        self.tokenizer = None
        if isinstance(model, (str, os.PathLike)) and os.path.exists(os.path.join(model, "tokenizer.json")):
            from transformers import AutoTokenizer

            self.tokenizer = AutoTokenizer.from_pretrained(model, use_fast=True)
            config.eos = self.tokenizer.eos_token_id
        self.scheduler = Scheduler(config)

    def exit(self):
        self.model_runner.call("exit")

    def add_request(self, prompt, sampling_params: SamplingParams, mm_inputs: dict | None = None):
        hashes = None
        if mm_inputs:
            pv, grid = mm_inputs.get("pixel_values"), mm_inputs.get("image_grid_thw")
            if mm_inputs.get("image_hashes") is not None:
                hashes = list(mm_inputs["image_hashes"])
            elif pv is not None and grid is not None:
                lens = (grid[:, 0] * grid[:, 1] * grid[:, 2]).tolist()
                hashes = [image_hash(p, g) for p, g in zip(torch.split(pv, lens), grid)]
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("no tokenizer in the model directory: pass token ids")
            prompt = self.tokenizer.encode(prompt)
        seq = Sequence(prompt, sampling_params, mm_inputs, hashes)
        self._set_positions(seq)
        self.scheduler.add(seq)
        return seq

    def _set_positions(self, seq: Sequence):
        hf = self.config.hf_config
        grids = seq.mm_inputs.get("image_grid_thw") if seq.mm_inputs else None
        if self.config.use_mrope and grids is not None and len(grids):
            pos, starts, delta = mrope_positions(seq.token_ids, grids.tolist(), hf.image_token_id,
                                                 hf.spatial_merge_size)
            seq.rope_positions = pos
            seq.image_rope_start = starts[0]
            seq.image_rope_starts = list(starts)
            seq.rope_delta = delta
        else:
            seq.rope_positions = None
            seq.find_image_token_range(hf.image_token_id)
            if seq.image_token_range is not None:
                s = seq.image_token_range[0]
                seq.image_rope_start = (s, s, s)
                seq.image_rope_starts = [(a, a, a) for a, _ in seq.image_ranges]
                seq.image_token_range = None  # decided again by the scheduler

    def _do_image_kv_copy(self, seqs: list[Sequence]):
        plan = image_kv_copy_plan(seqs, self.scheduler.block_manager)
        if plan is not None:
            self.model_runner.call("copy_image_kv", *plan)

    def _store_image_kv(self, seqs: list[Sequence]):
        bm = self.scheduler.block_manager
        for seq in seqs:
            if not seq.image_hashes or not seq.block_table:
                continue
            if seq.image_token_range is None:
                seq.find_image_token_range(self.scheduler.image_token_id)
            if seq.image_token_range is not None:
                bm.store_image_kv(seq)

    def step(self):
        seqs, is_prefill = self.scheduler.schedule()
        if is_prefill:
            self._do_image_kv_copy(seqs)
        token_ids, vit_time = self.model_runner.call("run", seqs, is_prefill)
        if is_prefill:
            now = time()
            for seq in seqs:
                if seq.mm_inputs:
                    seq.vit_time = vit_time
                seq.ttft = now - seq.start_time
            self._store_image_kv(seqs)
        self.scheduler.postprocess(seqs, token_ids)
        outputs = [seq for seq in seqs if seq.is_finished]
        num_tokens = sum(len(seq) for seq in seqs) if is_prefill else -len(seqs)
        return outputs, num_tokens

    def is_finished(self):
        return self.scheduler.is_finished()

    def generate(self, prompts, sampling_params, mm_inputs=None, use_tqdm: bool = False):
        if not isinstance(sampling_params, list):
            sampling_params = [sampling_params] * len(prompts)
        if mm_inputs is None:
            mm_inputs = [None] * len(prompts)
        for prompt, sp, mp in zip(prompts, sampling_params, mm_inputs):
            self.add_request(prompt, sp, mp)
        outputs = {}
        while not self.is_finished():
            out, _ = self.step()
            for seq in out:
                outputs[seq.seq_id] = seq
        seqs = [outputs[k] for k in sorted(outputs)]
        return [{
            "text": self.tokenizer.decode(s.completion_token_ids) if self.tokenizer else "",
            "token_ids": s.completion_token_ids,
            "vit_time": s.vit_time,
            "ttft": s.ttft,
        } for s in seqs]
