"""Request loop on one GPU: the reference's LLMEngine surface (engine/llm_engine.py).

add_request hashes each image (xxhash of its grid and pixel values, as
engine/encoder_cache_manager.py:24-29 does) before the Sequence -- and with it
the TTFT clock -- starts, scans the prompt's images once and records their
rotary starts.  A step schedules; for a prefill it copies the reused image KV
of warm requests (re-rotating the keys to the image's new rotary start; the
reference copies them unchanged, :58-89), runs the model, stamps the TTFT of
every prefilled request and registers its images for later reuse (:103-120).
generate() returns [{text, token_ids, vit_time, ttft}] (:125-167).
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
    # raw bytes of any dtype (numpy has no bf16), hashed in place through the buffer
    # protocol: the same digest as hashing numpy's tobytes() copy, without the copy
    h.update(pixel_values.detach().cpu().contiguous().view(torch.uint8).numpy())
    return h.intdigest()


def image_kv_copy_plan(seqs: list[Sequence], block_manager):
    """Slots of the reused image KV of a prefill step (engine/llm_engine.py:58-89).

    Token p of a reused image [s, e) with R recomputed tokens (p in [s + R, e))
    takes the row of token entry.img_start + (p - s) of the registered copy.
    Returns (old_slots, new_slots, deltas, seg_of_token) for
    ModelRunner.copy_image_kv -- every image of every sequence in one launch,
    image k being rotation segment k with delta = its rotary start here minus the
    registered one (deltas None when a rotary start is unknown) -- or None when
    nothing is reused.
    """
    bs = block_manager.block_size
    src, dst, seg, deltas = [], [], [], []
    rotary_known = True
    for seq in seqs:
        table = np.asarray(seq.block_table, dtype=np.int64)
        for span in seq.images:
            if span.reused == 0:
                continue
            entry = block_manager.get_image_kv_entry(span.hash)
            if entry is None:
                continue
            p = np.arange(span.start + span.recompute, span.end, dtype=np.int64)
            q = p - span.start + entry.img_start
            etable = np.asarray(entry.block_table, dtype=np.int64)
            src.append(etable[q // bs] * bs + q % bs)
            dst.append(table[p // bs] * bs + p % bs)
            seg.append(np.full(p.size, len(deltas), dtype=np.int32))
            if span.rope_start is None or entry.rope_start is None:
                rotary_known = False
                deltas.append([0, 0, 0])
            else:
                deltas.append([a - b for a, b in zip(span.rope_start, entry.rope_start)])
    if not src:
        return None
    return np.concatenate(src), np.concatenate(dst), (deltas if rotary_known else None), np.concatenate(seg)


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

    # ------------------------------------------------------------------ requests
    def add_request(self, prompt, sampling_params: SamplingParams, mm_inputs: dict | None = None) -> Sequence:
        hashes = None
        if mm_inputs:
            if mm_inputs.get("image_hashes") is not None:
                hashes = [int(h) for h in mm_inputs["image_hashes"]]
            else:
                pv, grid = mm_inputs.get("pixel_values"), mm_inputs.get("image_grid_thw")
                if pv is not None and grid is not None:
                    per_image = (grid[:, 0] * grid[:, 1] * grid[:, 2]).tolist()
                    hashes = [image_hash(p, g) for p, g in zip(torch.split(pv, per_image), grid)]
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("no tokenizer in the model directory: pass token ids")
            prompt = self.tokenizer.encode(prompt)
        seq = Sequence(prompt, sampling_params, mm_inputs, hashes)
        self._place_images(seq)
        self.scheduler.add(seq)
        return seq

    def _place_images(self, seq: Sequence) -> None:
        """Scan the prompt's images and give them (and the prompt) rotary positions:
        M-RoPE when the model uses it and grids are known, else token indices."""
        hf = self.config.hf_config
        spans = seq.scan_images(hf.image_token_id)
        grids = seq.mm_inputs.get("image_grid_thw") if seq.mm_inputs else None
        if self.config.use_mrope and grids is not None and len(grids):
            pos, starts, delta = mrope_positions(seq.token_ids, grids.tolist(), hf.image_token_id,
                                                 hf.spatial_merge_size)
            seq.rope_positions, seq.rope_delta = pos, delta
            seq.set_rope_starts(starts)
        else:
            seq.set_rope_starts([(s.start,) * 3 for s in spans])

    # ------------------------------------------------------------------ steps
    def _reuse_image_kv(self, seqs: list[Sequence]) -> None:
        plan = image_kv_copy_plan(seqs, self.scheduler.block_manager)
        if plan is not None:
            self.model_runner.call("copy_image_kv", *plan)

    def _register_images(self, seqs: list[Sequence]) -> None:
        """After a prefill the KV of every hashed image is in the cache: register it."""
        bm = self.scheduler.block_manager
        for seq in seqs:
            if seq.image_hashes and seq.block_table and seq.images:
                bm.store_image_kv(seq)

    # The reference's method names for the two hooks above.
    _do_image_kv_copy = _reuse_image_kv
    _store_image_kv = _register_images

    def step(self):
        seqs, is_prefill = self.scheduler.schedule()
        if is_prefill:
            self._reuse_image_kv(seqs)
        token_ids, vit_time = self.model_runner.call("run", seqs, is_prefill)
        if is_prefill:
            stamp = time()
            for seq in seqs:
                seq.ttft = stamp - seq.start_time
                if seq.mm_inputs:
                    seq.vit_time = vit_time
            self._register_images(seqs)
        self.scheduler.postprocess(seqs, token_ids)
        finished = [s for s in seqs if s.is_finished]
        return finished, (sum(len(s) for s in seqs) if is_prefill else -len(seqs))

    def is_finished(self):
        return self.scheduler.is_finished()

    def generate(self, prompts, sampling_params, mm_inputs=None, use_tqdm: bool = False):
        n = len(prompts)
        params = sampling_params if isinstance(sampling_params, list) else [sampling_params] * n
        mms = mm_inputs if mm_inputs is not None else [None] * n
        for prompt, sp, mm in zip(prompts, params, mms):
            self.add_request(prompt, sp, mm)
        done: dict[int, Sequence] = {}
        while not self.is_finished():
            finished, _ = self.step()
            done.update((s.seq_id, s) for s in finished)
        return [{
            "text": self.tokenizer.decode(s.completion_token_ids) if self.tokenizer else "",
            "token_ids": s.completion_token_ids,
            "vit_time": s.vit_time,
            "ttft": s.ttft,
        } for _, s in sorted(done.items())]
