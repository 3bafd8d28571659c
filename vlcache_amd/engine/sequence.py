"""Request state (engine/sequence.py:15-110 of the reference).

Same fields and semantics; the image-range scan is vectorised, and the rotary
start position of the image is recorded so that reused keys can be re-rotated.
Several images per prompt: `image_ranges` holds each image's token run,
`image_recompute[k]` the tokens recomputed of image k when its KV is reused
(None: computed in full) and `image_rope_starts[k]` its rotary start; the
single-image fields keep the reference's meaning (first to last image token).
"""
from __future__ import annotations

from copy import copy
from enum import Enum, auto
from itertools import count
import time

import numpy as np

from ..sampling_params import SamplingParams


class SequenceStatus(Enum):
    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


class Sequence:
    block_size = 256
    counter = count()

    def __init__(self, token_ids: list[int], sampling_params=SamplingParams(), mm_inputs: dict | None = None,
                 image_hashes: list[int] | None = None):
        self.seq_id = next(Sequence.counter)
        self.status = SequenceStatus.WAITING
        self.token_ids = copy(token_ids)
        self.last_token = token_ids[-1]
        self.num_tokens = len(self.token_ids)
        self.num_prompt_tokens = len(token_ids)
        self.num_cached_tokens = 0
        self.block_table: list[int] = []
        self.temperature = sampling_params.temperature
        self.max_tokens = sampling_params.max_tokens
        self.ignore_eos = sampling_params.ignore_eos
        self.mm_inputs = mm_inputs
        self.image_hashes = image_hashes
        # partial recompute
        self.image_token_range: tuple[int, int] | None = None
        self.num_recompute_tokens = 0
        self.is_partial_recompute = False
        self.image_ranges: list[tuple[int, int]] = []          # token run of each image
        self.image_recompute: list[int | None] = []           # per image: R if reused, else None
        # rotary positions: image start (t, h, w) and the text offset used after the prompt
        self.image_rope_start: tuple[int, int, int] | None = None
        self.image_rope_starts: list[tuple[int, int, int]] = []
        self.rope_delta = 0
        # timing
        self.start_time = time.time()
        self.vit_time = 0.0
        self.ttft = 0.0

    def __len__(self):
        return self.num_tokens

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def is_finished(self):
        return self.status == SequenceStatus.FINISHED

    @property
    def num_completion_tokens(self):
        return self.num_tokens - self.num_prompt_tokens

    @property
    def prompt_token_ids(self):
        return self.token_ids[:self.num_prompt_tokens]

    @property
    def completion_token_ids(self):
        return self.token_ids[self.num_prompt_tokens:]

    @property
    def num_blocks(self):
        return (self.num_tokens + self.block_size - 1) // self.block_size

    @property
    def last_block_num_tokens(self):
        return self.num_tokens - (self.num_blocks - 1) * self.block_size

    def find_image_token_range(self, image_token_id: int = 151655):
        """First to last image token, end exclusive (engine/sequence.py:91-100), and the
        maximal run of image tokens of each image (`image_ranges`)."""
        is_img = np.asarray(self.token_ids, dtype=np.int64) == image_token_id
        idx = np.flatnonzero(is_img)
        if idx.size:
            self.image_token_range = (int(idx[0]), int(idx[-1]) + 1)
            d = np.diff(np.concatenate([[0], is_img.astype(np.int8), [0]]))
            self.image_ranges = list(zip(np.flatnonzero(d == 1).tolist(), np.flatnonzero(d == -1).tolist()))

    @property
    def num_reused_tokens(self) -> int:
        """Image tokens whose KV is copied instead of computed."""
        return sum((e - s) - r for (s, e), r in zip(self.image_ranges, self.image_recompute) if r is not None)

    def computed_runs(self) -> list[tuple[int, int]]:
        """Maximal runs [a, b) of computed prompt tokens; each is a virtual sub-sequence
        with queries [a, b) and keys [0, b) (engine/model_runner.py:237-259 for one image)."""
        n = self.num_tokens
        gaps = sorted((s + r, e) for (s, e), r in zip(self.image_ranges, self.image_recompute)
                      if r is not None and s + r < e)
        runs, p = [], 0
        for a, b in gaps:
            if a > p:
                runs.append((p, a))
            p = b
        if p < n:
            runs.append((p, n))
        return runs

    def reset_partial_recompute(self):
        self.image_token_range = None
        self.num_recompute_tokens = 0
        self.is_partial_recompute = False
        self.image_recompute = []

    def append_token(self, token_id: int):
        self.token_ids.append(token_id)
        self.last_token = token_id
        self.num_tokens += 1
