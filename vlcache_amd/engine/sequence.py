"""Request state (engine/sequence.py:15-110 of the reference).

Same fields and semantics; the image-range scan is vectorised, and the rotary
start position of the image is recorded so that reused keys can be re-rotated.
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
        # rotary positions: image start (t, h, w) and the text offset used after the prompt
        self.image_rope_start: tuple[int, int, int] | None = None
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
        """First to last image token, end exclusive (single image)."""
        idx = np.flatnonzero(np.asarray(self.token_ids, dtype=np.int64) == image_token_id)
        if idx.size:
            self.image_token_range = (int(idx[0]), int(idx[-1]) + 1)

    def reset_partial_recompute(self):
        self.image_token_range = None
        self.num_recompute_tokens = 0
        self.is_partial_recompute = False

    def append_token(self, token_id: int):
        self.token_ids.append(token_id)
        self.last_token = token_id
        self.num_tokens += 1
