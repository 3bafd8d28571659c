"""Request state: tokens, KV block table, sampling settings, images and their reuse.

The public fields and properties are those the reference's engine reads
(engine/sequence.py:15-110: token counts, prompt/completion views, block counts,
image_token_range, num_recompute_tokens, is_partial_recompute, timing).  The
state behind them is organised per image: a prompt's images are scanned once,
when the request is added, into ImageSpan records (token run, content hash,
rotary start, reuse decision); the reference's single-image fields are views of
that list (the first to the last image token; the first reused image's R).
"""
from __future__ import annotations

import time
from dataclasses import dataclass
from enum import Enum, auto
from itertools import count

import numpy as np

from ..sampling_params import SamplingParams
from .positions import image_runs


class SequenceStatus(Enum):
    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


@dataclass
class ImageSpan:
    """One image of a prompt.  recompute: tokens recomputed at its start when its KV is
    reused from the registry (R = ceil(ratio * N)); None when it is computed in full."""
    start: int
    end: int
    hash: int | None = None
    rope_start: tuple | None = None
    recompute: int | None = None

    @property
    def size(self) -> int:
        return self.end - self.start

    @property
    def reused(self) -> int:
        return 0 if self.recompute is None else max(0, self.size - self.recompute)


class Sequence:
    block_size = 256  # fixed, as in the reference (engine/sequence.py:16)
    _ids = count()

    def __init__(self, token_ids: list[int], sampling_params: SamplingParams = SamplingParams(),
                 mm_inputs: dict | None = None, image_hashes: list[int] | None = None):
        if not token_ids:
            raise ValueError("a sequence needs at least one token")
        self.seq_id = next(Sequence._ids)
        self.status = SequenceStatus.WAITING
        self.token_ids = list(token_ids)
        self.num_prompt_tokens = len(self.token_ids)
        self.num_cached_tokens = 0
        self.block_table: list[int] = []
        self.temperature = sampling_params.temperature
        self.max_tokens = sampling_params.max_tokens
        self.ignore_eos = sampling_params.ignore_eos
        self.mm_inputs = mm_inputs
        self.image_hashes = image_hashes
        self.images: list[ImageSpan] = []
        self._scanned_for: int | None = None
        # Rotary positions of the prompt ([3, n] M-RoPE rows, or None for 1-D indices) and
        # the offset that continues them past the prompt: position of index p >= n is p + rope_delta.
        self.rope_positions: np.ndarray | None = None
        self.rope_delta = 0
        self.start_time = time.time()
        self.vit_time = 0.0
        self.ttft = 0.0

    # ------------------------------------------------------------------ tokens
    def __len__(self) -> int:
        return len(self.token_ids)

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)

    @property
    def last_token(self) -> int:
        return self.token_ids[-1]

    @property
    def is_finished(self) -> bool:
        return self.status is SequenceStatus.FINISHED

    @property
    def num_completion_tokens(self) -> int:
        return len(self.token_ids) - self.num_prompt_tokens

    @property
    def prompt_token_ids(self) -> list[int]:
        return self.token_ids[:self.num_prompt_tokens]

    @property
    def completion_token_ids(self) -> list[int]:
        return self.token_ids[self.num_prompt_tokens:]

    def append_token(self, token_id: int) -> None:
        self.token_ids.append(token_id)

    # ------------------------------------------------------------------ KV blocks
    @property
    def num_blocks(self) -> int:
        return -(-len(self.token_ids) // self.block_size)

    @property
    def last_block_num_tokens(self) -> int:
        return (len(self.token_ids) - 1) % self.block_size + 1

    # ------------------------------------------------------------------ images
    def scan_images(self, image_token_id: int = 151655) -> list[ImageSpan]:
        """Find the prompt's images (maximal runs of the image token) once; each gets the
        hash of the same rank in image_hashes."""
        if self._scanned_for != image_token_id:
            ids = np.asarray(self.token_ids[:self.num_prompt_tokens], dtype=np.int64)
            hashes = list(self.image_hashes or [])
            self.images = [ImageSpan(a, b, hashes[k] if k < len(hashes) else None)
                           for k, (a, b) in enumerate(image_runs(ids, image_token_id))]
            self._scanned_for = image_token_id
        return self.images

    def find_image_token_range(self, image_token_id: int = 151655) -> None:
        """The reference's name for the scan (engine/sequence.py:91-100)."""
        self.scan_images(image_token_id)

    def set_rope_starts(self, starts) -> None:
        for span, st in zip(self.images, starts):
            span.rope_start = None if st is None else tuple(int(x) for x in st)

    @property
    def image_token_range(self) -> tuple[int, int] | None:
        """First to last image token, end exclusive (the reference's single-image view)."""
        return (self.images[0].start, self.images[-1].end) if self.images else None

    @property
    def image_ranges(self) -> list[tuple[int, int]]:
        return [(s.start, s.end) for s in self.images]

    @property
    def image_recompute(self) -> list[int | None]:
        return [s.recompute for s in self.images]

    @image_recompute.setter
    def image_recompute(self, counts) -> None:
        for span, r in zip(self.images, counts):
            span.recompute = None if r is None else int(r)

    @property
    def image_rope_starts(self) -> list:
        return [s.rope_start for s in self.images]

    @property
    def image_rope_start(self):
        return self.images[0].rope_start if self.images else None

    @property
    def is_partial_recompute(self) -> bool:
        return any(s.recompute is not None for s in self.images)

    @property
    def num_recompute_tokens(self) -> int:
        """R of the first reused image (the reference's single-image count), else 0."""
        return next((s.recompute for s in self.images if s.recompute is not None), 0)

    @property
    def num_reused_tokens(self) -> int:
        """Image tokens whose KV is copied from the registry instead of computed."""
        return sum(s.reused for s in self.images)

    @property
    def prefill_cost(self) -> int:
        """Tokens a prefill of this sequence computes (the scheduler's budget unit)."""
        return len(self.token_ids) - self.num_reused_tokens

    def computed_runs(self) -> list[tuple[int, int]]:
        """Maximal runs [a, b) of tokens a prefill computes; each is a virtual
        sub-sequence with queries [a, b) and keys [0, b).  One reused image gives the
        reference's two sub-sequences (engine/model_runner.py:237-259)."""
        runs, cursor = [], 0
        for s in sorted(self.images, key=lambda x: x.start):
            if s.reused == 0:
                continue
            gap_start = s.start + s.recompute
            if gap_start > cursor:
                runs.append((cursor, gap_start))
            cursor = s.end
        if cursor < len(self.token_ids):
            runs.append((cursor, len(self.token_ids)))
        return runs

    def reset_partial_recompute(self) -> None:
        """Forget the reuse decisions (the scheduler decides again next time)."""
        for s in self.images:
            s.recompute = None

    # ------------------------------------------------------------------ positions
    def positions(self, start: int, end: int, mrope: bool) -> np.ndarray:
        """Rotary positions of tokens [start, end): int64 [3, n] (mrope) or [n].

        Inside the prompt they are the stored rows; past it (tokens generated
        before a preemption and now prefilled again) index p sits at p +
        rope_delta on every row, the rule decoding continues with."""
        idx = np.arange(start, end, dtype=np.int64)
        pos = self.rope_positions
        if pos is None:
            return np.tile(idx, (3, 1)) if mrope else idx
        n = pos.shape[1]
        if end <= n:
            out = pos[:, start:end]
        else:
            tail = np.arange(max(start, n), end, dtype=np.int64) + self.rope_delta
            out = np.concatenate([pos[:, start:min(end, n)], np.tile(tail, (3, 1))], axis=1)
        return np.ascontiguousarray(out) if mrope else np.ascontiguousarray(out[0])
