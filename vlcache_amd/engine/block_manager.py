"""Paged KV block allocator and image-KV registry (engine/block_manager.py:8-119 of the reference).

Same allocation, reference counting and partial-recompute decision, taken per
image when a prompt holds several.  The registry entry additionally records the
rotary start position of the cached image, which the re-rotation of reused keys
needs.
"""
from __future__ import annotations

import math
from collections import deque
from dataclasses import dataclass

from .sequence import Sequence


class Block:
    def __init__(self, block_id):
        self.block_id = block_id
        self.ref_count = 0

    def reset(self):
        self.ref_count = 1


@dataclass
class ImageKVEntry:
    block_table: list[int]   # full block table of the source sequence
    img_start: int           # image start token index in the source sequence
    img_end: int             # image end token index (exclusive)
    rope_start: tuple | None = None  # (t, h, w) rotary start position of the image in the source


class BlockManager:

    def __init__(self, num_blocks: int, block_size: int, recompute_ratio: float = 0.0):
        self.block_size = block_size
        self.recompute_ratio = recompute_ratio
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.free_block_ids: deque[int] = deque(range(num_blocks))
        self.used_block_ids: set[int] = set()
        self.image_kv_cache: dict[int, ImageKVEntry] = {}

    def _allocate_block(self) -> Block:
        block_id = self.free_block_ids.popleft()
        block = self.blocks[block_id]
        block.reset()
        self.used_block_ids.add(block_id)
        return block

    def _deallocate_block(self, block_id: int):
        assert self.blocks[block_id].ref_count == 0
        self.used_block_ids.remove(block_id)
        self.free_block_ids.append(block_id)

    def can_allocate(self, seq: Sequence) -> bool:
        return len(self.free_block_ids) >= seq.num_blocks

    def allocate(self, seq: Sequence):
        assert not seq.block_table
        for _ in range(seq.num_blocks):
            seq.block_table.append(self._allocate_block().block_id)

    def try_partial_recompute(self, seq: Sequence, image_token_id: int = 151655) -> bool:
        """Reuse decision (engine/block_manager.py:56-75), per image.

        Image k of the prompt is reused when the registry holds an entry for
        image_hashes[k] with the same number of tokens; its first
        R_k = ceil(ratio * N_k) tokens are recomputed (IEEE double, as the
        reference).  With one image this is the reference's decision exactly.
        """
        if self.recompute_ratio <= 0 or not seq.image_hashes:
            return False
        seq.find_image_token_range(image_token_id)
        if seq.image_token_range is None:
            return False
        seq.image_recompute = [None] * len(seq.image_ranges)
        for k, ((s, e), h) in enumerate(zip(seq.image_ranges, seq.image_hashes)):
            entry = self.image_kv_cache.get(h)
            if entry is not None and e - s == entry.img_end - entry.img_start:
                seq.image_recompute[k] = math.ceil(self.recompute_ratio * (e - s))
        hits = [r for r in seq.image_recompute if r is not None]
        if not hits:
            return False
        seq.num_recompute_tokens = hits[0]
        seq.is_partial_recompute = True
        return True

    def get_image_kv_entry(self, image_hash: int) -> ImageKVEntry | None:
        return self.image_kv_cache.get(image_hash)

    def store_image_kv(self, seq: Sequence):
        """Register the KV of each image of a prefilled sequence under its hash."""
        if not seq.image_hashes or seq.image_token_range is None:
            return
        ranges = seq.image_ranges or [seq.image_token_range]
        starts = seq.image_rope_starts or [seq.image_rope_start] * len(ranges)
        for (img_start, img_end), image_hash, rope in zip(ranges, seq.image_hashes, starts):
            old = self.image_kv_cache.get(image_hash)
            for i in range(img_start // self.block_size, (img_end - 1) // self.block_size + 1):
                self.blocks[seq.block_table[i]].ref_count += 1
            if old is not None:
                self._release_image_blocks(old)
            self.image_kv_cache[image_hash] = ImageKVEntry(list(seq.block_table), img_start, img_end, rope)

    def _release_image_blocks(self, entry: ImageKVEntry):
        for i in range(entry.img_start // self.block_size, (entry.img_end - 1) // self.block_size + 1):
            block_id = entry.block_table[i]
            block = self.blocks[block_id]
            block.ref_count -= 1
            if block.ref_count == 0:
                self._deallocate_block(block_id)

    def deallocate(self, seq: Sequence):
        for block_id in reversed(seq.block_table):
            block = self.blocks[block_id]
            block.ref_count -= 1
            if block.ref_count == 0:
                self._deallocate_block(block_id)
        seq.num_cached_tokens = 0
        seq.block_table.clear()

    def can_append(self, seq: Sequence) -> bool:
        return len(self.free_block_ids) >= (len(seq) % self.block_size == 1)

    def may_append(self, seq: Sequence):
        if len(seq) % self.block_size == 1:
            seq.block_table.append(self._allocate_block().block_id)
