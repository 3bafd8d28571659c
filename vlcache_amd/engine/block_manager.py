"""KV block pool and image-KV registry.

Behaviour follows the reference's BlockManager (engine/block_manager.py:8-128):
blocks are handed out in FIFO order of their release, a block is free when no
sequence and no registry entry references it, a warm request's images are
reused when the registry holds the same hash with the same token count
(R = ceil(ratio * N) tokens recomputed, in IEEE double, :56-75), and storing an
image pins the blocks under it so they outlive the source sequence, replacing
(and unpinning) an older entry of the same hash (:80-110).

The layout is this package's own: reference counts are one numpy int32 array,
the free list is a ring buffer of block ids (a batch of blocks is taken or
returned with one slice), and decisions are per image, so a prompt may hold
several images, each reused or computed on its own.  A registry entry also
records the image's rotary start, which the re-rotation of reused keys needs.

The registry is kept in least-recently-used order (a reuse decision or a store
touches an entry), and evict_images() releases its oldest entries when a request
does not fit the pool.  The reference keeps every entry until the same hash is
stored again, so a stream of distinct images fills its pool with pinned image
blocks and admission stops for good.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .sequence import Sequence


@dataclass
class ImageKVEntry:
    block_table: list[int]   # block table of the sequence the image was computed in
    img_start: int           # first image token in that sequence
    img_end: int             # one past the last image token
    rope_start: tuple | None = None  # (t, h, w) rotary start of the image there


class BlockManager:

    def __init__(self, num_blocks: int, block_size: int, recompute_ratio: float = 0.0):
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("the pool needs blocks of a positive size")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.recompute_ratio = recompute_ratio
        self.ref_counts = np.zeros(num_blocks, dtype=np.int32)
        self._ring = np.arange(num_blocks, dtype=np.int64)  # free ids, oldest release first
        self._head = 0
        self._nfree = num_blocks
        self.image_kv_cache: dict[int, ImageKVEntry] = {}

    # ------------------------------------------------------------------ pool
    @property
    def num_free_blocks(self) -> int:
        return self._nfree

    def free_block_ids(self) -> list[int]:
        """Free block ids in the order they will be handed out."""
        idx = (self._head + np.arange(self._nfree)) % self.num_blocks
        return self._ring[idx].tolist()

    def _take(self, n: int) -> np.ndarray:
        if n > self._nfree:
            raise RuntimeError(f"{n} blocks requested, {self._nfree} free")
        idx = (self._head + np.arange(n)) % self.num_blocks
        ids = self._ring[idx]
        self._head = (self._head + n) % self.num_blocks
        self._nfree -= n
        self.ref_counts[ids] = 1
        return ids

    def _unref(self, ids) -> None:
        """Drop one reference from each block of ids (distinct) and queue the ones left
        unreferenced, in the given order."""
        ids = np.asarray(ids, dtype=np.int64)
        if ids.size == 0:
            return
        if np.any(self.ref_counts[ids] <= 0):
            raise RuntimeError("releasing a block that is not referenced")
        self.ref_counts[ids] -= 1
        dead = ids[self.ref_counts[ids] == 0]
        if dead.size:
            tail = (self._head + self._nfree + np.arange(dead.size)) % self.num_blocks
            self._ring[tail] = dead
            self._nfree += dead.size

    def ref_count(self, block_id: int) -> int:
        return int(self.ref_counts[block_id])

    def can_allocate(self, seq: Sequence) -> bool:
        return self._nfree >= seq.num_blocks

    def allocate(self, seq: Sequence) -> None:
        if seq.block_table:
            raise RuntimeError("sequence already holds blocks")
        seq.block_table.extend(self._take(seq.num_blocks).tolist())

    def deallocate(self, seq: Sequence) -> None:
        self._unref(seq.block_table[::-1])
        seq.block_table.clear()
        seq.num_cached_tokens = 0

    def blocks_to_append(self, seq: Sequence) -> int:
        """Blocks the next decode step of seq needs: one when its newest token opened a block."""
        return 1 if len(seq) % self.block_size == 1 else 0

    def can_append(self, seq: Sequence) -> bool:
        return self._nfree >= self.blocks_to_append(seq)

    def may_append(self, seq: Sequence) -> None:
        n = self.blocks_to_append(seq)
        if n:
            seq.block_table.extend(self._take(n).tolist())

    # ------------------------------------------------------------------ image-KV registry
    def try_partial_recompute(self, seq: Sequence, image_token_id: int = 151655) -> bool:
        """Decide, per image, whether its KV is reused; returns True when any is.

        Image k is reused when the registry holds its hash with the same token
        count; its first ceil(ratio * N_k) tokens are then recomputed."""
        seq.reset_partial_recompute()
        if self.recompute_ratio <= 0 or not seq.image_hashes:
            return False
        for span in seq.scan_images(image_token_id):
            entry = self.image_kv_cache.get(span.hash) if span.hash is not None else None
            if entry is not None and entry.img_end - entry.img_start == span.size:
                span.recompute = math.ceil(self.recompute_ratio * span.size)
                self.image_kv_cache[span.hash] = self.image_kv_cache.pop(span.hash)  # most recently used
        return seq.is_partial_recompute

    def get_image_kv_entry(self, image_hash: int) -> ImageKVEntry | None:
        return self.image_kv_cache.get(image_hash)

    def _image_blocks(self, block_table, start: int, end: int) -> np.ndarray:
        first, last = start // self.block_size, (end - 1) // self.block_size
        return np.asarray(block_table[first:last + 1], dtype=np.int64)

    def store_image_kv(self, seq: Sequence) -> None:
        """Register every hashed image of a prefilled sequence (the last store of a hash wins)."""
        if not seq.image_hashes or not seq.block_table:
            return
        for span in seq.images:
            if span.hash is None:
                continue
            pinned = self._image_blocks(seq.block_table, span.start, span.end)
            self.ref_counts[pinned] += 1
            old = self.image_kv_cache.pop(span.hash, None)
            self.image_kv_cache[span.hash] = ImageKVEntry(list(seq.block_table), span.start, span.end,
                                                          span.rope_start)
            if old is not None:
                self._unpin(old)

    def _unpin(self, entry: ImageKVEntry) -> None:
        self._unref(self._image_blocks(entry.block_table, entry.img_start, entry.img_end))

    def evict_images(self, need_free: int, keep=()) -> int:
        """Release registry entries, least recently used first and skipping the hashes in
        keep, until need_free blocks are free or no entry is left to release; returns how
        many were released.  A released entry's blocks stay with any sequence that still
        holds them."""
        released = 0
        for h in list(self.image_kv_cache):
            if self._nfree >= need_free:
                break
            if h in keep:
                continue
            self.release_image(h)
            released += 1
        return released

    def release_image(self, image_hash: int) -> bool:
        """Drop a registry entry and unpin its blocks; False when the hash is unknown."""
        entry = self.image_kv_cache.pop(image_hash, None)
        if entry is None:
            return False
        self._unpin(entry)
        return True
