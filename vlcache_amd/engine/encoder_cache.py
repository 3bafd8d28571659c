"""Bounded GPU cache of visual embeddings, keyed by image hash.

The reference keeps the vision tower's output per image hash in a paged pool
whose size is the encoder_cache_ratio share of free memory, evicting the least
recently used images when a new one does not fit
(engine/encoder_cache_manager.py:6-70; sized at engine/model_runner.py:126-149,
read and written at :347-395).  A warm request reads an image's embeddings back
instead of running the vision tower and keeps its first R rows.

Here the pool is one bf16 tensor [num_pages, page_rows, hidden].  Pages are
handed out lowest id first, so an entry stored into a pool without holes
occupies consecutive pages and reading it back is a view of the pool, not a
gather; only the pages holding the rows asked for are touched.  Recency is a
use counter per entry; eviction removes the entry with the smallest until the
new image fits.  An image larger than the whole pool is not cached.
"""
from __future__ import annotations

import numpy as np
import torch


class EncoderCache:

    def __init__(self, num_pages: int, page_rows: int, hidden: int, dtype: torch.dtype, device):
        if num_pages < 0 or page_rows <= 0:
            raise ValueError("encoder cache needs a non-negative page count and positive page size")
        self.num_pages = num_pages
        self.page_rows = page_rows
        self.hidden = hidden
        self.pool = torch.empty(num_pages, page_rows, hidden, dtype=dtype, device=device)
        self._free = np.ones(num_pages, dtype=bool)
        self._entries: dict[int, tuple[np.ndarray, int]] = {}  # hash -> (pages, rows)
        self._last_use: dict[int, int] = {}
        self._clock = 0
        self.hits = self.misses = self.evictions = 0

    def __contains__(self, key: int) -> bool:
        return key in self._entries

    def __len__(self) -> int:
        return len(self._entries)

    @property
    def free_pages(self) -> int:
        return int(self._free.sum())

    def _touch(self, key: int) -> None:
        self._clock += 1
        self._last_use[key] = self._clock

    def _pages_for(self, rows: int) -> int:
        return -(-rows // self.page_rows)

    def get(self, key: int, rows: int | None = None) -> torch.Tensor | None:
        """The first `rows` embeddings of an image (all when None), or None on a miss.

        The result may be a view of the pool: it holds the image's rows only until the
        next put(), which can evict the entry and reuse its pages.  Copy it before then.
        """
        entry = self._entries.get(key)
        if entry is None:
            self.misses += 1
            return None
        pages, n = entry
        self.hits += 1
        self._touch(key)
        rows = n if rows is None else min(int(rows), n)
        need = pages[:self._pages_for(rows)]
        if need.size and np.all(np.diff(need) == 1):
            flat = self.pool[int(need[0]):int(need[0]) + need.size].view(-1, self.hidden)
        else:
            flat = self.pool[torch.as_tensor(need, device=self.pool.device)].view(-1, self.hidden)
        return flat[:rows]

    def _evict_one(self) -> None:
        victim = min(self._last_use, key=self._last_use.get)
        pages, _ = self._entries.pop(victim)
        del self._last_use[victim]
        self._free[pages] = True
        self.evictions += 1

    def put(self, key: int, embeds: torch.Tensor) -> bool:
        """Store an image's embeddings [rows, hidden]; False when it cannot fit the pool."""
        if embeds.dim() != 2 or embeds.shape[1] != self.hidden:
            raise ValueError(f"embeddings must be [rows, {self.hidden}]")
        if key in self._entries:
            self._touch(key)
            return True
        rows = embeds.shape[0]
        need = self._pages_for(rows)
        if need > self.num_pages:
            return False
        while int(self._free.sum()) < need:
            self._evict_one()
        pages = np.flatnonzero(self._free)[:need]
        self._free[pages] = False
        full, rest = divmod(rows, self.page_rows)
        src = embeds.to(self.pool.dtype)
        if np.all(np.diff(pages) == 1):
            self.pool[int(pages[0]):int(pages[0]) + need].view(-1, self.hidden)[:rows].copy_(src)
        else:
            idx = torch.as_tensor(pages[:full], device=self.pool.device)
            if full:
                self.pool.index_copy_(0, idx, src[:full * self.page_rows].view(full, self.page_rows, -1))
            if rest:
                self.pool[int(pages[full]), :rest].copy_(src[full * self.page_rows:])
        self._entries[key] = (pages, rows)
        self._touch(key)
        return True
