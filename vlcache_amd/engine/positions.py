"""Rotary positions of a prompt: 1-D (the reference) or Qwen2.5-VL M-RoPE.

The reference gives every token its index (engine/model_runner.py:240,247,281).
Qwen2.5-VL's own position rule (transformers get_rope_index /
get_vision_position_ids) gives text tokens (p, p, p) and an image starting at
position s the rows t = s, h = s + row, w = s + col on its merged grid; text
after the image resumes at s + max(h, w).  Images are the maximal runs of the
image token, in order, matched with their grids.
"""
from __future__ import annotations

import numpy as np


def image_runs(token_ids: np.ndarray, image_token_id: int):
    """[(start, end)] of the maximal runs of image_token_id."""
    is_img = np.asarray(token_ids) == image_token_id
    if not is_img.any():
        return []
    d = np.diff(np.concatenate([[0], is_img.astype(np.int8), [0]]))
    starts = np.flatnonzero(d == 1)
    ends = np.flatnonzero(d == -1)
    return list(zip(starts.tolist(), ends.tolist()))


def mrope_positions(token_ids, grids_thw, image_token_id: int, spatial_merge_size: int = 2):
    """Returns (positions int64 [3, n], image rope starts [(t, h, w)], rope_delta).

    grids_thw: per image (t, h, w) in patches before the spatial merge.
    rope_delta = max position + 1 - n: decode continues at len - 1 + rope_delta.
    """
    ids = np.asarray(token_ids)
    n = ids.size
    runs = image_runs(ids, image_token_id)
    if len(runs) != len(grids_thw):
        raise ValueError(f"{len(runs)} image-token runs but {len(grids_thw)} image grids")
    pos = np.empty((3, n), dtype=np.int64)
    starts = []
    cur = 0   # next position to assign
    prev = 0  # next token index
    for (a, e), (t, h, w) in zip(runs, grids_thw):
        pos[:, prev:a] = cur + np.arange(a - prev)
        cur += a - prev
        hm, wm = int(h) // spatial_merge_size, int(w) // spatial_merge_size
        if (e - a) != int(t) * hm * wm:
            raise ValueError(f"image run of {e - a} tokens does not match grid {(t, h, w)}")
        tt, hh, ww = np.meshgrid(np.arange(int(t)), np.arange(hm), np.arange(wm), indexing="ij")
        pos[0, a:e] = cur + tt.reshape(-1)
        pos[1, a:e] = cur + hh.reshape(-1)
        pos[2, a:e] = cur + ww.reshape(-1)
        starts.append((cur, cur, cur))
        cur += max(hm, wm)
        prev = e
    pos[:, prev:] = cur + np.arange(n - prev)
    cur += n - prev
    return pos, starts, int(pos.max()) + 1 - n if n else 0
