"""Bit-copy oracles of the KV scatter and the image-KV copy (test-only)."""
from __future__ import annotations

import numpy as np


def store_kvcache(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                  slot_mapping: np.ndarray) -> None:
    """In place: row `slot` of the caches <- row n of key/value, slot == -1 skipped.

    Restates store_kvcache_kernel (layers/attention.py:10-30): the kernel copies
    D = num_kv_heads * head_dim contiguous elements per token; k_cache/v_cache are
    viewed as [num_slots, D].  Arrays may be any dtype (bf16 is passed as uint16).
    """
    n = key.shape[0]
    d = int(np.prod(key.shape[1:]))
    kc = k_cache.reshape(-1, d)
    vc = v_cache.reshape(-1, d)
    keep = slot_mapping != -1
    slots = slot_mapping[keep].astype(np.int64)
    kc[slots] = key.reshape(n, d)[keep]
    vc[slots] = value.reshape(n, d)[keep]


def copy_image_kv(kv_cache: np.ndarray, old_slots, new_slots) -> None:
    """In place: flat[:, :, new] = flat[:, :, old] (engine/model_runner.py:177-180).

    kv_cache is [2, L, num_blocks, block_size, Hkv, hd]; the flat view is
    [2, L, num_blocks * block_size, Hkv * hd].  The right side is gathered
    before the assignment, as torch advanced indexing does.
    """
    s = kv_cache.shape
    flat = kv_cache.reshape(s[0], s[1], -1, s[4] * s[5])
    old = np.asarray(old_slots, dtype=np.int64)
    new = np.asarray(new_slots, dtype=np.int64)
    if old.size == 0:
        return
    flat[:, :, new] = flat[:, :, old].copy()
