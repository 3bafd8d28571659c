"""Rotary-embedding oracles: M-RoPE positions and re-rotation of cached K (test-only).

The reference applies 1-D RoPE (layers/rotary_embedding.py:6-48) and never moves
cached keys to new positions: the re-rotation is new on this path.  Its oracle
is the closed form R(pos_new) k = R(pos_new - pos_old) R(pos_old) k evaluated
with the reference's own fp32 formula, with M-RoPE's three position sections as
transformers' Qwen2.5-VL defines them (modeling_qwen2_5_vl.py
apply_multimodal_rotary_pos_emb, get_vision_position_ids, get_rope_index).
"""
from __future__ import annotations

import numpy as np
import torch


def inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """fp32 [head_dim/2]: 1 / theta^(2i/head_dim) (layers/rotary_embedding.py:29)."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))


def apply_rotary_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE in fp32, cast back to x's dtype (layers/rotary_embedding.py:6-14)."""
    x1, x2 = torch.chunk(x.float(), 2, dim=-1)
    y1 = x1 * cos - x2 * sin
    y2 = x2 * cos + x1 * sin
    return torch.cat((y1, y2), dim=-1).to(x.dtype)


def section_of_pair(head_dim: int, mrope_section) -> np.ndarray:
    """Section (0 = t, 1 = h, 2 = w) that drives rotation pair i.

    transformers splits the 2*head_dim/2 cos/sin channels into mrope_section * 2
    chunks and takes chunk c from section c % 3; pair i uses channels i and
    i + head_dim/2, which fall in chunks of the same section.
    """
    half = head_dim // 2
    assert sum(mrope_section) == half, "mrope_section must cover head_dim/2 pairs"
    sec = np.empty(half, dtype=np.int64)
    start = 0
    for s, n in enumerate(mrope_section):
        sec[start:start + n] = s
        start += n
    return sec


def rerotation_cos_sin(deltas, head_dim: int, theta: float, mrope_section=None) -> torch.Tensor:
    """fp32 [num_segments, head_dim/2, 2] = (cos, sin) of delta_section(i) * inv_freq[i].

    deltas: [num_segments, 3] integer (dt, dh, dw) per segment, or [num_segments]
    for a 1-D delta.  With mrope_section None all pairs use the t delta.  The
    angle is the fp32 product of the delta and inv_freq, as the reference's
    cos/sin cache computes freqs = t * inv_freq (layers/rotary_embedding.py:30-33).
    """
    d = torch.as_tensor(np.asarray(deltas), dtype=torch.float64)
    if d.dim() == 1:
        d = d[:, None].expand(-1, 3)
    half = head_dim // 2
    sec = np.zeros(half, dtype=np.int64) if mrope_section is None else section_of_pair(head_dim, mrope_section)
    per_pair = d[:, torch.as_tensor(sec)].to(torch.float32)  # [nseg, half]
    ang = per_pair * inv_freq(head_dim, theta)[None, :]
    return torch.stack((ang.cos(), ang.sin()), dim=-1).contiguous()


def rerotate_k(k: torch.Tensor, cos_sin: torch.Tensor, seg: torch.Tensor | None = None) -> torch.Tensor:
    """Rotate cached K rows k [n, Hkv, hd] (bf16) by their segment's (cos, sin).

    fp32 arithmetic of the reference formula, then a cast to k's dtype; pairs
    whose entry is exactly (1, 0) are returned bit for bit.
    """
    n = k.shape[0]
    seg = torch.zeros(n, dtype=torch.long) if seg is None else seg.long()
    cs = cos_sin[seg]  # [n, half, 2]
    cos = cs[..., 0][:, None, :]
    sin = cs[..., 1][:, None, :]
    y = apply_rotary_emb(k, cos, sin)
    ident = ((cs[..., 0] == 1.0) & (cs[..., 1] == 0.0))[:, None, :]
    ident = torch.cat((ident, ident), dim=-1).expand_as(k)
    return torch.where(ident, k, y)


def rerotate_copy_kv(kv_cache: torch.Tensor, old_slots, new_slots, cos_sin=None, seg=None,
                     rotate_k: bool = True) -> None:
    """In place on kv_cache [2, L, num_blocks, block_size, Hkv, hd] (bf16).

    The reference's all-layer copy flat[:, :, new] = flat[:, :, old]
    (engine/model_runner.py:177-180), with K of the copied rows re-rotated.
    """
    s = kv_cache.shape
    flat = kv_cache.view(s[0], s[1], -1, s[4], s[5])
    old = torch.as_tensor(old_slots, dtype=torch.long)
    new = torch.as_tensor(new_slots, dtype=torch.long)
    if old.numel() == 0:
        return
    k_src = flat[0][:, old].clone()  # [L, n, Hkv, hd]
    v_src = flat[1][:, old].clone()
    if rotate_k:
        L = k_src.shape[0]
        k_src = torch.stack([rerotate_k(k_src[l], cos_sin, seg) for l in range(L)])
    flat[0][:, new] = k_src
    flat[1][:, new] = v_src


def vision_position_ids(start: int, grid_thw, spatial_merge_size: int = 2, time_interval: int = 1):
    """int64 [3, T*H*W]: t = start + t_idx*interval, h = start + row, w = start + col.

    Restates get_vision_position_ids (transformers modeling_qwen2_5_vl.py) for
    grid_thw in patches (before the spatial merge).
    """
    t, h, w = (int(grid_thw[0]), int(grid_thw[1]) // spatial_merge_size,
               int(grid_thw[2]) // spatial_merge_size)
    tt, hh, ww = np.meshgrid(np.arange(t) * time_interval, np.arange(h) + start, np.arange(w) + start,
                             indexing="ij")
    pos = np.stack([tt, hh, ww]).reshape(3, -1)
    pos[0] += start
    return pos


def mrope_positions(segments, spatial_merge_size: int = 2):
    """int64 [3, n] M-RoPE positions of a text/image sequence (get_rope_index, images only).

    segments: list of ("text", length) and ("image", (t, h, w) in patches).  Text
    advances all three rows by 1 per token; an image starts at the current
    position and advances it by max(h, w) / merge.
    Returns (positions, image_starts) where image_starts[k] is the start
    position of image k.
    """
    cur = 0
    parts = []
    starts = []
    for kind, val in segments:
        if kind == "text":
            parts.append(np.tile(np.arange(val) + cur, (3, 1)))
            cur += val
        else:
            starts.append(cur)
            parts.append(vision_position_ids(cur, val, spatial_merge_size))
            cur += max(int(val[1]), int(val[2])) // spatial_merge_size
    return np.concatenate(parts, axis=1).astype(np.int64), starts


def rope_cache(max_positions: int, head_dim: int, theta: float) -> torch.Tensor:
    """fp32 [max_positions, 1, head_dim] = cat(cos, sin) of t * inv_freq.

    Restates RotaryEmbedding.__init__ (layers/rotary_embedding.py:29-35): the
    angle of pair i at position t is the single fp32 product t * inv_freq[i].
    """
    t = torch.arange(max_positions, dtype=torch.float)
    freqs = t[:, None] * inv_freq(head_dim, theta)[None, :]
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)[:, None, :]


def rope_rows(positions, cache: torch.Tensor, mrope_section=None):
    """(cos, sin) fp32 [n, 1, head_dim/2] of every token's pairs.

    1-D positions [n]: row positions[n] of the cache for every pair (the
    reference's gather, layers/rotary_embedding.py:45-47).  M-RoPE positions
    [3, n]: pair i reads row positions[section(i), n].
    """
    rows = cache.reshape(cache.shape[0], -1)
    half = rows.shape[1] // 2
    p = torch.as_tensor(np.asarray(positions), dtype=torch.long)
    if p.dim() == 1:
        cs = rows[p]
        return cs[:, None, :half], cs[:, None, half:]
    sec = torch.as_tensor(section_of_pair(2 * half, mrope_section))
    pair = torch.arange(half)
    pp = p[sec]  # [half, n]: position feeding pair i
    cos = rows[pp, pair[:, None]].t()
    sin = rows[pp, half + pair[:, None]].t()
    return cos[:, None, :], sin[:, None, :]


def rope_store_kvcache(positions, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cache: torch.Tensor,
                       mrope_section=None, k_cache: torch.Tensor | None = None,
                       v_cache: torch.Tensor | None = None, slot_mapping=None):
    """Rotated (q, k) and, in place, the paged store of the rotated k and of v.

    The per-layer sequence of models/qwen3.py:84-85: RotaryEmbedding.forward
    (layers/rotary_embedding.py:37-48) on q and k, then store_kvcache
    (layers/attention.py:33-40) of k and v.  q/k/v are bf16 [n, H, hd]; caches
    are bf16 tensors viewed as [num_slots, Hkv * hd]; slot -1 is skipped.
    """
    cos, sin = rope_rows(positions, cache, mrope_section)
    q_rot = apply_rotary_emb(q, cos, sin)
    k_rot = apply_rotary_emb(k, cos, sin)
    if k_cache is not None:
        from .scatter import store_kvcache
        store_kvcache(k_rot.view(torch.int16).numpy(), v.contiguous().view(torch.int16).numpy(),
                      k_cache.view(torch.int16).numpy(), v_cache.view(torch.int16).numpy(),
                      np.asarray(slot_mapping))
    return q_rot, k_rot
