"""Rotary embeddings of the text decoder: 1-D RoPE and Qwen2.5-VL's M-RoPE.

apply_rotary_emb and RotaryEmbedding follow layers/rotary_embedding.py:6-48 of
the reference (rotate-half pairs (i, i + hd/2), fp32 math, a cos/sin cache of
max_position rows), evaluated eagerly.  The reference's get_rope ignores
rope_scaling (:51-60) and so never applies Qwen2.5-VL's three position
sections; MRotaryEmbedding adds them: positions are [3, N] (temporal, height,
width) and pair i takes its angle from section(i) of mrope_section
(e.g. [16, 24, 24]: pairs 0-15 temporal, 16-39 height, 40-63 width).
"""
from __future__ import annotations

import torch
from torch import nn


def apply_rotary_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    x1, x2 = torch.chunk(x.float(), 2, dim=-1)
    y1 = x1 * cos - x2 * sin
    y2 = x2 * cos + x1 * sin
    return torch.cat((y1, y2), dim=-1).to(x.dtype)


def inv_freq(rotary_dim: int, base: float) -> torch.Tensor:
    return 1.0 / (base ** (torch.arange(0, rotary_dim, 2, dtype=torch.float) / rotary_dim))


class RotaryEmbedding(nn.Module):

    def __init__(self, head_size: int, rotary_dim: int, max_position_embeddings: int, base: float) -> None:
        super().__init__()
        assert rotary_dim == head_size
        self.head_size = head_size
        self.base = base
        freqs = torch.einsum("i,j -> ij", torch.arange(max_position_embeddings, dtype=torch.float),
                             inv_freq(rotary_dim, base))
        cache = torch.cat((freqs.cos(), freqs.sin()), dim=-1).unsqueeze_(1)
        self.register_buffer("cos_sin_cache", cache, persistent=False)

    def _cos_sin(self, positions: torch.Tensor):
        cos_sin = self.cos_sin_cache[positions]
        return cos_sin.chunk(2, dim=-1)

    def forward(self, positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor):
        cos, sin = self._cos_sin(positions)
        return apply_rotary_emb(query, cos, sin), apply_rotary_emb(key, cos, sin)


class MRotaryEmbedding(RotaryEmbedding):
    """M-RoPE: positions [3, N]; pair i rotates by positions[section(i)] * inv_freq[i]."""

    def __init__(self, head_size: int, rotary_dim: int, max_position_embeddings: int, base: float,
                 mrope_section) -> None:
        super().__init__(head_size, rotary_dim, max_position_embeddings, base)
        assert sum(mrope_section) == rotary_dim // 2
        self.mrope_section = tuple(int(x) for x in mrope_section)
        sec = torch.repeat_interleave(torch.arange(3), torch.tensor(self.mrope_section))
        self.register_buffer("pair_section", sec, persistent=False)

    def _cos_sin(self, positions: torch.Tensor):
        if positions.dim() == 1:
            return super()._cos_sin(positions)
        half = self.head_size // 2
        rows = self.cos_sin_cache[:, 0]                      # [max_pos, hd] = (cos | sin)
        pair = torch.arange(half, device=positions.device)
        p = positions[self.pair_section.to(positions.device)]  # [half, N]: position feeding pair i
        cos = rows[p, pair[:, None]].t()                     # [N, half]
        sin = rows[p, half + pair[:, None]].t()
        return cos.unsqueeze(1), sin.unsqueeze(1)


def get_rope(head_size: int, rotary_dim: int, max_position: int, base: float, rope_scaling: dict | None = None):
    section = (rope_scaling or {}).get("mrope_section") if isinstance(rope_scaling, dict) else None
    if section:
        return MRotaryEmbedding(head_size, rotary_dim, max_position, base, section)
    return RotaryEmbedding(head_size, rotary_dim, max_position, base)
