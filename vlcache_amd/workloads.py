"""Warm-request workloads of the partial-recompute prefill path and their work counts.

A warm request is one sequence [text prefix | image | text suffix] whose image KV
is cached from an earlier request.  The first R = ceil(ratio * N) image tokens
are recomputed (engine/block_manager.py:72) together with the text; the other
N - R image tokens are reused.  prepare_prefill (engine/model_runner.py:237-276)
turns it into two virtual sub-sequences: (sq, sk) = (P + R, P + R) and
(S, P + N + S).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

IMAGE_TOKEN_ID = 151655
BLOCK_SIZE = 256


@dataclass(frozen=True)
class ModelShape:
    name: str
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    hidden: int
    rope_theta: float = 1e6
    mrope_section: tuple = (16, 24, 24)


QWEN25_VL_3B = ModelShape("Qwen2.5-VL-3B", 36, 16, 2, 128, 2048)
QWEN25_VL_7B = ModelShape("Qwen2.5-VL-7B", 28, 28, 4, 128, 3584)


def merged_grid(width: int, height: int, patch: int = 14, merge: int = 2, min_pixels: int = 56 * 56,
                max_pixels: int = 28 * 28 * 1280 * 100):
    """(h, w) merged token grid of an image: each side rounded to a multiple of patch*merge.

    The 4K image (3840x2160) gives 77 x 137 = 10549 tokens and 1920x1080 gives
    39 x 69 = 2691 tokens.
    """
    f = patch * merge
    h = max(f, round(height / f) * f)
    w = max(f, round(width / f) * f)
    return h // f, w // f


@dataclass
class WarmRequest:
    prefix: int
    n_image: int
    suffix: int
    ratio: float
    cached_prefix: int  # text prefix length the image KV was cached at
    grid_hw: tuple = (0, 0)

    @property
    def R(self) -> int:
        return math.ceil(self.ratio * self.n_image)

    @property
    def length(self) -> int:
        return self.prefix + self.n_image + self.suffix

    @property
    def n_reused(self) -> int:
        return self.n_image - self.R

    @property
    def n_computed(self) -> int:
        return self.prefix + self.R + self.suffix

    def subseqs(self):
        """[(sq, sk)] of the two virtual sub-sequences (ratio > 0) or of the full sequence."""
        if self.ratio <= 0:
            return [(self.length, self.length)]
        a = self.prefix + self.R
        return [(a, a), (self.suffix, self.length)]

    @property
    def delta(self) -> int:
        return self.prefix - self.cached_prefix


@dataclass
class Workload:
    name: str
    model: ModelShape
    requests: list = field(default_factory=list)

    def cu_seqlens(self):
        cu_q, cu_k = [0], [0]
        for r in self.requests:
            for sq, sk in r.subseqs():
                cu_q.append(cu_q[-1] + sq)
                cu_k.append(cu_k[-1] + sk)
        return cu_q, cu_k


def cfg1() -> Workload:
    """CPU-runnable single layer: 3B shapes, 64 + 1024 (32x32) + 32, ratio 0.1, cached at prefix 16."""
    m = ModelShape("Qwen2.5-VL-3B (1 layer)", 1, 16, 2, 128, 2048)
    return Workload("cfg1-3B-1layer-1k-image-r0.1", m, [WarmRequest(64, 1024, 32, 0.1, 16, (32, 32))])


def cfg2() -> Workload:
    """3B, 36 layers, 128 + 4K image (77x137 = 10549) + 64, ratio 0.1, cached at prefix 40."""
    h, w = merged_grid(3840, 2160)
    return Workload("cfg2-3B-4k-image-r0.1", QWEN25_VL_3B, [WarmRequest(128, h * w, 64, 0.1, 40, (h, w))])


def cfg3() -> Workload:
    """3B, 4K image, ratio 0.0: dense causal prefill of the whole 10741-token sequence."""
    h, w = merged_grid(3840, 2160)
    return Workload("cfg3-3B-4k-image-full-recompute", QWEN25_VL_3B,
                    [WarmRequest(128, h * w, 64, 0.0, 128, (h, w))])


def cfg4(seed: int = 0) -> Workload:
    """3B, 8 warm requests sharing one cached 4K image; prefixes U[16,512], suffixes U[16,256]."""
    h, w = merged_grid(3840, 2160)
    rng = np.random.default_rng(seed)
    pre = rng.integers(16, 513, size=8)
    suf = rng.integers(16, 257, size=8)
    reqs = [WarmRequest(int(p), h * w, int(s), 0.05, 128, (h, w)) for p, s in zip(pre, suf)]
    return Workload("cfg4-3B-8seq-shared-4k-image-r0.05", QWEN25_VL_3B, reqs)


def attention_flops(cu_seqlens_q, cu_seqlens_k, num_heads_q: int, head_dim: int, causal: bool = True) -> int:
    """4 * hd * Hq * (unmasked (query, key) pairs); bottom-right causal; softmax excluded."""
    pairs = 0
    for b in range(len(cu_seqlens_q) - 1):
        sq = int(cu_seqlens_q[b + 1]) - int(cu_seqlens_q[b])
        sk = int(cu_seqlens_k[b + 1]) - int(cu_seqlens_k[b])
        if causal:
            i = np.arange(sq, dtype=np.int64)
            pairs += int(np.clip(i + 1 + sk - sq, 0, sk).sum())
        else:
            pairs += sq * sk
    return 4 * head_dim * num_heads_q * pairs


def rerotate_bytes(n_tokens: int, num_layers: int, num_kv_heads: int, head_dim: int, with_v: bool = True) -> int:
    """HBM bytes of the all-layer reuse copy: each row read once and written once (bf16)."""
    planes = 2 if with_v else 1
    return planes * num_layers * n_tokens * num_kv_heads * head_dim * 2 * 2


def scatter_bytes(n_tokens: int, num_kv_heads: int, head_dim: int) -> int:
    """HBM bytes of one layer's store_kvcache: K and V rows read and written (bf16)."""
    return 2 * n_tokens * num_kv_heads * head_dim * 2 * 2


def rope_store_bytes(n_tokens: int, num_heads: int, num_kv_heads: int, head_dim: int) -> int:
    """HBM bytes of one layer's fused RoPE + KV store.

    q rows read and written, k and v rows read and written to the cache (bf16),
    plus per token its cos/sin row (head_dim fp32), three int64 positions and
    the int32 slot.
    """
    rows = 2 * (num_heads + 2 * num_kv_heads) * head_dim * 2
    return n_tokens * (rows + head_dim * 4 + 3 * 8 + 4)
