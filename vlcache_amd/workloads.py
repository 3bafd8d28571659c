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
    """One warm request.  Single image: prefix text, an image of n_image tokens (merged
    grid grid_hw), suffix text.  Several images: `layout`, a tuple of ("text", n) and
    ("image", (h, w)) parts.  Every image was cached standalone after cached_prefix
    text tokens; each keeps its first ceil(ratio * N) tokens recomputed."""
    prefix: int = 0
    n_image: int = 0
    suffix: int = 0
    ratio: float = 0.0
    cached_prefix: int = 0  # text prefix length the image KV was cached at
    grid_hw: tuple = (0, 0)
    layout: tuple | None = None

    def parts(self):
        if self.layout is not None:
            return list(self.layout)
        parts = [("text", self.prefix), ("image", tuple(self.grid_hw)), ("text", self.suffix)]
        return [p for p in parts if p[0] == "image" or p[1] > 0]

    def images(self):
        """[(start, end, (h, w))] token range of each image."""
        out, p = [], 0
        for kind, val in self.parts():
            n = val if kind == "text" else int(val[0]) * int(val[1])
            if kind == "image":
                out.append((p, p + n, (int(val[0]), int(val[1]))))
            p += n
        return out

    def rope_starts(self):
        """M-RoPE start position of each image: text advances 1 per token, an image max(h, w)."""
        out, cur = [], 0
        for kind, val in self.parts():
            if kind == "text":
                cur += val
            else:
                out.append(cur)
                cur += max(int(val[0]), int(val[1]))
        return out

    def recompute(self):
        """Recomputed tokens of each image: ceil(ratio * N) (IEEE double), all of it at ratio 0."""
        return [math.ceil(self.ratio * (e - s)) if self.ratio > 0 else e - s for s, e, _ in self.images()]

    @property
    def R(self) -> int:
        return self.recompute()[0]

    @property
    def length(self) -> int:
        return sum(v if k == "text" else int(v[0]) * int(v[1]) for k, v in self.parts())

    @property
    def n_reused(self) -> int:
        return sum((e - s) - r for (s, e, _), r in zip(self.images(), self.recompute()))

    @property
    def n_computed(self) -> int:
        return self.length - self.n_reused

    def runs(self):
        """Maximal runs [a, b) of computed tokens (one image: [0, P + R) and [P + N, len))."""
        if self.ratio <= 0:
            return [(0, self.length)]
        runs, p = [], 0
        for (s, e, _), r in zip(self.images(), self.recompute()):
            if s + r < e:
                if s + r > p:
                    runs.append((p, s + r))
                p = e
        if p < self.length:
            runs.append((p, self.length))
        return runs

    def subseqs(self):
        """[(sq, sk)] of the virtual sub-sequences: queries [a, b), keys [0, b)."""
        return [(b - a, b) for a, b in self.runs()]

    def deltas(self):
        """Rotary shift of each image: its start here minus its start when cached."""
        return [st - self.cached_prefix for st in self.rope_starts()]

    @property
    def delta(self) -> int:
        return self.deltas()[0]


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


def _shape_3b(num_layers: int) -> ModelShape:
    if num_layers == QWEN25_VL_3B.num_layers:
        return QWEN25_VL_3B
    return ModelShape(f"Qwen2.5-VL-3B ({num_layers} layers)", num_layers, 16, 2, 128, 2048)


def cfg2(num_layers: int = 36) -> Workload:
    """3B, 36 layers, 128 + 4K image (77x137 = 10549) + 64, ratio 0.1, cached at prefix 40."""
    h, w = merged_grid(3840, 2160)
    return Workload("cfg2-3B-4k-image-r0.1", _shape_3b(num_layers),
                    [WarmRequest(128, h * w, 64, 0.1, 40, (h, w))])


def cfg3(num_layers: int = 36) -> Workload:
    """3B, 4K image, ratio 0.0: dense causal prefill of the whole 10741-token sequence."""
    h, w = merged_grid(3840, 2160)
    return Workload("cfg3-3B-4k-image-full-recompute", _shape_3b(num_layers),
                    [WarmRequest(128, h * w, 64, 0.0, 128, (h, w))])


def cfg4(seed: int = 0, num_layers: int = 36) -> Workload:
    """3B, 8 warm requests sharing one cached 4K image; prefixes U[16,512], suffixes U[16,256]."""
    h, w = merged_grid(3840, 2160)
    rng = np.random.default_rng(seed)
    pre = rng.integers(16, 513, size=8)
    suf = rng.integers(16, 257, size=8)
    reqs = [WarmRequest(int(p), h * w, int(s), 0.05, 128, (h, w)) for p, s in zip(pre, suf)]
    return Workload("cfg4-3B-8seq-shared-4k-image-r0.05", _shape_3b(num_layers), reqs)


def cfg5(num_layers: int = 28) -> Workload:
    """7B, batch 4, two images per request: 64 text + 1920x1080 image (39x69 = 2691) + 64 text
    + 4K image (77x137 = 10549) + 64 text = 13432 tokens, ratio 0.02, each image cached
    standalone after 64 text tokens (image 1 keeps its rotary start, image 2 moves by 133)."""
    g1, g2 = merged_grid(1920, 1080), merged_grid(3840, 2160)
    layout = (("text", 64), ("image", g1), ("text", 64), ("image", g2), ("text", 64))
    m = QWEN25_VL_7B if num_layers == QWEN25_VL_7B.num_layers else ModelShape(
        f"Qwen2.5-VL-7B ({num_layers} layers)", num_layers, 28, 4, 128, 3584)
    reqs = [WarmRequest(ratio=0.02, cached_prefix=64, layout=layout) for _ in range(4)]
    return Workload("cfg5-7B-4seq-two-images-r0.02", m, reqs)


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
