"""Qwen2.5-VL vision tower (the cold path in front of the encoder cache).

Mirrors Qwen2_5_VisionTransformer (models/qwen2_5_vl.py:341-527) and what it
calls: patch embedding, window permutation, 32 blocks of RMSNorm + attention +
SwiGLU MLP (:219-305), the 2x2 patch merger (:308-338) and the inverse
permutation.  Most blocks attend within windows of 4x4 merged units (8x8
patches); the blocks in fullatt_block_indexes attend over whole images.

On gfx950:
  * the window layout (window order, window and image boundaries, patch
    positions) is integer host work, vectorised with numpy, computed once per
    batch of images;
  * each block's q/k rotation and the split of the QKV projection into
    128-dim head rows run as one kernel (vlc_vision_rope_pad);
  * attention runs on the varlen attention kernel in its contiguous,
    non-causal mode (the reference calls flash_attn_varlen_func with
    causal=False and cu_seqlens_q == cu_seqlens_k, :200-210), in its 80-dim
    variant: heads stay zero-padded 128-element rows, the products skip the
    padding; one work plan per boundary list serves every block;
  * each RMSNorm (with its residual add) and the MLP's SiLU-and-multiply run
    as one kernel each; GEMMs and the merger's GELU run on torch (hipBLASLt).

As in the reference, the rotary angles are rounded to bf16 before cos/sin
(:486-487) and the rotation itself is bf16 arithmetic.  The Conv3d patch
embedding (kernel == stride) is a GEMM over flattened patches.
"""
from __future__ import annotations

from collections import OrderedDict
from types import SimpleNamespace

import numpy as np
import torch
from torch import nn

from . import kernels
from .layers.layernorm import RMSNorm

# Public Qwen2.5-VL vision_config values (3B and 7B share them but out_hidden_size).
VISION_DEFAULTS = dict(depth=32, hidden_size=1280, intermediate_size=3420, num_heads=16, in_channels=3,
                       patch_size=14, temporal_patch_size=2, spatial_merge_size=2, window_size=112,
                       fullatt_block_indexes=[7, 15, 23, 31], hidden_act="silu")


def vision_config(d: dict | None, out_hidden_size: int) -> SimpleNamespace:
    """A checkpoint's vision_config over the public defaults; out_hidden_size defaults to the text hidden size."""
    d = dict(d or {})
    v = dict(VISION_DEFAULTS, out_hidden_size=out_hidden_size)
    v.update({k: val for k, val in d.items() if val is not None})
    if "in_chans" in d and "in_channels" not in d:
        v["in_channels"] = d["in_chans"]
    if v["hidden_size"] % v["num_heads"]:
        raise ValueError("vision hidden_size must be a multiple of num_heads")
    if v["hidden_act"] != "silu":
        raise ValueError(f"vision hidden_act {v['hidden_act']!r} is not supported (silu only)")
    return SimpleNamespace(**v)


class VisionLayout:
    """Host-side integer layout of one batch of images (models/qwen2_5_vl.py:93-126, :392-441, :465-503).

    window_index: merged units in window order (units row-major within a window,
    windows row-major within a frame, frames and images in order); cu_window:
    window boundaries in patches, empty windows dropped; cu_full: one sequence
    per image (t*h*w patches); patch_order: the patch permutation that window
    order implies; pos_hw: (row, column) of each patch in window order;
    reverse: the unit permutation back to image order.
    """

    def __init__(self, grids, window_size: int, merge: int, patch: int):
        self.grids = [tuple(int(v) for v in g) for g in grids]
        ws = window_size // merge // patch
        if ws <= 0:
            raise ValueError("window_size must cover at least one merged unit")
        unit = merge * merge
        orders, lens, pos, cu_full = [], [], [], [0]
        base = 0
        for t, h, w in self.grids:
            if t <= 0 or h <= 0 or w <= 0 or h % merge or w % merge:
                raise ValueError(f"image grid {(t, h, w)} is not a positive multiple of the merge size")
            lh, lw = h // merge, w // merge
            ti, r, c = (a.ravel() for a in np.meshgrid(np.arange(t), np.arange(lh), np.arange(lw),
                                                     indexing="ij"))
            wr, wc = r // ws, c // ws
            orders.append(np.lexsort((c, r, wc, wr, ti)) + base)
            nwh, nww = -(-lh // ws), -(-lw // ws)
            counts = np.bincount((ti * nwh + wr) * nww + wc, minlength=t * nwh * nww)
            lens.append(counts[counts > 0])
            # patch (row, column) of unit (r, c), sub-patch (i, j): (r*m + i, c*m + j)
            sub = np.arange(unit)
            pos.append(np.stack([(r[:, None] * merge + sub[None, :] // merge).ravel(),
                                 (c[:, None] * merge + sub[None, :] % merge).ravel()], axis=-1))
            cu_full.append(cu_full[-1] + t * h * w)
            base += t * lh * lw
        self.num_units = base
        self.num_patches = base * unit
        self.window_index = np.concatenate(orders) if orders else np.zeros(0, np.int64)
        self.cu_window = [0] + (np.cumsum(np.concatenate(lens)) * unit).tolist() if lens else [0]
        self.cu_full = cu_full
        self.patch_order = (self.window_index[:, None] * unit + np.arange(unit)[None, :]).ravel()
        pos_all = np.concatenate(pos) if pos else np.zeros((0, 2), np.int64)
        self.pos_hw = np.ascontiguousarray(pos_all[self.patch_order].astype(np.int32))
        self.reverse = np.argsort(self.window_index, kind="stable")
        self.max_pos = max((max(h, w) for _, h, w in self.grids), default=1)


class VisionMLP(nn.Module):
    """SwiGLU with biases (models/qwen2_5_vl.py:219-243); SiLU-and-multiply as one kernel."""

    def __init__(self, dim: int, inter: int):
        super().__init__()
        self.inter = inter
        self.gate_up_proj = nn.Linear(dim, 2 * inter, bias=True)
        self.down_proj = nn.Linear(inter, dim, bias=True)

    def forward(self, x):
        return self.down_proj(kernels.silu_mul(self.gate_up_proj(x)))


class VisionAttention(nn.Module):
    """QKV projection, 2-D rotary, non-causal varlen attention, output projection (:128-216)."""

    def __init__(self, dim: int, num_heads: int):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        if self.head_dim > kernels.HEAD_DIM or self.head_dim % 16:
            raise ValueError(f"vision head_dim {self.head_dim} is not supported (a multiple of 16, <= 128)")
        self.qkv = nn.Linear(dim, 3 * dim, bias=True)
        self.proj = nn.Linear(dim, dim, bias=True)

    def forward(self, x, run: "_Run", full: bool):
        n = x.shape[0]
        qkv = self.qkv(x)
        heads = kernels.vision_rope_pad(qkv, run.pos_hw, run.cos, run.sin, self.num_heads, self.head_dim)
        cu, plan = (run.cu_full, run.plan_full) if full else (run.cu_window, run.plan_window)
        o = kernels.varlen_attention(heads[:, 0], heads[:, 1], heads[:, 2], cu, cu, self.head_dim ** -0.5,
                                     causal=False, plan=plan, head_dim=run.attn_head_dim)
        return self.proj(o[..., :self.head_dim].reshape(n, self.num_heads * self.head_dim))


class VisionBlock(nn.Module):
    """(:246-305): x + attn(norm1(x)), then the residual add fused into norm2, + mlp."""

    def __init__(self, dim: int, inter: int, num_heads: int, eps: float):
        super().__init__()
        self.norm1 = RMSNorm(dim, eps)
        self.norm2 = RMSNorm(dim, eps)
        self.attn = VisionAttention(dim, num_heads)
        self.mlp = VisionMLP(dim, inter)

    def forward(self, x, run, full: bool):
        a = self.attn(self.norm1(x), run, full)
        h, x = self.norm2(x, a)
        return x + self.mlp(h)


class PatchMerger(nn.Module):
    """RMSNorm, 2x2 units to one row, Linear-GELU-Linear (:308-338)."""

    def __init__(self, out_dim: int, dim: int, merge: int):
        super().__init__()
        self.hidden = dim * merge * merge
        self.ln_q = RMSNorm(dim, 1e-6)
        self.mlp = nn.Sequential(nn.Linear(self.hidden, self.hidden), nn.GELU(), nn.Linear(self.hidden, out_dim))

    def forward(self, x):
        return self.mlp(self.ln_q(x).view(-1, self.hidden))


class _Run:
    """Device-side inputs of one forward shared by every block."""

    def __init__(self, **kw):
        self.__dict__.update(kw)


class VisionTransformer(nn.Module):
    """Pixel patches [sum t*h*w, C*T*P*P] + grids -> visual embeddings [sum t*h*w/4, out_hidden]."""

    def __init__(self, cfg: SimpleNamespace, eps: float = 1e-6, plan_cache: int = 8):
        super().__init__()
        self.cfg = cfg
        dim = cfg.hidden_size
        self.merge = cfg.spatial_merge_size
        self.patch_dim = cfg.in_channels * cfg.temporal_patch_size * cfg.patch_size * cfg.patch_size
        self.head_dim = dim // cfg.num_heads
        self.patch_embed = nn.Linear(self.patch_dim, dim, bias=False)
        self.blocks = nn.ModuleList(VisionBlock(dim, cfg.intermediate_size, cfg.num_heads, eps)
                                    for _ in range(cfg.depth))
        self.merger = PatchMerger(cfg.out_hidden_size, dim, self.merge)
        self.full = set(int(i) for i in cfg.fullatt_block_indexes)
        d = self.head_dim // 2
        # theta^(-2i/d), theta = 1e4 (Qwen2_5_VisionRotaryEmbedding, built where the model is built)
        self.register_buffer("inv_freq", 1.0 / (10000.0 ** (torch.arange(0, d, 2, dtype=torch.float) / d)),
                             persistent=False)
        self._runs: OrderedDict = OrderedDict()
        self._plan_cache = plan_cache

    @property
    def device(self):
        return self.patch_embed.weight.device

    @property
    def dtype(self):
        return self.patch_embed.weight.dtype

    def rope_tables(self, max_pos: int):
        """bf16 cos/sin [max_pos, head_dim/4] of the bf16-rounded angles p * inv_freq (:452-462, :486-487)."""
        ang = torch.arange(max_pos, dtype=torch.float, device=self.device)[:, None] * self.inv_freq[None, :]
        ang = ang.to(torch.bfloat16)
        return ang.cos().contiguous(), ang.sin().contiguous()

    def _prepare(self, grids) -> _Run:
        key = tuple(tuple(int(v) for v in g) for g in grids)
        run = self._runs.get(key)
        if run is not None:
            self._runs.move_to_end(key)
            return run
        cfg = self.cfg
        lay = VisionLayout(key, cfg.window_size, self.merge, cfg.patch_size)
        dev = self.device
        h = cfg.num_heads

        def cu_t(cu):
            return torch.tensor(cu, dtype=torch.int32, device=dev)

        cos, sin = self.rope_tables(lay.max_pos)
        # 80-dim heads have a kernel of their own; other widths run as zero-padded 128-dim heads
        ahd = self.head_dim if self.head_dim in kernels.ATTN_HEAD_DIMS else kernels.HEAD_DIM
        run = _Run(layout=lay, attn_head_dim=ahd,
                   patch_order=torch.from_numpy(lay.patch_order).to(dev),
                   reverse=torch.from_numpy(lay.reverse).to(dev),
                   pos_hw=torch.from_numpy(lay.pos_hw).to(dev),
                   cos=cos, sin=sin,
                   cu_window=cu_t(lay.cu_window), cu_full=cu_t(lay.cu_full),
                   plan_window=kernels.plan_attention(lay.cu_window, lay.cu_window, h, h, ahd, False, dev),
                   plan_full=kernels.plan_attention(lay.cu_full, lay.cu_full, h, h, ahd, False, dev))
        self._runs[key] = run
        while len(self._runs) > self._plan_cache:
            self._runs.popitem(last=False)
        return run

    @torch.inference_mode()
    def forward(self, pixel_values: torch.Tensor, grids) -> torch.Tensor:
        run = self._prepare(grids)
        lay = run.layout
        if pixel_values.dim() != 2 or pixel_values.shape != (lay.num_patches, self.patch_dim):
            raise ValueError(f"pixel_values must be [{lay.num_patches}, {self.patch_dim}] for grids {lay.grids}, "
                             f"got {tuple(pixel_values.shape)}")
        pix = pixel_values.to(self.device, self.dtype)
        x = self.patch_embed(pix.index_select(0, run.patch_order))
        for i, blk in enumerate(self.blocks):
            x = blk(x, run, i in self.full)
        return self.merger(x).index_select(0, run.reverse)

    @torch.no_grad()
    def load_checkpoint_weights(self, weights: dict) -> None:
        """Load checkpoint-named tensors (patch_embed.proj.weight [hidden, C, T, P, P],
        blocks.i.mlp.{gate,up}_proj packed into gate_up_proj, the rest by name)."""
        own = dict(self.named_parameters())
        used = set()
        for name, t in weights.items():
            if name == "patch_embed.proj.weight":
                own["patch_embed.weight"].copy_(t.reshape(t.shape[0], -1))
            elif ".mlp.gate_proj." in name or ".mlp.up_proj." in name:
                tgt = own[name.replace(".gate_proj.", ".gate_up_proj.").replace(".up_proj.", ".gate_up_proj.")]
                half = tgt.shape[0] // 2
                (tgt[:half] if ".gate_proj." in name else tgt[half:]).copy_(t)
                used.add(name.replace(".gate_proj.", ".gate_up_proj.").replace(".up_proj.", ".gate_up_proj."))
                continue
            else:
                own[name].copy_(t)
            used.add("patch_embed.weight" if name == "patch_embed.proj.weight" else name)
        missing = set(own) - used
        if missing:
            raise KeyError(f"vision weights missing: {sorted(missing)[:5]}")
