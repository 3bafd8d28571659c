"""fp32 oracle of the Qwen2.5-VL vision tower as the reference runs it (test-only).

Restates models/qwen2_5_vl.py:93-531 on the CPU:

* rot_pos_ids            :93-126   (h, w) of every patch, merge-unit blocks row-major;
* window_index           :392-441  merged units regrouped into windows of
                                   window_size // merge // patch units a side, plus
                                   the window boundaries (x merge unit) with empty
                                   windows dropped (torch.unique_consecutive, :477);
* full_cu_seqlens        :494-503  one sequence per image (the reference prepends an
                                   extra 0, an empty first sequence: omitted here);
* rotary_angles          :452-462, :486-487  p * inv_freq with inv_freq =
                                   theta^(-2i/d), theta 1e4, d = head_dim / 2 (the
                                   HF Qwen2_5_VisionRotaryEmbedding the reference
                                   imports); the reference casts these angles to the
                                   activation dtype BEFORE cos/sin (:486), bf16_angles
                                   reproduces that rounding;
* rope_bf16              :180-199  q*cos + rotate_half(q)*sin with every product and
                                   the sum rounded to bf16 (the reference's cos/sin
                                   and q are bf16 tensors);
* vision_forward         :465-527  patch embed (Conv3d with kernel == stride, a
                                   GEMM over flattened patches), window permutation,
                                   blocks (:292-305: RMSNorm, attention over windows
                                   or whole images per fullatt_block_indexes,
                                   residual add fused into the second RMSNorm,
                                   SwiGLU MLP with biases), merger (:319-338:
                                   RMSNorm, 4 units -> one row, Linear-GELU-Linear),
                                   inverse permutation.

Parameters use the checkpoint's names (HF Qwen2_5_VisionTransformerPretrainedModel:
patch_embed.proj.weight [hidden, C, T, P, P]; blocks.i.{norm1,norm2}.weight;
blocks.i.attn.{qkv,proj}.{weight,bias}; blocks.i.mlp.{gate_proj,up_proj,down_proj}.
{weight,bias}; merger.ln_q.weight; merger.mlp.{0,2}.{weight,bias}).

Pinned in tests/test_oracle_vision.py: rot_pos_ids, window_index and full_cu_seqlens
against transformers' get_vision_position_ids / get_vision_window_index /
get_vision_attention_seqlens (an independent implementation in this image) and a
hand-derived known answer; vision_forward with bf16_angles=False against
transformers' Qwen2_5_VisionTransformerPretrainedModel in fp32 on tiny configs;
rotary_angles' bf16 rounding by a closed form (the angle table is
bf16(p * inv_freq)); rope_bf16 against the fp32 rotation (within 2 bf16 ulps) and
exactly at angle 0.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


def rot_pos_ids(t: int, h: int, w: int, merge: int) -> np.ndarray:
    """[t*h*w, 2] (row, col) of every patch in the processor's order (:93-126, :452-456)."""
    r = np.arange(h).reshape(h // merge, merge, 1, 1)
    c = np.arange(w).reshape(1, 1, w // merge, merge)
    hh = np.broadcast_to(r, (h // merge, merge, w // merge, merge)).transpose(0, 2, 1, 3).reshape(-1)
    ww = np.broadcast_to(c, (h // merge, merge, w // merge, merge)).transpose(0, 2, 1, 3).reshape(-1)
    one = np.stack([hh, ww], axis=-1)
    return np.tile(one, (t, 1))


def window_index(grids, window_size: int, merge: int, patch: int):
    """(window_index [units], cu_window_seqlens list) over several images (:392-441, :477).

    Loops over every padded window as the reference does: a window of the padded
    grid contributes its valid units in row-major order, and its length times the
    merge unit to the boundaries; zero-length windows are then dropped.
    """
    ws = window_size // merge // patch
    unit = merge * merge
    index, cu, base = [], [0], 0
    for t, h, w in grids:
        lh, lw = h // merge, w // merge
        pad_h, pad_w = ws - lh % ws, ws - lw % ws   # a full extra window when divisible (:409-410)
        nwh, nww = (lh + pad_h) // ws, (lw + pad_w) // ws
        for ti in range(t):
            for a in range(nwh):
                for b in range(nww):
                    n = 0
                    for r in range(a * ws, (a + 1) * ws):
                        for c in range(b * ws, (b + 1) * ws):
                            if r < lh and c < lw:
                                index.append(base + ti * lh * lw + r * lw + c)
                                n += 1
                    cu.append(cu[-1] + n * unit)
        base += t * lh * lw
    dedup = [cu[0]] + [x for p, x in zip(cu, cu[1:]) if x != p]
    return np.asarray(index, dtype=np.int64), dedup


def full_cu_seqlens(grids) -> list[int]:
    """One sequence per image (:494-503), without the reference's leading empty sequence."""
    cu = [0]
    for t, h, w in grids:
        cu.append(cu[-1] + t * h * w)
    return cu


def inv_freq(head_dim: int, theta: float = 10000.0) -> torch.Tensor:
    d = head_dim // 2
    return 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float) / d))


def rotary_angles(pos: np.ndarray, head_dim: int, bf16_angles: bool = True) -> torch.Tensor:
    """[N, head_dim/2] angles (h-axis frequencies, then w-axis) of patches at `pos` [N, 2]."""
    f = inv_freq(head_dim)
    p = torch.as_tensor(np.asarray(pos), dtype=torch.float32)
    ang = (p[:, :, None] * f[None, None, :]).reshape(p.shape[0], -1)
    if bf16_angles:
        ang = ang.to(torch.bfloat16).float()
    return ang


def rope_bf16(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [N, H, D] bf16, cos/sin [N, D] bf16 -> bf16, rounded after each product and the sum."""
    half = x.shape[-1] // 2
    xr = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    a = (x.float() * cos[:, None, :].float()).to(torch.bfloat16)
    b = (xr.float() * sin[:, None, :].float()).to(torch.bfloat16)
    return (a.float() + b.float()).to(torch.bfloat16)


def _rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def _rope_f32(x, cos, sin):
    half = x.shape[-1] // 2
    return x * cos[:, None, :] + torch.cat((-x[..., half:], x[..., :half]), dim=-1) * sin[:, None, :]


def _attention(q, k, v, cu, scale):
    out = torch.empty_like(q)
    for s, e in zip(cu, cu[1:]):
        if e == s:
            continue
        qs, ks, vs = (t[s:e].transpose(0, 1) for t in (q, k, v))   # [H, L, D]
        p = torch.softmax((qs @ ks.transpose(1, 2)) * scale, dim=-1)
        out[s:e] = (p @ vs).transpose(0, 1)
    return out


def vision_forward(params: dict, pixel_values: torch.Tensor, grids, cfg: dict,
                   bf16_angles: bool = True, eps: float = 1e-6) -> torch.Tensor:
    """[sum t*h*w / merge^2, out_hidden] fp32 embeddings of the images (:465-527)."""
    P = {k: v.float() for k, v in params.items()}
    hidden, heads = cfg["hidden_size"], cfg["num_heads"]
    hd = hidden // heads
    merge = cfg["spatial_merge_size"]
    unit = merge * merge
    wproj = P["patch_embed.proj.weight"].reshape(hidden, -1)
    x = pixel_values.float().reshape(pixel_values.shape[0], -1) @ wproj.t()
    pos = np.concatenate([rot_pos_ids(t, h, w, merge) for t, h, w in grids])
    widx, cu_win = window_index(grids, cfg["window_size"], merge, cfg["patch_size"])
    cu_full = full_cu_seqlens(grids)
    n = x.shape[0]
    x = x.reshape(n // unit, unit, hidden)[torch.as_tensor(widx)].reshape(n, hidden)
    pos = pos.reshape(n // unit, unit, 2)[widx].reshape(n, 2)
    ang = rotary_angles(pos, hd, bf16_angles)
    emb = torch.cat((ang, ang), dim=-1)
    cos, sin = emb.cos(), emb.sin()
    scale = hd ** -0.5
    full = set(cfg["fullatt_block_indexes"])
    for i in range(cfg["depth"]):
        b = f"blocks.{i}."
        hn = _rms(x, P[b + "norm1.weight"], eps)
        qkv = hn @ P[b + "attn.qkv.weight"].t() + P[b + "attn.qkv.bias"]
        q, k, v = qkv.reshape(n, 3, heads, hd).unbind(1)
        q, k = _rope_f32(q, cos, sin), _rope_f32(k, cos, sin)
        o = _attention(q, k, v, cu_full if i in full else cu_win, scale).reshape(n, hidden)
        x = x + (o @ P[b + "attn.proj.weight"].t() + P[b + "attn.proj.bias"])
        hn = _rms(x, P[b + "norm2.weight"], eps)
        g = hn @ P[b + "mlp.gate_proj.weight"].t() + P[b + "mlp.gate_proj.bias"]
        u = hn @ P[b + "mlp.up_proj.weight"].t() + P[b + "mlp.up_proj.bias"]
        x = x + ((F.silu(g) * u) @ P[b + "mlp.down_proj.weight"].t() + P[b + "mlp.down_proj.bias"])
    m = _rms(x, P["merger.ln_q.weight"], eps).reshape(-1, unit * hidden)
    m = F.gelu(m @ P["merger.mlp.0.weight"].t() + P["merger.mlp.0.bias"])
    m = m @ P["merger.mlp.2.weight"].t() + P["merger.mlp.2.bias"]
    rev = np.argsort(widx)
    return m[torch.as_tensor(rev)]


def random_params(cfg: dict, seed: int = 0, in_channels: int = 3, temporal: int = 2,
                  qkv_std: float | None = None) -> dict:
    """Seeded checkpoint-named parameters, rounded to bf16 values (fp32 tensors).

    qkv weights default to std 1/sqrt(hidden), so attention scores are O(1) and the
    softmax is far from uniform; the other projections use 0.5/sqrt(fan_in) and
    norm weights 1 +- 0.1, keeping the residual stream bounded over many blocks.
    """
    g = torch.Generator().manual_seed(seed)
    hid, inter, out = cfg["hidden_size"], cfg["intermediate_size"], cfg["out_hidden_size"]
    unit = cfg["spatial_merge_size"] ** 2
    patch = cfg["patch_size"]

    def w(o, i, std=None):
        return torch.randn(o, i, generator=g) * (std if std is not None else 0.5 / math.sqrt(i))

    def bias(o):
        return torch.randn(o, generator=g) * 0.02

    def norm(o):
        return 1.0 + 0.1 * torch.randn(o, generator=g)

    p = {"patch_embed.proj.weight": w(hid, in_channels * temporal * patch * patch, 1.0 / math.sqrt(
        in_channels * temporal * patch * patch)).reshape(hid, in_channels, temporal, patch, patch)}
    for i in range(cfg["depth"]):
        b = f"blocks.{i}."
        p[b + "norm1.weight"] = norm(hid)
        p[b + "norm2.weight"] = norm(hid)
        p[b + "attn.qkv.weight"] = w(3 * hid, hid, qkv_std if qkv_std is not None else 1.0 / math.sqrt(hid))
        p[b + "attn.qkv.bias"] = bias(3 * hid)
        p[b + "attn.proj.weight"] = w(hid, hid)
        p[b + "attn.proj.bias"] = bias(hid)
        p[b + "mlp.gate_proj.weight"] = w(inter, hid)
        p[b + "mlp.gate_proj.bias"] = bias(inter)
        p[b + "mlp.up_proj.weight"] = w(inter, hid)
        p[b + "mlp.up_proj.bias"] = bias(inter)
        p[b + "mlp.down_proj.weight"] = w(hid, inter)
        p[b + "mlp.down_proj.bias"] = bias(hid)
    p["merger.ln_q.weight"] = norm(hid)
    p["merger.mlp.0.weight"] = w(unit * hid, unit * hid)
    p["merger.mlp.0.bias"] = bias(unit * hid)
    p["merger.mlp.2.weight"] = w(out, unit * hid)
    p["merger.mlp.2.bias"] = bias(out)
    return {k: v.to(torch.bfloat16).float() for k, v in p.items()}
