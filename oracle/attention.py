"""fp32 oracle of varlen paged GQA causal attention (test-only).

Restates the call flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q,
max_seqlen_k, cu_seqlens_k, softmax_scale, causal=True, block_table) at
layers/attention.py:64-70, with flash-attn's documented semantics: causal masks
are aligned to the bottom-right corner (query i of a sequence with lengths
(sq, sk) sees keys j <= i + sk - sq), key j of sequence b is row
block_table[b, j // page] * page + j % page of the cache when a block table is
given (the cache is read back after store_kvcache, layers/attention.py:62-66),
q head h reads kv head h // (Hq / Hkv), and a row that sees no key is zero.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def gather_keys(cache: torch.Tensor, block_table_row, sk: int, page_size: int) -> torch.Tensor:
    """[sk, Hkv, hd] rows of a paged cache [num_blocks, page, Hkv, hd] for one sequence."""
    j = torch.arange(sk)
    bt = torch.as_tensor(block_table_row, dtype=torch.long)
    rows = bt[j // page_size] * page_size + j % page_size
    return cache.reshape(-1, cache.shape[-2], cache.shape[-1])[rows]


def varlen_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, softmax_scale: float, causal: bool = True,
                     block_table=None, page_size: int = 256, q_chunk: int = 2048) -> torch.Tensor:
    """fp32 [total_q, Hq, hd].  q, k, v may be bf16; the math is fp32 (SDPA, math backend)."""
    cu_q = [int(x) for x in cu_seqlens_q]
    cu_k = [int(x) for x in cu_seqlens_k]
    hq, hd = q.shape[1], q.shape[2]
    out = torch.zeros(q.shape[0], hq, hd, dtype=torch.float32)
    for b in range(len(cu_q) - 1):
        sq, sk = cu_q[b + 1] - cu_q[b], cu_k[b + 1] - cu_k[b]
        if sq == 0:
            continue
        if block_table is not None:
            kb = gather_keys(k, block_table[b], sk, page_size).float()
            vb = gather_keys(v, block_table[b], sk, page_size).float()
        else:
            kb = k[cu_k[b]:cu_k[b + 1]].float()
            vb = v[cu_k[b]:cu_k[b + 1]].float()
        group = hq // kb.shape[1]
        kb = kb.repeat_interleave(group, dim=1).transpose(0, 1)  # [Hq, sk, hd]
        vb = vb.repeat_interleave(group, dim=1).transpose(0, 1)
        qb = q[cu_q[b]:cu_q[b + 1]].float().transpose(0, 1)      # [Hq, sq, hd]
        for a in range(0, sq, q_chunk):
            e = min(sq, a + q_chunk)
            # Keys past the chunk's last causal limit are masked for every row of the
            # chunk; leaving them out of the product changes no result.
            hi = min(sk, max(0, e + sk - sq)) if causal else sk
            if hi == 0:
                continue
            i = torch.arange(a, e)[:, None]
            j = torch.arange(hi)[None, :]
            mask = (j <= i + sk - sq) if causal else torch.ones(e - a, hi, dtype=torch.bool)
            o = F.scaled_dot_product_attention(qb[:, a:e], kb[:, :hi], vb[:, :hi], attn_mask=mask,
                                               scale=softmax_scale)
            # flash-attn convention: a row with no visible key is 0 (SDPA gives NaN).
            o = torch.where(mask.any(dim=1)[None, :, None], o, torch.zeros_like(o))
            out[cu_q[b] + a:cu_q[b] + e] = o.transpose(0, 1)
    return out


def brute_force_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, softmax_scale: float, causal=True,
                          block_table=None, page_size: int = 256) -> np.ndarray:
    """float64 element loops for tiny shapes: an independent check of varlen_attention."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    hq, hd = q.shape[1], q.shape[2]
    hkv = k.shape[-2]
    group = hq // hkv
    out = np.zeros((q.shape[0], hq, hd))
    for b in range(len(cu_seqlens_q) - 1):
        q0, k0 = int(cu_seqlens_q[b]), int(cu_seqlens_k[b])
        sq, sk = int(cu_seqlens_q[b + 1]) - q0, int(cu_seqlens_k[b + 1]) - k0
        for i in range(sq):
            for h in range(hq):
                g = h // group
                scores, vals = [], []
                for j in range(sk):
                    if causal and j > i + sk - sq:
                        continue
                    if block_table is not None:
                        blk = int(block_table[b][j // page_size])
                        kr = k[blk, j % page_size, g]
                        vr = v[blk, j % page_size, g]
                    else:
                        kr = k[k0 + j, g]
                        vr = v[k0 + j, g]
                    scores.append(softmax_scale * float(np.dot(q[q0 + i, h], kr)))
                    vals.append(vr)
                if not scores:
                    continue
                s = np.array(scores)
                p = np.exp(s - s.max())
                out[q0 + i, h] = (p[:, None] * np.array(vals)).sum(0) / p.sum()
    return out

