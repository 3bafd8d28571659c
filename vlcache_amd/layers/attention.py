"""Drop-in attention layer and KV scatter for the warm partial-recompute prefill.

Same public surface as layers/attention.py of the reference:
  * store_kvcache(key, value, k_cache, v_cache, slot_mapping) -- same arguments
    and preconditions (:33-40); the copy runs in the gfx950 scatter kernel.
  * Attention(num_heads, head_dim, scale, num_kv_heads) with k_cache/v_cache
    attributes bound by the model runner and forward(q, k, v) reading the global
    Context (:43-75): prefill attends through the block table when the step has
    one (the cache is read back after the scatter, :65-66) and over the fresh
    contiguous k/v otherwise; decode attends through the block table with one
    query per sequence and returns [B, 1, Hq, hd] (:71-74).
Prefill runs in the gfx950 varlen GQA kernel, decode in the paged decode kernel.  forward_rope(positions,
q, k, v, rotary_emb) is the fused form of the caller's sequence RoPE -> forward
(models/qwen3.py:84-85): one kernel rotates q and k and stores k and v.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import kernels
from ..utils.context import Context, get_context


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    kernels.store_kvcache_raw(key, value, k_cache, v_cache, slot_mapping)


def _plan(context: Context, num_heads: int, num_kv_heads: int, head_dim: int, device):
    """The step's attention plan; built here (one device-to-host copy) if the caller gave none."""
    plan = context.attn_plan
    if plan is None or plan.num_heads_q != num_heads or plan.num_heads_kv != num_kv_heads:
        cu_q = context.cu_seqlens_q_host or context.cu_seqlens_q.tolist()
        cu_k = context.cu_seqlens_k_host or context.cu_seqlens_k.tolist()
        plan = kernels.plan_attention(cu_q, cu_k, num_heads, num_kv_heads, head_dim, True, device)
        context.attn_plan = plan
    return plan


class Attention(nn.Module):

    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        context = get_context()
        k_cache, v_cache = self.k_cache, self.v_cache
        if k_cache.numel() and v_cache.numel():
            store_kvcache(k, v, k_cache, v_cache, context.slot_mapping)
        return self._attend(q, k, v, context)

    def forward_rope(self, positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     rotary_emb, q_inplace: bool = False) -> torch.Tensor:
        """rotary_emb(positions, q, k) then forward(q, k, v) (models/qwen3.py:84-85), bit for bit,
        with the rotation and the KV store in one kernel (kernels.rope_store_kvcache).

        rotary_emb is the layer's RotaryEmbedding / MRotaryEmbedding: its fp32
        cos/sin cache and, for [3, N] positions, its mrope_section.  q_inplace
        rotates q inside the caller's buffer (e.g. the QKV projection output)
        instead of a new tensor.
        """
        context = get_context()
        k_cache, v_cache = self.k_cache, self.v_cache
        store = bool(k_cache.numel() and v_cache.numel())
        # Without a block table the prefill attends over the fresh keys, so it needs them rotated.
        need_k = context.is_prefill and (context.block_tables is None or not store)
        section = getattr(rotary_emb, "mrope_section", None) if positions.dim() == 2 else None
        q, k_rot = kernels.rope_store_kvcache(
            positions, q, k, v, rotary_emb.cos_sin_cache, section,
            k_cache if store else None, v_cache if store else None,
            context.slot_mapping if store else None, q_out=q if q_inplace else None, return_k=need_k)
        return self._attend(q, k_rot, v, context)

    def _attend(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, context: Context) -> torch.Tensor:
        k_cache, v_cache = self.k_cache, self.v_cache
        if context.is_prefill:
            if context.block_tables is not None:
                k, v = k_cache, v_cache
            plan = _plan(context, self.num_heads, self.num_kv_heads, self.head_dim, q.device)
            return kernels.varlen_attention(q, k, v, context.cu_seqlens_q, context.cu_seqlens_k, self.scale,
                                            True, context.block_tables, plan=plan)
        # decode: one query per sequence against its cached context (layers/attention.py:71-74)
        if kernels.decode_supported(self.num_heads, self.num_kv_heads, self.head_dim, k_cache.shape[1]):
            plan = context.decode_plan
            if plan is None or plan.batch != q.shape[0] or plan.num_heads_q != self.num_heads or \
                    (context.max_seqlen_k or 0) > plan.max_seqlen_k:
                max_k = context.max_seqlen_k or None
                if context.cu_seqlens_k_host is not None:
                    cu = context.cu_seqlens_k_host
                    max_k = max((cu[i + 1] - cu[i] for i in range(len(cu) - 1)), default=0)
                plan = kernels.plan_decode(q.shape[0], self.num_heads, self.num_kv_heads, self.head_dim,
                                           k_cache.shape[1], max_k if max_k is not None else
                                           int(context.context_lens.max().item()), q.device)
                context.decode_plan = plan
            o = kernels.decode_attention(q, k_cache, v_cache, context.context_lens, context.block_tables,
                                         self.scale, plan=plan, max_seqlen_k=context.max_seqlen_k or None)
        else:  # shapes the decode kernel does not take: the varlen kernel with one query per sequence
            plan = _plan(context, self.num_heads, self.num_kv_heads, self.head_dim, q.device)
            o = kernels.varlen_attention(q, k_cache, v_cache, context.cu_seqlens_q, context.cu_seqlens_k,
                                         self.scale, True, context.block_tables, plan=plan)
        return o.unsqueeze(1)
