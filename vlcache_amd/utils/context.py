"""Per-step attention metadata shared by every attention layer.

Mirrors utils/context.py of the reference (Context, get_context, set_context,
reset_context; :5-27) with the same positional fields.  Keyword-only additions
carry what the gfx950 attention needs from the host without a device-to-host
copy: the prefill work plan built once per step, the host copies of the
sequence boundaries it was built from, and the decode launch plan.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class Context:
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    attn_plan: object | None = None      # vlcache_amd.kernels.AttnPlan shared by all layers
    cu_seqlens_q_host: list | None = None
    cu_seqlens_k_host: list | None = None
    decode_plan: object | None = None    # vlcache_amd.kernels.DecodePlan shared by all layers


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0,
                slot_mapping=None, context_lens=None, block_tables=None, *, attn_plan=None,
                cu_seqlens_q_host=None, cu_seqlens_k_host=None, decode_plan=None):
    global _CONTEXT
    _CONTEXT = Context(is_prefill, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, slot_mapping,
                       context_lens, block_tables, attn_plan, cu_seqlens_q_host, cu_seqlens_k_host, decode_plan)


def reset_context():
    global _CONTEXT
    _CONTEXT = Context()
