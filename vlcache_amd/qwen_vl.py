"""Qwen2.5-VL text decoder: the caller of the attention layer on the hot path.

Mirrors the forward of models/qwen3.py (Qwen3Attention :71-87, decoder layer
:145-158, model :172-186; with attention_bias absent the reference builds the
Qwen2.5-VL variant: QKV bias, no q/k norm) and of
Qwen2_5_VLForConditionalGeneration.forward (models/qwen2_5_vl.py:562-580: the
image-token rows of the embeddings are replaced by visual embeddings).

GEMMs run on torch (hipBLASLt) except calls of at most 16 rows (decode steps),
which stream the weights through vlc_linear_skinny (layers.linear.Linear); per layer the rotary
embedding of q and k and the KV store run as one gfx950 kernel and the
attention as another (layers.attention.Attention), each RMSNorm (with its
residual add) as one kernel and the MLP's SiLU-and-multiply as one.
When the model config carries a vision_config the model owns the vision tower
(vision.VisionTransformer, the cold path behind the encoder cache).
Weights are random N(0, 0.02) unless loaded by the caller.
"""
from __future__ import annotations

import re

import torch
from torch import nn

from . import kernels
from .layers.attention import Attention
from .layers.layernorm import RMSNorm
from .layers.linear import Linear
from .layers.rotary_embedding import get_rope
from .utils.context import get_context
from .vision import VisionTransformer, vision_config

IMAGE_TOKEN_ID = 151655


class DecoderAttention(nn.Module):
    # True: RoPE and the KV store run as one kernel (Attention.forward_rope);
    # False: the reference's sequence, torch RoPE then Attention.forward.
    fused_rope = True

    def __init__(self, cfg):
        super().__init__()
        self.num_heads = cfg.num_attention_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim
        self.qkv_proj = Linear(cfg.hidden_size, self.q_size + 2 * self.kv_size, bias=True)
        self.o_proj = Linear(self.q_size, cfg.hidden_size, bias=False)
        self.rotary_emb = get_rope(self.head_dim, self.head_dim, cfg.max_position_embeddings,
                                   getattr(cfg, "rope_theta", 1e6), getattr(cfg, "rope_scaling", None))
        self.attn = Attention(self.num_heads, self.head_dim, self.head_dim ** -0.5, self.num_kv_heads)

    def forward(self, positions, hidden_states):
        qkv = self.qkv_proj(hidden_states)
        q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
        q = q.view(-1, self.num_heads, self.head_dim)
        k = k.view(-1, self.num_kv_heads, self.head_dim)
        v = v.view(-1, self.num_kv_heads, self.head_dim)  # strided view into qkv rows
        if self.fused_rope:
            # one kernel: rotate q (in the qkv buffer) and k, store rotated k and v in the cache
            o = self.attn.forward_rope(positions, q, k, v, self.rotary_emb, q_inplace=True)
        else:
            q, k = self.rotary_emb(positions, q, k)
            o = self.attn(q, k, v)
        return self.o_proj(o.flatten(1, -1))


class MLP(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.inter = cfg.intermediate_size
        self.gate_up_proj = Linear(cfg.hidden_size, 2 * cfg.intermediate_size, bias=False)
        self.down_proj = Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)

    def forward(self, x):
        return self.down_proj(kernels.silu_mul(self.gate_up_proj(x)))


class DecoderLayer(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.self_attn = DecoderAttention(cfg)
        self.mlp = MLP(cfg)
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)

    def forward(self, positions, hidden_states, residual):
        if residual is None:
            hidden_states, residual = self.input_layernorm(hidden_states), hidden_states
        else:
            hidden_states, residual = self.input_layernorm(hidden_states, residual)
        hidden_states = self.self_attn(positions, hidden_states)
        hidden_states, residual = self.post_attention_layernorm(hidden_states, residual)
        return self.mlp(hidden_states), residual


class TextModel(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList([DecoderLayer(cfg) for _ in range(cfg.num_hidden_layers)])
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)

    def forward(self, input_ids, positions, inputs_embeds=None):
        hidden_states = self.embed_tokens(input_ids) if inputs_embeds is None else inputs_embeds
        residual = None
        for layer in self.layers:
            hidden_states, residual = layer(positions, hidden_states, residual)
        hidden_states, _ = self.norm(hidden_states, residual)
        return hidden_states


class Qwen2_5_VLForConditionalGeneration(nn.Module):
    """Text side of Qwen2.5-VL with visual-embedding injection; logits of the last row per sub-sequence."""

    def __init__(self, cfg):
        super().__init__()
        self.config = cfg
        vcfg = getattr(cfg, "vision_config", None)
        self.visual = (VisionTransformer(vision_config(vcfg, cfg.hidden_size), eps=cfg.rms_norm_eps)
                       if vcfg is not None else None)
        self.model = TextModel(cfg)
        self.lm_head = Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        if getattr(cfg, "tie_word_embeddings", False):
            self.lm_head.weight = self.model.embed_tokens.weight

    def get_visual_features(self, pixel_values, grid_thw):
        if self.visual is None:
            raise RuntimeError("the model config has no vision_config: there is no vision tower")
        return self.visual(pixel_values, grid_thw)

    def forward(self, input_ids, positions, visual_embeds=None, image_rows=None):
        """image_rows: int64 device indices of the image tokens in input_ids, when the caller
        knows them (the engine does, from its host copy of the ids): the visual rows are then
        placed without the device-to-host synchronisation that a boolean mask costs."""
        inputs_embeds = self.model.embed_tokens(input_ids)
        if visual_embeds is not None:
            if image_rows is not None:
                if image_rows.numel() != visual_embeds.shape[0]:
                    raise ValueError(f"{image_rows.numel()} image tokens, {visual_embeds.shape[0]} visual rows")
                inputs_embeds.index_copy_(0, image_rows, visual_embeds.to(inputs_embeds.dtype))
            else:
                mask = input_ids == getattr(self.config, "image_token_id", IMAGE_TOKEN_ID)
                # The reference asserts the count here (a device-to-host sync); a
                # mismatch raises inside the masked assignment instead.
                inputs_embeds[mask] = visual_embeds.to(inputs_embeds.dtype)
        return self.model(input_ids, positions, inputs_embeds=inputs_embeds)

    def compute_logits(self, hidden_states):
        ctx = get_context()
        if ctx.is_prefill:  # last row of every (virtual) sequence (layers/embed_head.py:56-60)
            hidden_states = hidden_states[ctx.cu_seqlens_q[1:] - 1].contiguous()
        return self.lm_head(hidden_states)


@torch.no_grad()
def random_init_(model: nn.Module, std: float = 0.02, seed: int = 0) -> None:
    """N(0, std) weights, zero biases, unit norm weights (synthetic checkpoint)."""
    g = torch.Generator(device=next(model.parameters()).device)
    g.manual_seed(seed)
    for name, p in model.named_parameters():
        if re.search(r"(norm\d?|ln_q)\.weight$", name):
            p.fill_(1.0)
        elif name.endswith(".bias"):
            p.zero_()
        else:
            p.normal_(0.0, std, generator=g)


class Sampler(nn.Module):
    """Gumbel-max sampling at temperature (layers/sampler.py:10-15)."""

    def forward(self, logits, temperatures):
        logits = logits.float().div_(temperatures.unsqueeze(dim=1))
        probs = torch.softmax(logits, dim=-1)
        return probs.div_(torch.empty_like(probs).exponential_(1).clamp_min_(1e-10)).argmax(dim=-1)
