"""Device state of the warm partial-recompute prefill hot path on synthetic inputs.

One warm request (or a batch of them) runs, per step:
  1. the all-layer reuse copy of the cached image KV with K re-rotated to the
     image's new position (one launch; ModelRunner.copy_image_kv,
     engine/model_runner.py:170-180);
  2. per layer, the rotary embedding of the recomputed tokens' q and k at their
     M-RoPE positions fused with the store of k and v into the paged cache
     (RotaryEmbedding.forward + store_kvcache, layers/rotary_embedding.py:37-48,
     layers/attention.py:62-63), then the varlen paged GQA causal attention of
     the recomputed queries against the whole cache (layers/attention.py:64-70).
Inputs are seeded N(0, 1) bf16: cached K/V, the recomputed tokens' q/k/v rows
as the QKV projection lays them out (q, k and v are views of one buffer).
Block ids are a seeded permutation of the pool; the cached image's blocks and
each request's blocks are disjoint, as the reference's allocator guarantees
(the cached entry's blocks stay referenced, engine/block_manager.py:91-94).
"""
from __future__ import annotations

import numpy as np
import torch

from . import kernels
from .engine.positions import mrope_positions
from .layers.rotary_embedding import get_rope
from .workloads import BLOCK_SIZE, IMAGE_TOKEN_ID, Workload

MAX_POSITIONS = 128000  # Qwen2.5-VL max_position_embeddings: rows of the rotary cache


def _slots(bt, positions):
    bt = np.asarray(bt, dtype=np.int64)
    p = np.asarray(positions, dtype=np.int64)
    return bt[p // BLOCK_SIZE] * BLOCK_SIZE + p % BLOCK_SIZE


class WarmPrefillHotPath:
    def __init__(self, wl: Workload, device, seed: int = 0, rotate: bool = True):
        self.wl = wl
        m = wl.model
        self.model = m
        self.device = torch.device(device)
        dev = self.device
        rng = np.random.default_rng(seed)
        reqs = wl.requests
        cached_prefix = reqs[0].cached_prefix
        # Block pool: one cached entry per distinct image (by its grid), stored standalone
        # after cached_prefix text tokens, plus each request's own blocks.
        grids = []
        for r in reqs:
            for _, _, hw in r.images():
                if hw not in grids:
                    grids.append(hw)
        entry_nbs = [-(-(cached_prefix + hw[0] * hw[1]) // BLOCK_SIZE) for hw in grids]
        seq_nbs = [-(-r.length // BLOCK_SIZE) for r in reqs]
        nb = sum(entry_nbs) + sum(seq_nbs)
        perm = rng.permutation(nb)
        entry_bts, p = {}, 0
        for hw, n in zip(grids, entry_nbs):
            entry_bts[hw] = perm[p:p + n]
            p += n
        seq_bts = []
        for n in seq_nbs:
            seq_bts.append(perm[p:p + n])
            p += n
        self.num_blocks = nb

        L, hkv, hd, hq = m.num_layers, m.num_kv_heads, m.head_dim, m.num_heads
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.kv_cache = torch.randn(2, L, nb, BLOCK_SIZE, hkv, hd, generator=g, device=dev,
                                    dtype=torch.bfloat16)
        self.k_caches = [self.kv_cache[0, l] for l in range(L)]
        self.v_caches = [self.kv_cache[1, l] for l in range(L)]

        # reuse copy: old -> new slots of every reused image token; one rotation segment
        # per (request, image), shifted by the image's new rotary start minus its cached one
        old, new, seg, deltas = [], [], [], []
        slot_map, bts, cu_q, cu_k, pos_cols = [], [], [0], [0], []
        for r, bt in zip(reqs, seq_bts):
            if r.ratio > 0:
                for (s_, e_, hw), rc, d in zip(r.images(), r.recompute(), r.deltas()):
                    reuse = np.arange(s_ + rc, e_)
                    old.append(_slots(entry_bts[hw], cached_prefix + (reuse - s_)))
                    new.append(_slots(bt, reuse))
                    seg.append(np.full(reuse.size, len(deltas), dtype=np.int32))
                    deltas.append([d] * 3)
            comp = np.concatenate([np.arange(a, b) for a, b in r.runs()])
            slot_map.append(_slots(bt, comp))
            toks = np.ones(r.length, dtype=np.int64)
            grids_thw = []
            for s_, e_, hw in r.images():
                toks[s_:e_] = IMAGE_TOKEN_ID
                grids_thw.append((1, 2 * hw[0], 2 * hw[1]))
            pos_all, _, _ = mrope_positions(toks, grids_thw, IMAGE_TOKEN_ID)
            pos_cols.append(pos_all[:, comp])
            row = np.full(max(seq_nbs), -1, dtype=np.int32)
            row[:len(bt)] = bt
            for sq, sk in r.subseqs():
                cu_q.append(cu_q[-1] + sq)
                cu_k.append(cu_k[-1] + sk)
                bts.append(row)
        if not deltas:
            deltas = [[0, 0, 0]]
        cat = lambda xs, dt: np.concatenate(xs).astype(dt) if xs else np.zeros(0, dtype=dt)
        self.old_slots = torch.from_numpy(cat(old, np.int64)).to(dev)
        self.new_slots = torch.from_numpy(cat(new, np.int64)).to(dev)
        self.seg = torch.from_numpy(cat(seg, np.int32)).to(dev)
        self.deltas = deltas
        self.cos_sin = kernels.rerotation_table(deltas, hd, m.rope_theta, m.mrope_section, device=dev)
        self.rotate = rotate
        self.n_reused = int(self.old_slots.numel())

        n_q = cu_q[-1]
        self.n_computed = n_q
        self.cu_q_host, self.cu_k_host = cu_q, cu_k
        self.cu_q = torch.tensor(cu_q, dtype=torch.int32, device=dev)
        self.cu_k = torch.tensor(cu_k, dtype=torch.int32, device=dev)
        self.slot_mapping = torch.from_numpy(np.concatenate(slot_map).astype(np.int32)).to(dev)
        self.block_tables = torch.from_numpy(np.stack(bts)).to(dev)
        # recomputed tokens: qkv rows as the QKV projection lays them out (q, k and
        # v are strided views); rope_store writes the rotated q to a contiguous
        # tensor, as RotaryEmbedding returns one, and leaves the inputs unchanged.
        qkv = torch.randn(n_q, (hq + 2 * hkv) * hd, generator=g, device=dev, dtype=torch.bfloat16)
        self.qkv = qkv
        self.q_in = qkv[:, :hq * hd].view(n_q, hq, hd)
        self.k_in = qkv[:, hq * hd:(hq + hkv) * hd].view(n_q, hkv, hd)
        self.v = qkv[:, (hq + hkv) * hd:].view(n_q, hkv, hd)
        self.q = torch.empty(n_q, hq, hd, device=dev, dtype=torch.bfloat16)   # rotated q
        self.k = torch.empty(n_q, hkv, hd, device=dev, dtype=torch.bfloat16)  # rotated k (contiguous)
        self.positions = torch.from_numpy(np.ascontiguousarray(np.concatenate(pos_cols, axis=1))).to(dev)
        self.rope = get_rope(hd, hd, MAX_POSITIONS, m.rope_theta, {"mrope_section": list(m.mrope_section)}).to(dev)
        self.rope_k_out = not any(r.ratio > 0 for r in reqs)  # contiguous attention reads the fresh keys
        # rotated q and k (no store) so that attention and scatter have valid inputs before a step
        kernels.rope_store_kvcache(self.positions, self.q_in, self.k_in, self.v, self.rope.cos_sin_cache,
                                   m.mrope_section, q_out=self.q, k_out=self.k)
        self.scale = hd ** -0.5
        # Block tables exist only when a request is partial; otherwise attention
        # reads the fresh contiguous k/v (engine/model_runner.py:294-299,
        # layers/attention.py:65-66).
        self.paged = any(r.ratio > 0 for r in reqs)
        self.plan = kernels.plan_attention(cu_q, cu_k, hq, hkv, hd, True, dev)
        self.out = torch.empty(n_q, hq, hd, dtype=torch.bfloat16, device=dev)

    # ---- the kernels ----
    def rerotate(self):
        kernels.rerotate_copy_kv(self.kv_cache, self.old_slots, self.new_slots, self.cos_sin, self.seg,
                                 rotate_k=self.rotate)

    def rope_store(self, layer: int):
        """Rotate q and k at the M-RoPE positions; store rotated k and v in layer's cache."""
        kernels.rope_store_kvcache(self.positions, self.q_in, self.k_in, self.v, self.rope.cos_sin_cache,
                                   self.model.mrope_section, self.k_caches[layer], self.v_caches[layer],
                                   self.slot_mapping, q_out=self.q,
                                   k_out=self.k if self.rope_k_out else None)

    def torch_rope(self):
        """The unfused reference sequence's rotation: torch eager RoPE of q and k."""
        return self.rope(self.positions, self.q_in, self.k_in)

    def scatter(self, layer: int):
        """store_kvcache of the rotated k and of v (the reference's separate scatter)."""
        kernels.store_kvcache_raw(self.k, self.v, self.k_caches[layer], self.v_caches[layer],
                                  self.slot_mapping)

    def attention(self, layer: int):
        if not self.paged:
            return kernels.varlen_attention(self.q, self.k, self.v, self.cu_q, self.cu_k, self.scale, True,
                                            None, plan=self.plan, out=self.out)
        return kernels.varlen_attention(self.q, self.k_caches[layer], self.v_caches[layer], self.cu_q,
                                        self.cu_k, self.scale, True, self.block_tables, plan=self.plan,
                                        out=self.out)

    def step(self):
        if self.n_reused:
            self.rerotate()
        for layer in range(self.model.num_layers):
            self.rope_store(layer)
            self.attention(layer)
        return self.out
