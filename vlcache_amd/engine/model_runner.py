"""Per-GPU executor (engine/model_runner.py of the reference), one GPU.

Same method surface: call, copy_image_kv, prepare_prefill, prepare_decode,
prepare_sample, run_model, run, allocate_kv_cache, exit.  Differences:
  * copy_image_kv(old_slots, new_slots, deltas=None, seg_of_token=None) runs the
    all-layer reuse copy as one gfx950 kernel; with deltas it also re-rotates K
    to the image's new rotary position (without deltas it is the reference's
    plain copy, bit for bit);
  * prepare_prefill builds the step's attention work plan once (host lists are
    at hand) and passes it through the Context to every layer; prepare_decode
    passes a decode launch plan (cached per batch size and context bucket);
  * positions are M-RoPE [3, N] when the model config has mrope_section and
    use_mrope is set, else the reference's 1-D positions;
  * host preparation is vectorised (numpy) instead of per-token Python loops;
  * visual embeddings come from a bounded encoder cache (engine/encoder_cache.py)
    sized by encoder_cache_ratio; the images that miss it take the caller's
    image_embeds when given, else run through the vision tower in one batch (an
    image repeated in the batch runs once); a miss with neither pixel_values nor
    a vision tower uses seeded synthetic embeddings only when the config opts in
    (synthetic_vision), and raises otherwise;
  * every decode plan shares one workspace sized once for max_num_seqs requests
    of up to max_model_len tokens;
  * with enforce_eager off, decode steps replay HIP graphs captured per batch size
    on first use (the reference captures CUDA graphs at start-up);
  * no tensor parallelism, no shared-memory RPC: one process, one GPU.
"""
from __future__ import annotations

from time import perf_counter

import numpy as np
import torch

from .. import kernels
from ..config import Config
from .encoder_cache import EncoderCache
from ..qwen_vl import Qwen2_5_VLForConditionalGeneration, Sampler, random_init_
from ..utils.context import get_context, reset_context, set_context
from .sequence import Sequence


def _slots(block_table, positions: np.ndarray, block_size: int) -> np.ndarray:
    bt = np.asarray(block_table, dtype=np.int64)
    return bt[positions // block_size] * block_size + positions % block_size


def _h2d(arr, dtype, device):
    t = torch.from_numpy(np.ascontiguousarray(arr)).to(dtype)
    return t.pin_memory().to(device, non_blocking=True)


_TORCH_DTYPES = {np.dtype(np.int64): torch.int64, np.dtype(np.int32): torch.int32,
                 np.dtype(np.float32): torch.float32}


def _h2d_many(device, *arrays):
    """(array, numpy dtype) pairs -> device tensors of the same shapes, sent in ONE copy.

    The arrays are cast and packed at 16-byte aligned offsets into one pinned buffer
    (torch's pinned-memory cache hands it out again only once its copy has completed),
    the buffer goes to the device with one non-blocking copy, and each result is a view
    of the device copy.  A step's index arrays are a few KB to a few hundred KB each: a
    copy per array costs more host time than the bytes do.
    """
    items = [np.ascontiguousarray(a, dtype=dt) for a, dt in arrays]
    offsets, total = [], 0
    for a in items:
        offsets.append(total)
        total += -(-a.nbytes // 16) * 16
    host = torch.empty(max(total, 16), dtype=torch.uint8, pin_memory=torch.device(device).type == "cuda")
    buf = host.numpy()
    for a, o in zip(items, offsets):
        buf[o:o + a.nbytes] = a.reshape(-1).view(np.uint8)
    dev = host.to(device, non_blocking=True)
    return [dev[o:o + a.nbytes].view(_TORCH_DTYPES[a.dtype]).view(a.shape) for a, o in zip(items, offsets)]


class ModelRunner:

    def __init__(self, config: Config, rank: int = 0, event=None):
        assert rank == 0 and config.tensor_parallel_size == 1
        self.config = config
        hf = config.hf_config
        self.block_size = config.kvcache_block_size
        self.enforce_eager = config.enforce_eager
        self.world_size = 1
        self.rank = 0
        self.device = torch.device("cuda", 0)
        torch.cuda.set_device(self.device)
        self.dtype = hf.torch_dtype
        # Built under the default dtype, as the reference does (engine/model_runner.py:33-34):
        # parameters are bf16 while tensors created with an explicit dtype, such as the
        # fp32 rotary cos/sin cache, keep it.  A blanket .to(bf16) would round that cache.
        prev = torch.get_default_dtype()
        torch.set_default_dtype(self.dtype)
        try:
            with torch.device(self.device):
                self.model = Qwen2_5_VLForConditionalGeneration(hf)
        finally:
            torch.set_default_dtype(prev)
        assert all(m.cos_sin_cache.dtype == torch.float32 for m in self.model.modules()
                   if hasattr(m, "cos_sin_cache"))
        random_init_(self.model, seed=config.seed)
        self.model.eval()
        self.sampler = Sampler()
        self.num_layers = hf.num_hidden_layers
        self.num_kv_heads = hf.num_key_value_heads
        self.num_cus = torch.cuda.get_device_properties(self.device).multi_processor_count
        self.num_heads = hf.num_attention_heads
        self.head_dim = hf.head_dim
        self._logit_indices = None  # host list of the kept logit rows (partial steps)
        self._logit_rows = None     # the same rows on the device
        self._staged_temperatures = None  # the step's temperatures, sent with its other inputs
        self._decode_plans: dict = {}
        self._decode_workspace = None
        self._graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self._graph_vars = None
        self._graph_host = None
        self._graph_pool = None
        self.allocate_kv_cache()

    def call(self, method_name, *args):
        return getattr(self, method_name)(*args)

    def exit(self):
        torch.cuda.synchronize()

    # ------------------------------------------------------------------ memory
    def allocate_kv_cache(self):
        """KV cache and encoder cache.  Without an explicit block count the memory left
        under gpu_memory_utilization is split: encoder_cache_ratio of it to the encoder
        cache, the rest to KV blocks (engine/model_runner.py:126-149); with an explicit
        count the encoder cache gets the same ratio relative to the KV cache's share."""
        config = self.config
        hf = config.hf_config
        block_bytes = 2 * self.num_layers * self.block_size * self.num_kv_heads * self.head_dim * self.dtype.itemsize
        ratio = min(max(config.encoder_cache_ratio, 0.0), 0.95)
        if config.num_kvcache_blocks <= 0:
            free, total = torch.cuda.mem_get_info()
            budget = free - total * (1.0 - config.gpu_memory_utilization)
            encoder_bytes = budget * ratio
            config.num_kvcache_blocks = int(budget - encoder_bytes) // block_bytes
        else:
            encoder_bytes = config.num_kvcache_blocks * block_bytes * ratio / (1.0 - ratio)
        assert config.num_kvcache_blocks > 0
        page_bytes = self.block_size * hf.hidden_size * self.dtype.itemsize
        self.encoder_cache = EncoderCache(max(0, int(encoder_bytes) // page_bytes), self.block_size,
                                          hf.hidden_size, self.dtype, self.device)
        self.kv_cache = torch.empty(2, self.num_layers, config.num_kvcache_blocks, self.block_size,
                                    self.num_kv_heads, self.head_dim, dtype=self.dtype, device=self.device)
        layer_id = 0
        for module in self.model.modules():
            if hasattr(module, "k_cache") and hasattr(module, "v_cache"):
                module.k_cache = self.kv_cache[0, layer_id]
                module.v_cache = self.kv_cache[1, layer_id]
                layer_id += 1
        assert layer_id == self.num_layers

    # ------------------------------------------------------------------ reuse copy
    @torch.inference_mode()
    def copy_image_kv(self, old_slots, new_slots, deltas=None, seg_of_token=None):
        """Copy reused image KV of every layer from old to new slots; re-rotate K by `deltas`.

        deltas: None (plain copy) or [num_segments][3] (dt, dh, dw) rotary shifts;
        seg_of_token: segment of each token (None = all segment 0).
        """
        old = np.asarray(old_slots, dtype=np.int64)
        if old.size == 0:
            return
        rotate = deltas is not None and self.config.rerotate_reused_kv and bool(np.any(np.asarray(deltas)))
        arrays = [(old, np.int64), (new_slots, np.int64)]
        if rotate:
            hf = self.config.hf_config
            section = (hf.rope_scaling or {}).get("mrope_section") if self.config.use_mrope else None
            # (cos, sin) table on the host, sent with the slot lists in one copy
            arrays.append((kernels.rerotation_table(deltas, self.head_dim, hf.rope_theta, section).numpy(),
                           np.float32))
            if seg_of_token is not None:
                arrays.append((seg_of_token, np.int32))
        dev = _h2d_many(self.device, *arrays)
        cos_sin = dev[2] if rotate else None
        seg = dev[3] if rotate and seg_of_token is not None else None
        kernels.rerotate_copy_kv(self.kv_cache, dev[0], dev[1], cos_sin, seg, rotate_k=rotate)

    # ------------------------------------------------------------------ step preparation
    def _checked_ids(self, ids: np.ndarray) -> np.ndarray:
        """Token ids must index the embedding table: an id outside [0, vocab_size) is refused
        here rather than read out of bounds on the device."""
        vocab = self.config.hf_config.vocab_size
        if ids.size and (int(ids.min()) < 0 or int(ids.max()) >= vocab):
            bad = int(ids[(ids < 0) | (ids >= vocab)][0])
            raise ValueError(f"token id {bad} is outside the vocabulary [0, {vocab})")
        return ids

    def _positions(self, seq: Sequence, start: int, end: int) -> np.ndarray:
        return seq.positions(start, end, self.config.use_mrope)

    def prepare_prefill(self, seqs: list[Sequence]):
        input_ids, positions, slot_mapping = [], [], []
        cu_q, cu_k = [0], [0]
        max_q = max_k = 0
        vbts = []
        logit_indices = []
        vidx = 0
        has_partial = False
        mm = {"image_hashes": [], "image_grid_thw": [], "image_embeds": [], "pixel_values": [], "recompute": []}
        has_mm = False
        for seq in seqs:
            n = len(seq)
            if seq.mm_inputs:
                has_mm = True
                grids = seq.mm_inputs.get("image_grid_thw")
                embeds = seq.mm_inputs.get("image_embeds")
                pixels = seq.mm_inputs.get("pixel_values")
                p0 = 0
                for i in range(0 if grids is None else grids.shape[0]):
                    g = tuple(int(x) for x in grids[i])
                    mm["image_hashes"].append(seq.image_hashes[i])
                    mm["image_grid_thw"].append(g)
                    mm["image_embeds"].append(None if embeds is None else embeds[i])
                    # pixel_values holds every image's patches back to back (t*h*w rows each)
                    npatch = g[0] * g[1] * g[2]
                    mm["pixel_values"].append(None if pixels is None else pixels[p0:p0 + npatch])
                    p0 += npatch
                    r = seq.images[i].recompute if i < len(seq.images) else None
                    mm["recompute"].append(r if r is not None else 0)
            if seq.is_partial_recompute:
                has_partial = True
                # One image: (sub1: Q = K = [0, a+R)), (sub2: Q = [e, n), K = [0, n)); several
                # images: every maximal run of computed tokens, K = everything before its end.
                runs = seq.computed_runs()
                for qs, qe in runs:
                    input_ids.append(np.asarray(seq.token_ids[qs:qe], dtype=np.int64))
                    positions.append(self._positions(seq, qs, qe))
                    slot_mapping.append(_slots(seq.block_table, np.arange(qs, qe), self.block_size))
                    cu_q.append(cu_q[-1] + (qe - qs))
                    cu_k.append(cu_k[-1] + qe)
                    max_q, max_k = max(max_q, qe - qs), max(max_k, qe)
                    vbts.append(seq.block_table)
                logit_indices.append(vidx + len(runs) - 1)
                vidx += len(runs)
            else:
                input_ids.append(np.asarray(seq.token_ids, dtype=np.int64))
                positions.append(self._positions(seq, 0, n))
                cu_q.append(cu_q[-1] + n)
                cu_k.append(cu_k[-1] + n)
                max_q, max_k = max(max_q, n), max(max_k, n)
                if seq.block_table:
                    slot_mapping.append(_slots(seq.block_table, np.arange(n), self.block_size))
                    vbts.append(seq.block_table)
                logit_indices.append(vidx)
                vidx += 1
        plan_host, ws_bytes = kernels.plan_attention_host(cu_q, cu_k, self.num_heads, self.num_kv_heads,
                                                          self.head_dim, True, self.num_cus)
        ids = self._checked_ids(np.concatenate(input_ids))
        host = {"input_ids": (ids, np.int64), "positions": (np.concatenate(positions, axis=-1), np.int64),
                "cu_q": (cu_q, np.int32), "cu_k": (cu_k, np.int32),
                "slots": (np.concatenate(slot_mapping) if slot_mapping else np.zeros(0), np.int32),
                "plan": (plan_host, np.int32)}
        if has_mm:  # where the visual rows go, known here on the host
            host["image_rows"] = (np.flatnonzero(ids == self.config.hf_config.image_token_id), np.int64)
        if has_partial:  # the rows whose logits are kept
            host["logit_rows"] = (logit_indices, np.int64)
        host["temperatures"] = ([s.temperature for s in seqs], np.float32)
        if has_partial and vbts:
            width = max(len(bt) for bt in vbts)
            bt = np.full((len(vbts), width), -1, dtype=np.int32)
            for i, row in enumerate(vbts):
                bt[i, :len(row)] = row
            host["block_tables"] = (bt, np.int32)
        # every input of the step, the attention plan included, in one host-to-device copy
        dev = dict(zip(host, _h2d_many(self.device, *host.values())))
        if has_mm:
            mm["image_rows"] = dev["image_rows"]
        plan = kernels.attn_plan_on_device(plan_host, ws_bytes, dev["plan"], cu_q, cu_k, self.num_heads,
                                           self.num_kv_heads, True)
        set_context(True, dev["cu_q"], dev["cu_k"], max_q, max_k, dev["slots"], None, dev.get("block_tables"),
                    attn_plan=plan, cu_seqlens_q_host=cu_q, cu_seqlens_k_host=cu_k)
        self._logit_indices = logit_indices if has_partial else None
        self._logit_rows = dev.get("logit_rows")
        self._staged_temperatures = dev["temperatures"]
        input_ids, positions = dev["input_ids"], dev["positions"]
        return input_ids, positions, (mm if has_mm else None)

    def _decode_host_arrays(self, seqs: list[Sequence]):
        """Host inputs of a decode step (engine/model_runner.py:322-338): last token ids,
        positions (M-RoPE rows when used), the new token's slot, context lengths and the
        block tables padded with -1."""
        n = len(seqs)
        input_ids = self._checked_ids(np.array([s.last_token for s in seqs], dtype=np.int64))
        lens = np.array([len(s) for s in seqs], dtype=np.int64)
        pos = lens - 1
        if self.config.use_mrope:
            pos = np.tile(pos + np.array([s.rope_delta for s in seqs], dtype=np.int64), (3, 1))
        slot = np.array([s.block_table[-1] * self.block_size + s.last_block_num_tokens - 1 for s in seqs],
                        dtype=np.int64)
        width = max(len(s.block_table) for s in seqs)
        bt = np.full((n, width), -1, dtype=np.int32)
        for i, s in enumerate(seqs):
            bt[i, :len(s.block_table)] = s.block_table
        return input_ids, pos, slot, lens, bt

    def prepare_decode(self, seqs: list[Sequence]):
        n = len(seqs)
        input_ids, pos, slot, lens, bt = self._decode_host_arrays(seqs)
        cu_q = list(range(n + 1))
        cu_k = [0] + np.cumsum(lens).tolist()
        plan = dplan = None
        if kernels.decode_supported(self.num_heads, self.num_kv_heads, self.head_dim, self.block_size):
            dplan = self._decode_plan(n, int(lens.max()))
        else:
            plan = kernels.plan_attention(cu_q, cu_k, self.num_heads, self.num_kv_heads, self.head_dim, True,
                                          self.device)
        cu_q_t, cu_k_t, slot_t, lens_t, bt_t, ids_t, pos_t, self._staged_temperatures = _h2d_many(
            self.device, (cu_q, np.int32), (cu_k, np.int32), (slot, np.int32), (lens, np.int32), (bt, np.int32),
            (input_ids, np.int64), (pos, np.int64), ([s.temperature for s in seqs], np.float32))
        set_context(False, cu_q_t, cu_k_t, 1, int(lens.max()), slot_t, lens_t, bt_t, attn_plan=plan,
                    cu_seqlens_q_host=cu_q, cu_seqlens_k_host=cu_k, decode_plan=dplan)
        return ids_t, pos_t

    def _decode_plan(self, batch: int, max_len: int):
        """Decode launch plan for this batch size, sized for contexts up to the next multiple of
        1024 tokens.  Plans are host records; all of them share one workspace, allocated
        zeroed once for the largest any batch of at most max_num_seqs requests and
        max_model_len tokens needs (every call leaves its ticket counters at zero)."""
        cap = -(-max(max_len, 1) // 1024) * 1024
        key = (batch, cap)
        plan = self._decode_plans.get(key)
        if plan is None:
            plan = kernels.plan_decode(batch, self.num_heads, self.num_kv_heads, self.head_dim, self.block_size,
                                       cap, self.device, workspace=False)
            if self._decode_workspace is None:
                self._decode_workspace = torch.zeros(self._decode_workspace_bytes(), dtype=torch.uint8,
                                                     device=self.device)
            if plan.workspace_bytes > self._decode_workspace.numel():  # contexts beyond max_model_len
                self._decode_workspace = torch.zeros(plan.workspace_bytes, dtype=torch.uint8, device=self.device)
                self._decode_plans.clear()
                self._graphs.clear()  # captured graphs hold the old workspace's address
            plan.workspace = self._decode_workspace
            if len(self._decode_plans) > 4096:
                self._decode_plans.clear()
            self._decode_plans[key] = plan
        return plan

    def _decode_workspace_bytes(self) -> int:
        cap = -(-max(self.config.max_model_len, 1) // 1024) * 1024
        need = 16
        for b in range(1, max(1, self.config.max_num_seqs) + 1):
            p = kernels.plan_decode(b, self.num_heads, self.num_kv_heads, self.head_dim, self.block_size, cap,
                                    self.device, workspace=False)
            need = max(need, p.workspace_bytes)
        return need

    def prepare_sample(self, seqs: list[Sequence]):
        return _h2d(np.array([s.temperature for s in seqs], dtype=np.float32), torch.float32, self.device)

    # ------------------------------------------------------------------ vision inputs
    def _num_units(self, grid) -> int:
        m = self.config.hf_config.spatial_merge_size
        return int(grid[0]) * (int(grid[1]) // m) * (int(grid[2]) // m)

    def _process_visual(self, mm: dict):
        """Visual embeddings of every image of the batch, cache first (engine/model_runner.py:347-405).

        A hit reads the image's first R rows back (all rows when R is 0).  Misses
        take the caller's image_embeds when given; those with pixel_values run
        through the vision tower in one call (the time of that call is vit_time),
        an image repeated in the batch once; every new result is offered to the
        cache.  A miss with neither uses seeded synthetic embeddings when
        Config.synthetic_vision opts in and raises otherwise.
        """
        hashes, grids = mm["image_hashes"], mm["image_grid_thw"]
        if not hashes:
            return None, 0.0
        # Rows each image contributes, and their place in the output.  Every result is
        # copied into its slice as soon as it is known: a cache hit is a view of the
        # pool, and a later put() of this call may evict that entry and reuse its pages.
        sizes = []
        for grid, r in zip(grids, mm["recompute"]):
            n = self._num_units(grid)
            sizes.append(min(int(r), n) if r > 0 else n)
        offs = np.concatenate([[0], np.cumsum(sizes)]).tolist()
        out = torch.empty(offs[-1], self.config.hf_config.hidden_size, dtype=self.dtype, device=self.device)

        def place(i, emb):
            if emb.shape[0] < sizes[i]:
                raise ValueError(f"image {i}: {emb.shape[0]} embedding rows, {sizes[i]} needed")
            out[offs[i]:offs[i + 1]].copy_(emb[:sizes[i]])

        run: dict[int, list[int]] = {}          # hash -> indices waiting for the vision tower
        vit_time = 0.0
        for i, (h, grid, given, pix, r) in enumerate(zip(hashes, grids, mm["image_embeds"], mm["pixel_values"],
                                                         mm["recompute"])):
            rows = r if r > 0 else None
            hit = self.encoder_cache.get(h, rows)
            if hit is not None:
                place(i, hit)
                continue
            n = self._num_units(grid)
            if given is not None:
                emb = given.to(self.device, self.dtype)
            elif h in run:
                run[h].append(i)
                continue
            elif pix is not None and self.model.visual is not None:
                run[h] = [i]
                continue
            elif self.config.synthetic_vision:
                g = torch.Generator(device=self.device)
                g.manual_seed(h & ((1 << 63) - 1))
                emb = torch.randn(n, self.config.hf_config.hidden_size, generator=g, device=self.device,
                                  dtype=self.dtype)
            else:
                why = ("the request carries no pixel_values or image_embeds" if self.model.visual is not None
                       else "the model has no vision tower (pass mm_inputs['image_embeds'], or construct the "
                            "engine with synthetic_vision=True for synthetic embeddings)")
                raise RuntimeError(f"image {h:#x} is not in the encoder cache and {why}")
            if emb.shape[0] != n:
                raise ValueError(f"image_embeds has {emb.shape[0]} rows, the grid {tuple(grid)} gives {n}")
            place(i, emb)
            self.encoder_cache.put(h, emb)
        if run:
            first = [idx[0] for idx in run.values()]
            pv = torch.cat([mm["pixel_values"][i].to(self.device) for i in first], dim=0)
            torch.cuda.synchronize(self.device)
            t0 = perf_counter()
            emb_all = self.model.get_visual_features(pv, [grids[i] for i in first])
            torch.cuda.synchronize(self.device)
            vit_time = perf_counter() - t0
            for (h, idx), emb in zip(run.items(), torch.split(emb_all, [self._num_units(grids[i]) for i in first])):
                for i in idx:
                    place(i, emb)
                self.encoder_cache.put(h, emb)
        return out, vit_time

    # ------------------------------------------------------------------ decode graphs
    # With enforce_eager=False a decode step replays a HIP graph of the model's decode
    # forward, as the reference replays CUDA graphs (engine/model_runner.py:418-432,
    # 453-479): inputs go into static buffers sized for the largest batch, the graph of
    # the smallest captured batch size >= the step's batch replays, the logits are
    # computed from its output rows.  Graphs are captured on first use of a batch size
    # (1, 2, 4, 8, then multiples of 16 up to min(max_num_seqs, 512)), all in one memory
    # pool.  Every kernel of the forward takes its inputs from device memory: the token
    # ids, positions, slots, context lengths and block tables of the static buffers,
    # and one decode launch plan per batch size that covers max_model_len (its shared
    # workspace's counters return to zero after each call).  Padding rows carry slot -1
    # (not stored) and context length 0 (zero output).
    def _graph_buckets(self) -> list[int]:
        top = min(self.config.max_num_seqs, 512)
        return [b for b in (1, 2, 4, 8) if b <= top] + list(range(16, top + 1, 16))

    def _graph_decode_ok(self, n: int) -> bool:
        return (not self.enforce_eager and n <= self._graph_buckets()[-1] and
                kernels.decode_supported(self.num_heads, self.num_kv_heads, self.head_dim, self.block_size))

    def _graph_static(self):
        if self._graph_vars is None:
            mb = self._graph_buckets()[-1]
            width = -(-self.config.max_model_len // self.block_size)
            dev = self.device
            rows = 3 if self.config.use_mrope else 1
            self._graph_vars = dict(
                input_ids=torch.zeros(mb, dtype=torch.int64, device=dev),
                positions=torch.zeros(rows, mb, dtype=torch.int64, device=dev),
                slot_mapping=torch.full((mb,), -1, dtype=torch.int32, device=dev),
                context_lens=torch.zeros(mb, dtype=torch.int32, device=dev),
                block_tables=torch.full((mb, width), -1, dtype=torch.int32, device=dev),
                outputs=torch.zeros(mb, self.config.hf_config.hidden_size, dtype=self.dtype, device=dev))
            self._graph_host = {k: torch.empty(v.shape, dtype=v.dtype, pin_memory=True)
                                for k, v in self._graph_vars.items() if k != "outputs"}
            self._graph_pool = torch.cuda.graph_pool_handle()
        return self._graph_vars

    def _graph_context(self, bs: int):
        gv = self._graph_static()
        cap = -(-max(self.config.max_model_len, 1) // 1024) * 1024
        set_context(False, None, None, 1, cap, gv["slot_mapping"][:bs], gv["context_lens"][:bs],
                    gv["block_tables"][:bs], decode_plan=self._decode_plan(bs, cap))

    def _graph_positions(self, bs: int):
        pos = self._graph_static()["positions"][:, :bs]
        return pos if self.config.use_mrope else pos[0]

    def _capture_decode_graph(self, bs: int):
        gv = self._graph_static()
        # The warm-up run below executes: put its rows in the padding state first (no
        # slot stored, empty contexts).  After earlier replays the static buffers still
        # hold a previous step's slots and block tables, whose blocks may belong to
        # another request by now.
        gv["input_ids"][:bs].zero_()
        gv["positions"][:, :bs].zero_()
        gv["slot_mapping"][:bs].fill_(-1)
        gv["context_lens"][:bs].zero_()
        gv["block_tables"][:bs].fill_(-1)
        self._graph_context(bs)
        ids, pos = gv["input_ids"][:bs], self._graph_positions(bs)
        gv["outputs"][:bs] = self.model(ids, pos)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, self._graph_pool):
            gv["outputs"][:bs] = self.model(ids, pos)
        torch.cuda.synchronize(self.device)
        reset_context()
        self._graphs[bs] = g
        return g

    def _run_decode_graph(self, seqs: list[Sequence]) -> torch.Tensor:
        n = len(seqs)
        bs = next(b for b in self._graph_buckets() if b >= n)
        input_ids, pos, slot, lens, bt = self._decode_host_arrays(seqs)
        gv = self._graph_static()
        g = self._graphs.get(bs)
        if g is None:
            g = self._capture_decode_graph(bs)
        width = gv["block_tables"].shape[1]
        if bt.shape[1] > width:
            raise ValueError(f"a sequence needs {bt.shape[1]} blocks, more than max_model_len allows ({width})")
        # Fill the pinned host mirrors of the static buffers (padding rows included), then
        # copy each mirror's first bs rows up; the previous step's copies are done (its
        # sampled tokens were read back), so the mirrors are free to overwrite.
        hv = self._graph_host
        rows = gv["positions"].shape[0]
        hv["input_ids"][:bs] = 0
        hv["input_ids"][:n] = torch.from_numpy(input_ids)
        hv["positions"][:, :bs] = 0
        hv["positions"][:, :n] = torch.from_numpy(pos.reshape(rows, n))
        hv["slot_mapping"][:bs] = -1
        hv["slot_mapping"][:n] = torch.from_numpy(slot.astype(np.int32))
        hv["context_lens"][:bs] = 0
        hv["context_lens"][:n] = torch.from_numpy(lens.astype(np.int32))
        hv["block_tables"][:bs] = -1
        hv["block_tables"][:n, :bt.shape[1]] = torch.from_numpy(bt)
        for key in ("input_ids", "slot_mapping", "context_lens", "block_tables"):
            gv[key][:bs].copy_(hv[key][:bs], non_blocking=True)
        gv["positions"][:, :bs].copy_(hv["positions"][:, :bs], non_blocking=True)
        g.replay()
        set_context(False)
        return self.model.compute_logits(gv["outputs"][:n])

    # ------------------------------------------------------------------ execution
    @torch.inference_mode()
    def run_model(self, input_ids, positions, is_prefill, mm=None):
        visual, vit_time = self._process_visual(mm) if (is_prefill and mm) else (None, 0.0)
        rows = mm.get("image_rows") if (visual is not None and mm) else None
        hidden = self.model(input_ids, positions, visual, rows)
        return self.model.compute_logits(hidden), vit_time

    @torch.inference_mode()
    def run(self, seqs: list[Sequence], is_prefill: bool):
        if not is_prefill and self._graph_decode_ok(len(seqs)):
            temperatures = self.prepare_sample(seqs)
            logits = self._run_decode_graph(seqs)
            token_ids = self.sampler(logits, temperatures).tolist()
            reset_context()
            return token_ids, 0.0
        if is_prefill:
            input_ids, positions, mm = self.prepare_prefill(seqs)
        else:
            input_ids, positions = self.prepare_decode(seqs)
            mm = None
        # prepare_prefill/prepare_decode sent the temperatures with the step's other inputs
        temperatures, self._staged_temperatures = self._staged_temperatures, None
        logits, vit_time = self.run_model(input_ids, positions, is_prefill, mm)
        if is_prefill and self._logit_rows is not None:
            logits = logits.index_select(0, self._logit_rows)  # device indices: no sync
        token_ids = self.sampler(logits, temperatures).tolist()
        reset_context()
        return token_ids, vit_time
