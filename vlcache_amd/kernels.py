"""torch-facing wrappers of the gfx950 kernels (C ABI in include/vlc_capi.h).

torch supplies device memory and the current stream; every computation runs in
the HIP library.  Tensors must live on a HIP device: there is no CPU path.
"""
from __future__ import annotations

import ctypes
import functools
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

HEAD_DIM = 128  # the attention kernel's head dimension
_PLAN_HEAD_DIM = 10  # header word of a vlc_attn_plan plan holding its head_dim
ATTN_HEAD_DIMS = (128, 80)  # head_dims of vlc_varlen_attn_fwd (80: contiguous k/v only)


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _require_device(name: str, *tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{name}: tensors must be on a HIP device (got {t.device}); "
                               "the gfx950 kernels have no CPU path")


def _num_cus(device: torch.device) -> int:
    return torch.cuda.get_device_properties(device).multi_processor_count


# --------------------------------------------------------------------------- scatter
def store_kvcache_raw(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                      v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Scatter K/V rows of fresh tokens into the paged cache (vlc_store_kvcache).

    key/value: [N, Hkv, hd] with contiguous rows (value may have any row stride);
    caches: [num_blocks, block_size, Hkv, hd] contiguous rows; slot_mapping: int32 [N].
    """
    _require_device("store_kvcache", key, value, k_cache, v_cache, slot_mapping)
    if slot_mapping.dtype != torch.int32:
        raise TypeError("slot_mapping must be int32")
    n = key.shape[0]
    d = key.shape[1] * key.shape[2]
    if value.shape != key.shape or slot_mapping.numel() != n:
        raise ValueError("key, value and slot_mapping must agree in the number of tokens")
    if key.dtype != value.dtype or k_cache.dtype != key.dtype or v_cache.dtype != key.dtype:
        raise TypeError("key, value and the caches must share one dtype")
    for name, t in (("key", key), ("value", value)):
        if t.stride(-1) != 1 or t.stride(1) != key.shape[2]:
            raise ValueError(f"{name}: each token row must be {d} contiguous elements")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache must be contiguous")
    num_slots = k_cache.numel() // d
    if v_cache.numel() // d != num_slots:
        raise ValueError("k_cache and v_cache differ in size")
    st = _lib.load().vlc_store_kvcache(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(), num_slots, slot_mapping.data_ptr(), n, d,
        key.element_size(), _stream(key))
    _lib.check("vlc_store_kvcache", st)


# --------------------------------------------------------------------------- fused RoPE + scatter
def _check_heads(name: str, t: torch.Tensor, n: int, heads: int, hd: int) -> None:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bf16")
    if t.dim() != 3 or tuple(t.shape) != (n, heads, hd):
        raise ValueError(f"{name}: expected [{n}, {heads}, {hd}], got {tuple(t.shape)}")
    if t.stride(-1) != 1 or t.stride(1) != hd:
        raise ValueError(f"{name}: heads must be contiguous rows of {hd} elements")


def rope_store_kvcache(positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor | None,
                       cos_sin_cache: torch.Tensor, mrope_section=None,
                       k_cache: torch.Tensor | None = None, v_cache: torch.Tensor | None = None,
                       slot_mapping: torch.Tensor | None = None, q_out: torch.Tensor | None = None,
                       k_out: torch.Tensor | None = None, return_k: bool = False):
    """Rotate q and k and store the rotated k and v into the paged cache (vlc_rope_store_kvcache).

    One launch for RotaryEmbedding.forward (layers/rotary_embedding.py:37-48) plus
    store_kvcache (layers/attention.py:33-40).  positions: int64 [N] (1-D) or
    [3, N] (M-RoPE, with mrope_section); q [N, Hq, hd], k/v [N, Hkv, hd] bf16
    with contiguous head rows (any token row stride, e.g. views of the QKV
    output); cos_sin_cache: the rotary module's fp32 [max_pos, (1,) hd] cache.
    Caches and slot_mapping may be None (rotation only).  Returns (q_rot, k_rot):
    q_rot is q_out (a new contiguous tensor when None; pass q_out=q to rotate in
    place); k_rot is k_out, a new tensor when return_k, else None.
    """
    _require_device("rope_store_kvcache", positions, q, k, v, cos_sin_cache, k_cache, v_cache, slot_mapping,
                    q_out, k_out)
    n, hq, hd = q.shape
    hkv = k.shape[1]
    _check_heads("q", q, n, hq, hd)
    _check_heads("k", k, n, hkv, hd)
    if positions.dtype != torch.int64 or positions.stride(-1) != 1:
        raise TypeError("positions must be int64 with contiguous rows")
    if positions.dim() == 1:
        rows, pos_rs, sec = 1, 0, None
        if positions.numel() != n:
            raise ValueError("positions must hold one entry per token")
    elif positions.dim() == 2 and positions.shape[0] == 3:
        if mrope_section is None:
            raise ValueError("[3, N] positions need mrope_section")
        if positions.shape[1] != n:
            raise ValueError("positions must hold one column per token")
        rows, pos_rs = 3, positions.stride(0)
        sec = (ctypes.c_int32 * 3)(*[int(x) for x in mrope_section])
    else:
        raise ValueError("positions must be [N] or [3, N]")
    cs = cos_sin_cache
    if cs.dtype != torch.float32 or cs.shape[-1] != hd or cs.stride(-1) != 1:
        raise ValueError(f"cos_sin_cache must be fp32 [max_pos, (1,) {hd}] with contiguous rows")
    if cs.dim() == 3 and cs.shape[1] != 1 or cs.dim() not in (2, 3):
        raise ValueError("cos_sin_cache must be [max_pos, hd] or [max_pos, 1, hd]")
    store = k_cache is not None or v_cache is not None
    num_slots = 0
    if store:
        if k_cache is None or v_cache is None or slot_mapping is None or v is None:
            raise ValueError("storing needs k_cache, v_cache, slot_mapping and v")
        _check_heads("v", v, n, hkv, hd)
        if slot_mapping.dtype != torch.int32 or slot_mapping.numel() != n:
            raise ValueError("slot_mapping must be int32 [N]")
        if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise ValueError("k_cache/v_cache must be contiguous")
        if k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
            raise TypeError("caches must be bf16")
        num_slots = k_cache.numel() // (hkv * hd)
        if v_cache.numel() // (hkv * hd) != num_slots or k_cache.shape[-1] != hd or k_cache.shape[-2] != hkv:
            raise ValueError("caches must be [..., Hkv, hd] of equal size")
    if q_out is None:
        q_out = torch.empty(n, hq, hd, dtype=torch.bfloat16, device=q.device)
    else:
        _check_heads("q_out", q_out, n, hq, hd)
    if k_out is None and return_k:
        k_out = torch.empty(n, hkv, hd, dtype=torch.bfloat16, device=q.device)
    elif k_out is not None:
        _check_heads("k_out", k_out, n, hkv, hd)
    st = _lib.load().vlc_rope_store_kvcache(
        q.data_ptr(), q.stride(0), q_out.data_ptr(), q_out.stride(0),
        k.data_ptr(), k.stride(0), k_out.data_ptr() if k_out is not None else None,
        k_out.stride(0) if k_out is not None else 0,
        v.data_ptr() if v is not None else None, v.stride(0) if v is not None else 0,
        hq, hkv, hd, positions.data_ptr(), rows, pos_rs, sec,
        cs.data_ptr(), cs.stride(0), cs.shape[0],
        k_cache.data_ptr() if store else None, v_cache.data_ptr() if store else None, num_slots,
        slot_mapping.data_ptr() if store else None, n, _stream(q))
    _lib.check("vlc_rope_store_kvcache", st)
    return q_out, k_out


# --------------------------------------------------------------------------- rerotate
@functools.lru_cache(maxsize=16)
def _rotation_pairs(head_dim: int, theta: float, mrope_section: tuple | None):
    """Section index (long [hd/2]) and fp32 inv_freq of each rotation pair; constants of a
    model, computed once (read-only: callers index them, never write)."""
    half = head_dim // 2
    sec = torch.zeros(half, dtype=torch.long)
    if mrope_section is not None:
        if sum(mrope_section) != half:
            raise ValueError("mrope_section must sum to head_dim / 2")
        sec = torch.repeat_interleave(torch.arange(3), torch.as_tensor(list(mrope_section)))
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    return sec, inv


def rerotation_table(deltas, head_dim: int, theta: float, mrope_section=None,
                     device=None) -> torch.Tensor:
    """fp32 [num_segments, head_dim/2, 2] (cos, sin) of the per-pair rotation angle.

    deltas: [num_segments, 3] (dt, dh, dw) position shifts, or [num_segments] for
    a 1-D shift.  Pair i (dims i, i + hd/2) turns by delta_section(i) *
    inv_freq[i], inv_freq[i] = theta^(-2i/hd) in fp32 as the reference's rotary
    cache computes it (layers/rotary_embedding.py:29-33); section(i) follows
    mrope_section (e.g. [16, 24, 24]: t for i < 16, h for i < 40, w after),
    or the t delta for every pair when mrope_section is None.
    """
    d = np.asarray(deltas, dtype=np.float64)
    if d.ndim == 1:
        d = np.repeat(d[:, None], 3, axis=1)
    sec, inv = _rotation_pairs(head_dim, float(theta),
                               None if mrope_section is None else tuple(int(x) for x in mrope_section))
    # the fp32 angles in numpy (the same IEEE roundings as torch's), cos/sin in torch
    ang = torch.from_numpy(d[:, sec.numpy()].astype(np.float32) * inv.numpy()[None, :])
    tab = torch.stack((ang.cos(), ang.sin()), dim=-1).contiguous()
    return tab if device is None else tab.to(device)


def rerotate_copy_kv(kv_cache: torch.Tensor, old_slots: torch.Tensor, new_slots: torch.Tensor,
                     cos_sin: torch.Tensor | None = None, seg_of_token: torch.Tensor | None = None,
                     rotate_k: bool = True) -> None:
    """All-layer image-KV reuse copy with K re-rotation (vlc_rerotate_copy_kv).

    kv_cache: bf16 [2, L, num_blocks, block_size, Hkv, hd] (contiguous);
    old_slots/new_slots: int64 [n] on the device; cos_sin: fp32 [nseg, hd/2, 2];
    seg_of_token: int32 [n] or None (segment 0).  rotate_k=False is the
    reference's plain copy.
    """
    _require_device("rerotate_copy_kv", kv_cache, old_slots, new_slots, cos_sin, seg_of_token)
    if kv_cache.dtype != torch.bfloat16 or not kv_cache.is_contiguous() or kv_cache.dim() != 6:
        raise ValueError("kv_cache must be a contiguous bf16 [2, L, blocks, block_size, Hkv, hd] tensor")
    if old_slots.dtype != torch.int64 or new_slots.dtype != torch.int64:
        raise TypeError("old_slots/new_slots must be int64")
    n = old_slots.numel()
    if new_slots.numel() != n:
        raise ValueError("old_slots and new_slots differ in length")
    _, L, nb, bs, hkv, hd = kv_cache.shape
    nseg = 0
    if rotate_k:
        if cos_sin is None:
            raise ValueError("rotate_k needs a cos_sin table")
        if cos_sin.dtype != torch.float32 or not cos_sin.is_contiguous() or cos_sin.shape[1:] != (hd // 2, 2):
            raise ValueError("cos_sin must be contiguous fp32 [num_segments, head_dim/2, 2]")
        nseg = cos_sin.shape[0]
    if seg_of_token is not None:
        if seg_of_token.dtype != torch.int32 or seg_of_token.numel() != n:
            raise ValueError("seg_of_token must be int32 [n]")
    st = _lib.load().vlc_rerotate_copy_kv(
        kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.stride(1), L,
        old_slots.data_ptr(), new_slots.data_ptr(), n, nb * bs, hkv, hd,
        seg_of_token.data_ptr() if seg_of_token is not None else None,
        cos_sin.data_ptr() if (rotate_k and cos_sin is not None) else None,
        nseg, 1 if rotate_k else 0, _stream(kv_cache))
    _lib.check("vlc_rerotate_copy_kv", st)


# --------------------------------------------------------------------------- attention
@dataclass
class AttnPlan:
    """A work plan for vlc_varlen_attn_fwd, built once per step and shared by every layer."""
    host: np.ndarray           # int32 plan (kept alive: its pointer is passed to each call)
    dev: torch.Tensor          # device copy
    workspace: torch.Tensor | None
    num_seqs: int
    num_heads_q: int
    num_heads_kv: int
    causal: bool
    cu_seqlens_q: tuple
    cu_seqlens_k: tuple

    @property
    def num_items(self) -> int:
        return int(self.host[1])

    @property
    def num_combine(self) -> int:
        return int(self.host[2])

    @property
    def num_slots(self) -> int:
        return int(self.host[3])


def plan_attention_host(cu_seqlens_q, cu_seqlens_k, num_heads_q: int, num_heads_kv: int, head_dim: int,
                        causal: bool, num_cus: int = 256) -> tuple[np.ndarray, int]:
    """The host work list (vlc_attn_plan) from HOST sequence boundaries: (int32 plan, workspace bytes)."""
    lib = _lib.load()
    cu_q = np.ascontiguousarray(np.asarray(cu_seqlens_q, dtype=np.int32))
    cu_k = np.ascontiguousarray(np.asarray(cu_seqlens_k, dtype=np.int32))
    if cu_q.shape != cu_k.shape or cu_q.ndim != 1 or cu_q.size < 1:
        raise ValueError("cu_seqlens_q/k must be 1-D and of equal length")
    plan_len = ctypes.c_int64(0)
    ws = ctypes.c_int64(0)
    ip = ctypes.POINTER(ctypes.c_int32)
    args = (cu_q.ctypes.data_as(ip), cu_k.ctypes.data_as(ip), cu_q.size - 1, num_heads_q, num_heads_kv,
            head_dim, 1 if causal else 0, num_cus)
    st = lib.vlc_attn_plan(*args, None, 0, ctypes.byref(plan_len), ctypes.byref(ws))
    if st not in (0, _lib.VLC_ERR_CAPACITY):
        _lib.check("vlc_attn_plan", st)
    host = np.zeros(plan_len.value, dtype=np.int32)
    st = lib.vlc_attn_plan(*args, host.ctypes.data_as(ip), host.size, ctypes.byref(plan_len),
                           ctypes.byref(ws))
    _lib.check("vlc_attn_plan", st)
    return host, int(ws.value)


def attn_plan_on_device(host: np.ndarray, workspace_bytes: int, dev: torch.Tensor, cu_seqlens_q, cu_seqlens_k,
                        num_heads_q: int, num_heads_kv: int, causal: bool) -> AttnPlan:
    """An AttnPlan from a host plan and the caller's device copy of it (int32, same length); allocates
    the workspace on dev's device."""
    if dev.dtype != torch.int32 or dev.numel() != host.size or not dev.is_contiguous():
        raise ValueError("the device plan must be a contiguous int32 copy of the host plan")
    workspace = (torch.empty(workspace_bytes, dtype=torch.uint8, device=dev.device)
                 if workspace_bytes > 0 and dev.is_cuda else None)
    return AttnPlan(host, dev, workspace, len(cu_seqlens_q) - 1, num_heads_q, num_heads_kv, bool(causal),
                    tuple(int(x) for x in cu_seqlens_q), tuple(int(x) for x in cu_seqlens_k))


def plan_attention(cu_seqlens_q, cu_seqlens_k, num_heads_q: int, num_heads_kv: int,
                   head_dim: int, causal: bool, device, num_cus: int | None = None) -> AttnPlan:
    """Build the host work list (vlc_attn_plan) from HOST sequence boundaries and copy it to the device."""
    device = torch.device(device)
    if num_cus is None:
        num_cus = _num_cus(device) if device.type == "cuda" else 256
    host, ws = plan_attention_host(cu_seqlens_q, cu_seqlens_k, num_heads_q, num_heads_kv, head_dim, causal,
                                   num_cus)
    if device.type == "cuda":
        dev = torch.from_numpy(host).pin_memory().to(device, non_blocking=True)
    else:
        dev = torch.from_numpy(host.copy())
    return attn_plan_on_device(host, ws, dev, list(np.asarray(cu_seqlens_q).tolist()),
                               list(np.asarray(cu_seqlens_k).tolist()), num_heads_q, num_heads_kv, causal)


def _check_rows(name: str, t: torch.Tensor, heads: int) -> None:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bf16")
    if t.shape[-1] != HEAD_DIM or t.shape[-2] != heads:
        raise ValueError(f"{name}: expected [..., {heads}, {HEAD_DIM}], got {tuple(t.shape)}")
    if t.stride(-1) != 1 or t.stride(-2) != HEAD_DIM:
        raise ValueError(f"{name}: heads must be contiguous rows of {HEAD_DIM} elements")


def varlen_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, softmax_scale: float,
                     causal: bool = True, block_table: torch.Tensor | None = None,
                     plan: AttnPlan | None = None, out: torch.Tensor | None = None,
                     head_dim: int = HEAD_DIM) -> torch.Tensor:
    """Varlen GQA attention, paged (block_table given) or contiguous (vlc_varlen_attn_fwd).

    q: [total_q, Hq, 128] bf16.  Paged: k/v caches [num_blocks, page, Hkv, 128];
    contiguous: k/v [total_k, Hkv, 128] (v may be a strided view).  cu_seqlens_*:
    int32 device tensors.  plan: from plan_attention over the same host
    boundaries (and head_dim); when None it is built here from a device-to-host
    copy of the boundaries (a synchronisation).  head_dim 80 (contiguous only):
    heads stay 128-element rows, the products use dims 0..79 of q and k and
    0..95 of v (pass v zero-padded); output dims 96..127 are zero.
    """
    _require_device("varlen_attention", q, k, v, cu_seqlens_q, cu_seqlens_k, block_table)
    hq = q.shape[1]
    paged = block_table is not None
    hkv = k.shape[-2]
    _check_rows("q", q, hq)
    _check_rows("k", k, hkv)
    _check_rows("v", v, hkv)
    if cu_seqlens_q.dtype != torch.int32 or cu_seqlens_k.dtype != torch.int32:
        raise TypeError("cu_seqlens must be int32")
    num_seqs = cu_seqlens_q.numel() - 1
    if paged:
        if k.dim() != 4 or v.shape != k.shape:
            raise ValueError("paged k/v must be caches [num_blocks, page, Hkv, hd]")
        if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != num_seqs:
            raise ValueError("block_table must be int32 [num_seqs, max_blocks]")
        if block_table.stride(1) != 1:
            raise ValueError("block_table rows must be contiguous")
        k_rs, v_rs = k.stride(1), v.stride(1)
        if k.stride(0) != k.shape[1] * k_rs or v.stride(0) != v.shape[1] * v_rs:
            raise ValueError("paged caches must have contiguous pages")
        page, nblocks = k.shape[1], k.shape[0]
        bt_ptr, bt_rs = block_table.data_ptr(), block_table.stride(0)
    else:
        k_rs, v_rs = k.stride(0), v.stride(0)
        page, nblocks, bt_ptr, bt_rs = 0, 0, None, 0
    if head_dim not in ATTN_HEAD_DIMS or (head_dim != HEAD_DIM and paged):
        raise ValueError(f"head_dim {head_dim} is not supported (128, or 80 with contiguous k/v)")
    if plan is None:
        plan = plan_attention(cu_seqlens_q.tolist(), cu_seqlens_k.tolist(), hq, hkv, head_dim, causal,
                              q.device)
    if plan.num_seqs != num_seqs or plan.num_heads_q != hq or plan.num_heads_kv != hkv or plan.causal != bool(causal):
        raise ValueError("attention plan does not match the call")
    if int(plan.host[_PLAN_HEAD_DIM]) != head_dim:
        raise ValueError(f"attention plan was built for head_dim {int(plan.host[_PLAN_HEAD_DIM])}, the call has {head_dim}")
    # Bounds the kernel relies on, checked against the plan's host boundaries
    # (the device cu_seqlens must hold the same values).
    if plan.cu_seqlens_q[-1] > q.shape[0]:
        raise ValueError("cu_seqlens_q exceeds the rows of q")
    if paged:
        max_sk = max((plan.cu_seqlens_k[i + 1] - plan.cu_seqlens_k[i] for i in range(num_seqs)), default=0)
        if -(-max_sk // page) > block_table.shape[1]:
            raise ValueError("block_table has fewer columns than the longest sequence needs")
    elif plan.cu_seqlens_k[-1] > k.shape[0] or plan.cu_seqlens_k[-1] > v.shape[0]:
        raise ValueError("cu_seqlens_k exceeds the rows of k/v")
    if out is None:
        out = torch.empty(q.shape[0], hq, HEAD_DIM, dtype=torch.bfloat16, device=q.device)
    ws = plan.workspace
    st = _lib.load().vlc_varlen_attn_fwd(
        q.data_ptr(), q.stride(0), k.data_ptr(), k_rs, v.data_ptr(), v_rs,
        bt_ptr, bt_rs, page, nblocks, cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(),
        num_seqs, hq, hkv, head_dim, float(softmax_scale), 1 if causal else 0,
        plan.host.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), plan.dev.data_ptr(), plan.host.size,
        out.data_ptr(), out.stride(0), ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0, _stream(q))
    _lib.check("vlc_varlen_attn_fwd", st)
    return out


# --------------------------------------------------------------------------- decode attention
@dataclass
class DecodePlan:
    """Launch shape and workspace of vlc_decode_attn for one upper bound of the context length.

    The workspace's first batch * Hkv words are ticket counters: zero at
    allocation, and every call leaves them zero, so one plan serves every layer
    and step whose lengths stay within max_seqlen_k.
    """
    batch: int
    num_heads_q: int
    num_heads_kv: int
    page_size: int
    max_seqlen_k: int
    key_chunk: int
    grid_splits: int
    pipeline: int
    workspace: torch.Tensor | None
    workspace_bytes: int = 0


def decode_supported(num_heads_q: int, num_heads_kv: int, head_dim: int, page_size: int) -> bool:
    """Shapes vlc_decode_attn takes: head_dim 128, at most 16 q heads per kv head, page_size % 16 == 0."""
    return (head_dim == HEAD_DIM and num_heads_q % num_heads_kv == 0 and num_heads_q // num_heads_kv <= 16
            and page_size % 16 == 0)


def plan_decode(batch: int, num_heads_q: int, num_heads_kv: int, head_dim: int, page_size: int,
                max_seqlen_k: int, device, num_cus: int | None = None, num_splits: int = 0,
                pipeline: int = 0, workspace: bool = True) -> DecodePlan:
    """Size a decode launch (vlc_decode_attn_plan) and allocate its zeroed workspace.

    pipeline: kernel shape, 16 * waves per workgroup + stages per wave, plus 0x100
    for 16-key tiles (0x42, 0x22, 0x23, 0x24, 0x14, 0x142, 0x144, 0x182, 0x124),
    0 = the library's choice.  workspace=False sizes the launch only (for
    decode_attention_noalloc, which allocates nothing); plan.workspace is None.
    """
    lib = _lib.load()
    device = torch.device(device)
    if num_cus is None:
        num_cus = _num_cus(device) if device.type == "cuda" else 256
    chunk = ctypes.c_int32(0)
    splits = ctypes.c_int32(0)
    pipe = ctypes.c_int32(0)
    ws = ctypes.c_int64(0)
    st = lib.vlc_decode_attn_plan(batch, num_heads_q, num_heads_kv, head_dim, page_size, int(max_seqlen_k),
                                  num_cus, num_splits, pipeline, ctypes.byref(chunk), ctypes.byref(splits),
                                  ctypes.byref(pipe), ctypes.byref(ws))
    _lib.check("vlc_decode_attn_plan", st)
    buf = torch.zeros(max(ws.value, 16), dtype=torch.uint8, device=device) if workspace else None
    return DecodePlan(batch, num_heads_q, num_heads_kv, page_size, int(max_seqlen_k), chunk.value, splits.value,
                      pipe.value, buf, ws.value)


def _decode_args(q, k_cache, v_cache, cache_seqlens, block_table, out):
    """Shape checks shared by both decode entry points; returns (B, hq, hkv, page, nblocks)."""
    _require_device("decode_attention", q, k_cache, v_cache, cache_seqlens, block_table, out)
    B, hq = q.shape[0], q.shape[1]
    hkv = k_cache.shape[-2]
    _check_rows("q", q, hq)
    _check_rows("k_cache", k_cache, hkv)
    _check_rows("v_cache", v_cache, hkv)
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache/v_cache must be [num_blocks, page, Hkv, hd]")
    if k_cache.stride(0) != k_cache.shape[1] * k_cache.stride(1) or v_cache.stride(1) != k_cache.stride(1) \
            or v_cache.stride(0) != k_cache.stride(0):
        raise ValueError("paged caches must have contiguous pages and equal strides")
    if cache_seqlens.dtype != torch.int32 or cache_seqlens.numel() != B:
        raise ValueError("cache_seqlens must be int32 [B]")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != B \
            or block_table.stride(1) != 1:
        raise ValueError("block_table must be int32 [B, max_blocks] with contiguous rows")
    if out is not None and (out.shape != (B, hq, HEAD_DIM) or out.dtype != torch.bfloat16 or out.stride(-1) != 1
                            or out.stride(1) != HEAD_DIM):
        raise ValueError("out must be bf16 [B, Hq, 128] with contiguous head rows")
    return B, hq, hkv, k_cache.shape[1], k_cache.shape[0]


def _check_decode_plan(plan: DecodePlan, B, hq, hkv, page, max_seqlen_k):
    if (plan.batch, plan.num_heads_q, plan.num_heads_kv, plan.page_size) != (B, hq, hkv, page):
        raise ValueError("decode plan does not match the call")
    # The kernel attends at most the keys its grid covers (grid_splits * key_chunk,
    # i.e. the plan's max_seqlen_k rounded up): a longer context would be cut short.
    if max_seqlen_k is not None and int(max_seqlen_k) > plan.max_seqlen_k:
        raise ValueError(f"decode plan covers {plan.max_seqlen_k} keys, the call has contexts up to "
                         f"{int(max_seqlen_k)}: plan for the longest context")


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, cache_seqlens: torch.Tensor,
                     block_table: torch.Tensor, softmax_scale: float, plan: DecodePlan | None = None,
                     max_seqlen_k: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Paged GQA decode attention, one query per sequence (vlc_decode_attn).

    q: [B, Hq, 128] bf16 (any row stride between sequences); k_cache/v_cache:
    [num_blocks, page, Hkv, 128]; cache_seqlens: int32 [B] on the device;
    block_table: int32 [B, max_blocks].  The plan must cover the longest length:
    max_seqlen_k, when given, is checked against it.  Without a plan one is
    built here from max_seqlen_k, or from cache_seqlens (a device-to-host copy).
    Returns [B, Hq, 128].
    """
    B, hq, hkv, page, nblocks = _decode_args(q, k_cache, v_cache, cache_seqlens, block_table, out)
    if plan is None:
        if max_seqlen_k is None:
            max_seqlen_k = int(cache_seqlens.max().item()) if B else 0
        plan = plan_decode(B, hq, hkv, HEAD_DIM, page, max_seqlen_k, q.device)
    _check_decode_plan(plan, B, hq, hkv, page, max_seqlen_k)
    if plan.workspace is None:
        raise ValueError("decode plan has no workspace (built with workspace=False): use decode_attention_noalloc")
    if out is None:
        out = torch.empty(B, hq, HEAD_DIM, dtype=torch.bfloat16, device=q.device)
    ws = plan.workspace
    st = _lib.load().vlc_decode_attn(
        q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(1), page, nblocks,
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1], cache_seqlens.data_ptr(), B, hq, hkv,
        HEAD_DIM, float(softmax_scale), plan.key_chunk, plan.grid_splits, plan.pipeline, out.data_ptr(), out.stride(0),
        ws.data_ptr(), ws.numel(), _stream(q))
    _lib.check("vlc_decode_attn", st)
    return out


def decode_attention_noalloc(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                             cache_seqlens: torch.Tensor, block_table: torch.Tensor, softmax_scale: float,
                             plan: DecodePlan, out: torch.Tensor, max_seqlen_k: int | None = None) -> torch.Tensor:
    """decode_attention through vlc_decode_attn_noalloc: nothing is allocated.

    For callers that cannot allocate device memory (HIP graph capture, tight
    serving loops).  The split partials and ticket counters live in the
    library's fixed per-device scratch (DECODE_NOALLOC_MAX_BYTES); out is
    required; the plan only sizes the launch (plan_decode(..., workspace=False)
    builds one without a buffer).  Calls that overlap on one device race.
    """
    if out is None:
        raise ValueError("decode_attention_noalloc writes into a caller-supplied out")
    B, hq, hkv, page, nblocks = _decode_args(q, k_cache, v_cache, cache_seqlens, block_table, out)
    _check_decode_plan(plan, B, hq, hkv, page, max_seqlen_k)
    if plan.grid_splits > 1 and plan.workspace_bytes > _lib.DECODE_NOALLOC_MAX_BYTES:
        raise ValueError(f"decode call needs {plan.workspace_bytes} bytes of scratch, more than the "
                         f"{_lib.DECODE_NOALLOC_MAX_BYTES} of the allocation-free entry point")
    st = _lib.load().vlc_decode_attn_noalloc(
        q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(1), page, nblocks,
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1], cache_seqlens.data_ptr(), B, hq, hkv,
        HEAD_DIM, float(softmax_scale), plan.key_chunk, plan.grid_splits, plan.pipeline, out.data_ptr(), out.stride(0),
        _stream(q))
    _lib.check("vlc_decode_attn_noalloc", st)
    return out


# --------------------------------------------------------------------------- vision tower
def vision_rope_pad(qkv: torch.Tensor, pos_hw: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor,
                    num_heads: int, head_dim: int, padded_dim: int = HEAD_DIM,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """2-D rotary of the vision tower's q and k, split into padded head rows (vlc_vision_rope_pad).

    qkv: [N, 3 * num_heads * head_dim] bf16 (rows 16-byte aligned); pos_hw: int32
    [N, 2] (patch row, patch column); cos/sin tables: bf16 [max_pos, head_dim // 4].
    Returns out [N, 3, num_heads, padded_dim] bf16: q, k rotated, v copied, dims
    head_dim.. zero.
    """
    _require_device("vision_rope_pad", qkv, pos_hw, cos_table, sin_table, out)
    n = qkv.shape[0]
    if qkv.dtype != torch.bfloat16 or qkv.dim() != 2 or qkv.shape[1] != 3 * num_heads * head_dim or qkv.stride(1) != 1:
        raise ValueError(f"qkv must be bf16 [N, {3 * num_heads * head_dim}] with contiguous rows")
    if pos_hw.dtype != torch.int32 or tuple(pos_hw.shape) != (n, 2) or not pos_hw.is_contiguous():
        raise ValueError("pos_hw must be contiguous int32 [N, 2]")
    q4 = head_dim // 4
    for name, t in (("cos_table", cos_table), ("sin_table", sin_table)):
        if t.dtype != torch.bfloat16 or t.dim() != 2 or t.shape[1] != q4 or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous bf16 [max_pos, {q4}]")
    if cos_table.shape != sin_table.shape:
        raise ValueError("cos_table and sin_table differ in shape")
    if out is None:
        out = torch.empty(n, 3, num_heads, padded_dim, dtype=torch.bfloat16, device=qkv.device)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (n, 3, num_heads, padded_dim) or \
            out.stride(3) != 1 or out.stride(2) != padded_dim or out.stride(1) != num_heads * padded_dim:
        raise ValueError(f"out must be bf16 [N, 3, {num_heads}, {padded_dim}] with contiguous token rows")
    st = _lib.load().vlc_vision_rope_pad(
        qkv.data_ptr(), qkv.stride(0), pos_hw.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(),
        cos_table.shape[0], n, num_heads, head_dim, padded_dim, out.data_ptr(), out.stride(0), _stream(qkv))
    _lib.check("vlc_vision_rope_pad", st)
    return out


# --------------------------------------------------------------------------- norm and activation
def _rows2d(name: str, t: torch.Tensor, dim: int) -> None:
    if t.dtype != torch.bfloat16 or t.dim() != 2 or t.shape[1] != dim or t.stride(1) != 1:
        raise ValueError(f"{name} must be bf16 [rows, {dim}] with contiguous rows, got "
                         f"{tuple(t.shape)} {t.dtype}")


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None,
             out: torch.Tensor | None = None, residual_out: torch.Tensor | None = None):
    """RMSNorm of x [rows, dim] bf16 (vlc_rms_norm); with residual, of x + residual.

    Returns out, or (out, residual_out) when residual is given: residual_out =
    bf16(x + residual) (written in place into `residual` when residual_out is
    None), out the normalised fp32 sum times weight.
    """
    _require_device("rms_norm", x, weight, residual, out, residual_out)
    lead = x.shape[:-1]
    dim = x.shape[-1]
    x2 = x.reshape(-1, dim)
    _rows2d("x", x2, dim)
    if weight.dtype != torch.bfloat16 or weight.shape != (dim,) or not weight.is_contiguous():
        raise ValueError(f"weight must be contiguous bf16 [{dim}]")
    rows = x2.shape[0]
    o = torch.empty(rows, dim, dtype=torch.bfloat16, device=x.device) if out is None else out.reshape(-1, dim)
    _rows2d("out", o, dim)
    if residual is not None:
        r2 = residual.reshape(-1, dim)
        _rows2d("residual", r2, dim)
        ro = r2 if residual_out is None else residual_out.reshape(-1, dim)
        _rows2d("residual_out", ro, dim)
        if r2.shape[0] != rows or ro.shape[0] != rows:
            raise ValueError("x and residual differ in rows")
        rp, rs, rop, ros = r2.data_ptr(), r2.stride(0), ro.data_ptr(), ro.stride(0)
    else:
        rp, rs, rop, ros = None, 0, None, 0
    if o.shape[0] != rows:
        raise ValueError("out has the wrong number of rows")
    st = _lib.load().vlc_rms_norm(x2.data_ptr(), x2.stride(0), rp, rs, rop, ros, weight.data_ptr(), float(eps),
                                  rows, dim, o.data_ptr(), o.stride(0), _stream(x))
    _lib.check("vlc_rms_norm", st)
    o = o.view(*lead, dim)
    if residual is None:
        return o
    return o, ro.view(*lead, dim)


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """silu(gate) * up of a packed [rows, 2 * inter] bf16 projection (vlc_silu_mul) -> [rows, inter]."""
    _require_device("silu_mul", gate_up, out)
    lead = gate_up.shape[:-1]
    two = gate_up.shape[-1]
    if two % 2:
        raise ValueError("gate_up's last dim must be even")
    inter = two // 2
    g2 = gate_up.reshape(-1, two)
    _rows2d("gate_up", g2, two)
    rows = g2.shape[0]
    o = torch.empty(rows, inter, dtype=torch.bfloat16, device=gate_up.device) if out is None else out.reshape(-1, inter)
    _rows2d("out", o, inter)
    st = _lib.load().vlc_silu_mul(g2.data_ptr(), g2.stride(0), rows, inter, o.data_ptr(), o.stride(0),
                                  _stream(gate_up))
    _lib.check("vlc_silu_mul", st)
    return o.view(*lead, inter)


# --------------------------------------------------------------------------- skinny linear
SKINNY_MAX_ROWS = 16


def linear_skinny_supported(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> bool:
    """Whether vlc_linear_skinny takes this call (bf16, at most 16 rows, K % 32, N % 16, aligned rows)."""
    if not (x.is_cuda and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and x.dim() == 2):
        return False
    m, k = x.shape
    n = weight.shape[0]
    if m > SKINNY_MAX_ROWS or k % 32 or n % 16 or weight.shape[1] != k:
        return False
    if x.stride(1) != 1 or weight.stride(1) != 1 or x.stride(0) % 8 or weight.stride(0) % 8:
        return False
    if x.data_ptr() % 16 or weight.data_ptr() % 16:
        return False
    if bias is not None and (bias.dtype != torch.bfloat16 or not bias.is_contiguous() or bias.data_ptr() % 8):
        return False
    return True


def linear_skinny(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """x [M <= 16, K] @ weight[N, K]^T + bias (vlc_linear_skinny): the decode-step projections,
    weight-streaming on the matrix pipe; fp32 accumulation, one rounding to bf16."""
    _require_device("linear_skinny", x, weight, bias, out)
    if not linear_skinny_supported(x, weight, bias):
        raise ValueError(f"linear_skinny does not take x {tuple(x.shape)} / weight {tuple(weight.shape)}")
    m, k = x.shape
    n = weight.shape[0]
    if out is None:
        out = torch.empty(m, n, dtype=torch.bfloat16, device=x.device)
    st = _lib.load().vlc_linear_skinny(x.data_ptr(), x.stride(0), m, k, weight.data_ptr(), weight.stride(0), n,
                                       bias.data_ptr() if bias is not None else None, out.data_ptr(), out.stride(0),
                                       _stream(x))
    _lib.check("vlc_linear_skinny", st)
    return out
