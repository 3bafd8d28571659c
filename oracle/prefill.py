"""Integer host logic of the warm partial-recompute prefill (oracle; test-only).

Each function restates a reference function line for line in plain Python and
cites it.  Tests pin them with hand-derived known answers and invariants.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

IMAGE_TOKEN_ID = 151655  # engine/scheduler.py:10 (getattr default), test_partial_recompute.py:56
BLOCK_SIZE = 256  # engine/sequence.py:16 (Sequence.block_size, hard-coded)


def recompute_count(ratio: float, n_image_tokens: int) -> int:
    """R = ceil(ratio * N) in IEEE double (engine/block_manager.py:72)."""
    return math.ceil(ratio * n_image_tokens)


def find_image_token_range(token_ids, image_token_id: int = IMAGE_TOKEN_ID):
    """First to last image token, end exclusive; None without one (engine/sequence.py:91-100)."""
    start = end = -1
    for i, tid in enumerate(token_ids):
        if tid == image_token_id:
            if start == -1:
                start = i
            end = i + 1
    return None if start == -1 else (start, end)


def compute_slots(block_table, start: int, end: int, block_size: int = BLOCK_SIZE):
    """slot(p) = bt[p // bs] * bs + p % bs for p in [start, end) (engine/model_runner.py:160-168)."""
    return [block_table[p // block_size] * block_size + p % block_size for p in range(start, end)]


def image_kv_copy_slots(entry_block_table, entry_img_start, seq_block_table, img_start, img_end, R,
                        block_size: int = BLOCK_SIZE):
    """old/new slots of the reused image tokens (engine/llm_engine.py:70-88).

    Reused tokens are p in [img_start + R, img_end); the source sits at the same
    offset inside the cached entry's image (old_p = entry_img_start + p - img_start).
    """
    old, new = [], []
    for p in range(img_start + R, img_end):
        old_p = entry_img_start + (p - img_start)
        old.append(entry_block_table[old_p // block_size] * block_size + old_p % block_size)
    for p in range(img_start + R, img_end):
        new.append(seq_block_table[p // block_size] * block_size + p % block_size)
    return old, new


@dataclass
class SeqSpec:
    """The Sequence fields prepare_prefill reads (engine/sequence.py:15-37)."""
    token_ids: list
    block_table: list
    is_partial_recompute: bool = False
    image_token_range: tuple | None = None
    num_recompute_tokens: int = 0


@dataclass
class PrefillPlan:
    input_ids: list = field(default_factory=list)
    positions: list = field(default_factory=list)
    cu_seqlens_q: list = field(default_factory=lambda: [0])
    cu_seqlens_k: list = field(default_factory=lambda: [0])
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: list = field(default_factory=list)
    block_tables: list | None = None  # padded with -1; None unless a sequence is partial
    logit_indices: list | None = None


def prepare_prefill(seqs, block_size: int = BLOCK_SIZE) -> PrefillPlan:
    """Virtual sub-sequences, slot mapping and block tables (engine/model_runner.py:194-320).

    A partial sequence contributes two virtual sub-sequences (:237-276):
      sub1: Q = K = tokens [0, img_start + R)
      sub2: Q = tokens [img_end, len), K = tokens [0, len)
    A normal sequence contributes one (:278-292).  Block tables exist only when
    some sequence is partial (:294-299); rows are padded with -1 (:182-186).
    """
    out = PrefillPlan()
    vbts = []
    logit_indices = []
    vidx = 0
    has_partial = False
    for seq in seqs:
        seqlen = len(seq.token_ids)
        if seq.is_partial_recompute:
            has_partial = True
            img_start, img_end = seq.image_token_range
            R = seq.num_recompute_tokens
            q1 = k1 = img_start + R
            q2, k2 = seqlen - img_end, seqlen
            out.input_ids += seq.token_ids[0:img_start + R] + seq.token_ids[img_end:seqlen]
            out.positions += list(range(0, img_start + R)) + list(range(img_end, seqlen))
            out.cu_seqlens_q.append(out.cu_seqlens_q[-1] + q1)
            out.cu_seqlens_k.append(out.cu_seqlens_k[-1] + k1)
            out.cu_seqlens_q.append(out.cu_seqlens_q[-1] + q2)
            out.cu_seqlens_k.append(out.cu_seqlens_k[-1] + k2)
            out.max_seqlen_q = max(out.max_seqlen_q, q1, q2)
            out.max_seqlen_k = max(out.max_seqlen_k, k1, k2)
            if seq.block_table:
                out.slot_mapping += compute_slots(seq.block_table, 0, img_start + R, block_size)
                out.slot_mapping += compute_slots(seq.block_table, img_end, seqlen, block_size)
                vbts.append(list(seq.block_table))
                vbts.append(list(seq.block_table))
            logit_indices.append(vidx + 1)
            vidx += 2
        else:
            out.input_ids += list(seq.token_ids)
            out.positions += list(range(seqlen))
            out.cu_seqlens_q.append(out.cu_seqlens_q[-1] + seqlen)
            out.cu_seqlens_k.append(out.cu_seqlens_k[-1] + seqlen)
            out.max_seqlen_q = max(out.max_seqlen_q, seqlen)
            out.max_seqlen_k = max(out.max_seqlen_k, seqlen)
            if seq.block_table:
                out.slot_mapping += compute_slots(seq.block_table, 0, seqlen, block_size)
                vbts.append(list(seq.block_table))
            logit_indices.append(vidx)
            vidx += 1
    if has_partial and vbts:
        width = max(len(bt) for bt in vbts)
        out.block_tables = [bt + [-1] * (width - len(bt)) for bt in vbts]
    out.logit_indices = logit_indices if has_partial else None
    return out


def computed_runs(n_tokens: int, image_ranges, recompute_counts):
    """Maximal runs of recomputed tokens of one sequence with several images.

    Extends prepare_prefill's two sub-sequences (engine/model_runner.py:237-259)
    to any number of images: image k keeps its first R_k tokens computed and
    reuses the rest; every maximal run [a, b) of computed tokens becomes a
    virtual sub-sequence with Q = [a, b) and K = [0, b).  With one image this
    gives exactly the reference's (sub1, sub2) pair.
    Returns a list of (q_start, q_end) with K length = q_end.
    """
    computed = [True] * n_tokens
    for (s, e), r in zip(image_ranges, recompute_counts):
        for p in range(s + r, e):
            computed[p] = False
    runs = []
    p = 0
    while p < n_tokens:
        if computed[p]:
            a = p
            while p < n_tokens and computed[p]:
                p += 1
            runs.append((a, p))
        else:
            p += 1
    return runs
