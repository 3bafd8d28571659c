"""Step scheduler: prefill first, then decode, with recompute preemption.

Policy (the reference's, engine/scheduler.py:22-77): a step is a prefill step
whenever a waiting request can be admitted -- requests are admitted in arrival
order while the step's token budget (max_num_batched_tokens, where a warm
request pays only for the tokens it computes, :29-47) and the free blocks
allow; the first one that does not fit stops admission.  Otherwise it is a
decode step over the running requests in order; when the pool cannot give a
request the block its next token needs, the most recently admitted running
request is preempted (its blocks freed, back to the front of the waiting
queue, its prefill redone later), and a request that is the last one left
preempts itself.

Structure: admission and decode planning are separate functions; a decode step
whose block demand fits the free pool (the usual case) is planned in one pass
without the per-request preemption loop.  One addition to the policy: when a
request does not fit the free blocks, registered image KV that no request of
the step reuses is released (least recently used first) before admission gives
up; the reference never releases it, and its pool fills with image blocks.
"""
from __future__ import annotations

from collections import deque

from ..config import Config
from .block_manager import BlockManager
from .sequence import Sequence, SequenceStatus


class Scheduler:

    def __init__(self, config: Config):
        self.max_num_seqs = config.max_num_seqs
        self.max_num_batched_tokens = config.max_num_batched_tokens
        self.eos = config.eos
        self.image_token_id = getattr(config.hf_config, "image_token_id", 151655)
        self.block_manager = BlockManager(config.num_kvcache_blocks, config.kvcache_block_size,
                                          recompute_ratio=config.recompute_ratio)
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()

    def is_finished(self) -> bool:
        return not (self.waiting or self.running)

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    def schedule(self) -> tuple[list[Sequence], bool]:
        batch = self._admit()
        if batch:
            return batch, True
        batch = self._plan_decode()
        if not batch:
            raise RuntimeError("nothing to schedule: no request fits the KV block pool")
        return batch, False

    # ------------------------------------------------------------------ prefill
    def _admit(self) -> list[Sequence]:
        bm = self.block_manager
        admitted: list[Sequence] = []
        budget = self.max_num_batched_tokens
        while self.waiting and len(admitted) < self.max_num_seqs:
            seq = self.waiting[0]
            bm.try_partial_recompute(seq, self.image_token_id)
            cost = seq.prefill_cost
            if cost <= budget and not bm.can_allocate(seq):
                # registered images this step copies from stay; older ones make room
                keep = {sp.hash for s in (*admitted, seq) for sp in s.images if sp.reused > 0}
                bm.evict_images(seq.num_blocks, keep)
            if cost > budget or not bm.can_allocate(seq):
                seq.reset_partial_recompute()
                break
            bm.allocate(seq)
            budget -= cost
            seq.status = SequenceStatus.RUNNING
            self.running.append(self.waiting.popleft())
            admitted.append(seq)
        return admitted

    # ------------------------------------------------------------------ decode
    def _plan_decode(self) -> list[Sequence]:
        bm = self.block_manager
        n = min(len(self.running), self.max_num_seqs)
        front = [self.running[i] for i in range(n)]
        if sum(bm.blocks_to_append(s) for s in front) <= bm.num_free_blocks:
            for s in front:  # no pressure: the first n running requests all step
                bm.may_append(s)
            return front
        return self._plan_decode_under_pressure()

    def _plan_decode_under_pressure(self) -> list[Sequence]:
        bm = self.block_manager
        stepping: list[Sequence] = []
        pending = self.running
        while pending and len(stepping) < self.max_num_seqs:
            seq = pending.popleft()
            while bm.num_free_blocks < bm.blocks_to_append(seq) and pending:
                self.preempt(pending.pop())  # newest first
            if bm.num_free_blocks < bm.blocks_to_append(seq):
                self.preempt(seq)
                continue
            bm.may_append(seq)
            stepping.append(seq)
        # the requests that step keep their place at the front of the running queue
        self.running.extendleft(reversed(stepping))
        return stepping

    def preempt(self, seq: Sequence) -> None:
        seq.status = SequenceStatus.WAITING
        seq.reset_partial_recompute()
        self.block_manager.deallocate(seq)
        self.waiting.appendleft(seq)

    # ------------------------------------------------------------------ results
    def postprocess(self, seqs: list[Sequence], token_ids: list[int]) -> None:
        for seq, tok in zip(seqs, token_ids):
            seq.append_token(tok)
            done = seq.num_completion_tokens == seq.max_tokens or (not seq.ignore_eos and tok == self.eos)
            if done:
                seq.status = SequenceStatus.FINISHED
                self.block_manager.deallocate(seq)
                self.running.remove(seq)
