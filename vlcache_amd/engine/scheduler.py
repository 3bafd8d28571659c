"""Prefill-first FCFS scheduler (engine/scheduler.py:22-77 of the reference).

The token budget discounts reused image tokens (:29-47); decode appends one
token per running sequence and preempts from the back when blocks run out.
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

    def is_finished(self):
        return not self.waiting and not self.running

    def add(self, seq: Sequence):
        self.waiting.append(seq)

    def schedule(self) -> tuple[list[Sequence], bool]:
        scheduled = []
        num_seqs = 0
        num_batched_tokens = 0
        while self.waiting and num_seqs < self.max_num_seqs:
            seq = self.waiting[0]
            self.block_manager.try_partial_recompute(seq, self.image_token_id)
            if seq.is_partial_recompute:
                token_cost = len(seq) - seq.num_reused_tokens  # reused image tokens cost nothing
            else:
                token_cost = len(seq)
            if num_batched_tokens + token_cost > self.max_num_batched_tokens or not self.block_manager.can_allocate(seq):
                seq.reset_partial_recompute()
                break
            num_seqs += 1
            self.block_manager.allocate(seq)
            num_batched_tokens += token_cost
            seq.status = SequenceStatus.RUNNING
            self.waiting.popleft()
            self.running.append(seq)
            scheduled.append(seq)
        if scheduled:
            return scheduled, True
        while self.running and num_seqs < self.max_num_seqs:
            seq = self.running.popleft()
            while not self.block_manager.can_append(seq):
                if self.running:
                    self.preempt(self.running.pop())
                else:
                    self.preempt(seq)
                    break
            else:
                num_seqs += 1
                self.block_manager.may_append(seq)
                scheduled.append(seq)
        assert scheduled
        self.running.extendleft(reversed(scheduled))
        return scheduled, False

    def preempt(self, seq: Sequence):
        seq.status = SequenceStatus.WAITING
        seq.reset_partial_recompute()
        self.block_manager.deallocate(seq)
        self.waiting.appendleft(seq)

    def postprocess(self, seqs: list[Sequence], token_ids: list[int]):
        for seq, token_id in zip(seqs, token_ids):
            seq.append_token(token_id)
            if (not seq.ignore_eos and token_id == self.eos) or seq.num_completion_tokens == seq.max_tokens:
                seq.status = SequenceStatus.FINISHED
                self.block_manager.deallocate(seq)
                self.running.remove(seq)
