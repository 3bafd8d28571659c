"""Block pool and step scheduler of the reference, restated in plain Python (test-only).

Follows engine/block_manager.py:25-53,112-128 (a FIFO deque of free block ids,
reference counts; a sequence's blocks are released last to first) and
engine/scheduler.py:22-77 (prefill-first admission under a token budget,
decode with preemption of the newest running sequence, recompute on
re-admission), on text-only sequences.  Tests drive it and the package's
Scheduler with the same requests and compare every step.
"""
from __future__ import annotations

from collections import deque


class Seq:
    def __init__(self, seq_id: int, prompt_len: int, max_tokens: int):
        self.seq_id = seq_id
        self.num_tokens = prompt_len
        self.num_prompt_tokens = prompt_len
        self.max_tokens = max_tokens
        self.block_table: list[int] = []
        self.status = "waiting"

    def num_blocks(self, bs: int) -> int:
        return (self.num_tokens + bs - 1) // bs


class Pool:
    """engine/block_manager.py:25-53,112-128."""

    def __init__(self, num_blocks: int, block_size: int):
        self.bs = block_size
        self.ref = [0] * num_blocks
        self.free = deque(range(num_blocks))

    def take(self) -> int:
        b = self.free.popleft()
        self.ref[b] = 1
        return b

    def release(self, seq: Seq) -> None:
        for b in reversed(seq.block_table):
            self.ref[b] -= 1
            if self.ref[b] == 0:
                self.free.append(b)
        seq.block_table.clear()


class Scheduler:
    """engine/scheduler.py:22-77 (text-only: the token cost is the sequence length)."""

    def __init__(self, num_blocks: int, block_size: int, max_num_seqs: int, max_num_batched_tokens: int):
        self.pool = Pool(num_blocks, block_size)
        self.max_num_seqs = max_num_seqs
        self.max_num_batched_tokens = max_num_batched_tokens
        self.waiting: deque[Seq] = deque()
        self.running: deque[Seq] = deque()

    def schedule(self):
        scheduled, num_seqs, num_tokens = [], 0, 0
        bs = self.pool.bs
        while self.waiting and num_seqs < self.max_num_seqs:
            seq = self.waiting[0]
            if num_tokens + seq.num_tokens > self.max_num_batched_tokens or \
                    len(self.pool.free) < seq.num_blocks(bs):
                break
            num_seqs += 1
            seq.block_table = [self.pool.take() for _ in range(seq.num_blocks(bs))]
            num_tokens += seq.num_tokens
            seq.status = "running"
            self.waiting.popleft()
            self.running.append(seq)
            scheduled.append(seq)
        if scheduled:
            return scheduled, True
        while self.running and num_seqs < self.max_num_seqs:
            seq = self.running.popleft()
            while len(self.pool.free) < (seq.num_tokens % bs == 1):
                if self.running:
                    self.preempt(self.running.pop())
                else:
                    self.preempt(seq)
                    break
            else:
                num_seqs += 1
                if seq.num_tokens % bs == 1:
                    seq.block_table.append(self.pool.take())
                scheduled.append(seq)
        assert scheduled
        self.running.extendleft(reversed(scheduled))
        return scheduled, False

    def preempt(self, seq: Seq) -> None:
        seq.status = "waiting"
        self.pool.release(seq)
        self.waiting.appendleft(seq)

    def postprocess(self, seqs) -> None:
        for seq in seqs:
            seq.num_tokens += 1
            if seq.num_tokens - seq.num_prompt_tokens == seq.max_tokens:
                seq.status = "finished"
                self.pool.release(seq)
                self.running.remove(seq)
