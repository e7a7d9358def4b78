"""Prefill-first scheduler (reference: nanovllm/engine/scheduler.py:25-73).

Same policy as the reference: when requests are waiting, admit them in FIFO
order while the running set stays within `max_num_seqs` sequences, the batch within
`max_num_batched_tokens` prompt tokens and a KV-cache slot is free, and run
that prefill batch; otherwise run one decode step over every running
sequence. A sequence finishes on EOS (unless `ignore_eos`) or after
`max_tokens` generated tokens, and its slot is released.

KV memory is one contiguous slot of `max_model_len` positions per running
sequence, reserved at admission (see model_runner), so a running sequence can
always append and the reference's preemption path never triggers.
"""
from __future__ import annotations

from collections import deque

from nanovllm.engine.sequence import Sequence, SequenceStatus


class Scheduler:
    def __init__(self, max_num_seqs: int, max_num_batched_tokens: int, num_slots: int, eos: int):
        self.max_num_seqs = max_num_seqs
        self.max_num_batched_tokens = max_num_batched_tokens
        self.eos = eos
        self.free_slots = list(range(num_slots))[::-1]  # pop() hands out the lowest slot first
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()

    def is_finished(self) -> bool:
        return not self.waiting and not self.running

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    def schedule(self) -> tuple[list[Sequence], bool]:
        scheduled: list[Sequence] = []
        num_tokens = 0
        while self.waiting and len(self.running) < self.max_num_seqs and self.free_slots:
            seq = self.waiting[0]
            if num_tokens + len(seq) > self.max_num_batched_tokens:
                break
            self.waiting.popleft()
            seq.slot = self.free_slots.pop()
            seq.status = SequenceStatus.RUNNING
            num_tokens += len(seq)
            self.running.append(seq)
            scheduled.append(seq)
        if scheduled:
            return scheduled, True
        if not self.running:
            raise RuntimeError("a waiting request exceeds max_num_batched_tokens")
        return list(self.running), False

    def postprocess(self, seqs: list[Sequence], token_ids: list[int]) -> None:
        for seq, tok in zip(seqs, token_ids):
            seq.append_token(tok)
            if (not seq.ignore_eos and tok == self.eos) or seq.num_completion_tokens == seq.max_tokens:
                seq.status = SequenceStatus.FINISHED
                self.running.remove(seq)
                self.free_slots.append(seq.slot)
                self.free_slots.sort(reverse=True)
                seq.slot = -1
