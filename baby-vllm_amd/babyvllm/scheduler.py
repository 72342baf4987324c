"""Continuous-batching scheduler (babyvllm/scheduler.py:13-158).

Each step first continues the running sequences in order (decode tokens, or
the rest of a recomputed prompt), preempting from the back of the running list
(recompute: the victim's pages are freed and it is re-queued at the front of
the waiting queue) when the pool runs out; then admits waiting sequences in
order while the token budget, the sequence cap and the pool allow, reusing
prefix-cached pages. A whole prompt is scheduled in one step; a prompt longer
than the token budget, or needing more pages than the pool has, finishes with
reason LENGTH. The output carries each scheduled sequence's block table and
slot mapping, the inputs of the paged-KV kernels.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass

from babyvllm.kv_cache_manager import KVCacheManager
from babyvllm.sequence import Sequence, SequenceFinishReason, SequenceState


@dataclass
class SchedulerOutput:
    scheduled_sequences: list[Sequence]
    num_scheduled_tokens: dict[int, int]
    block_tables: dict[int, list[int]]
    slot_mappings: dict[int, list[int]]
    preempted_seqs: list[Sequence]


class Scheduler:
    def __init__(self, kv_cache_manager: KVCacheManager, max_num_batched_tokens: int = 2048,
                 max_num_seqs: int = 256):
        self.kv_cache_manager = kv_cache_manager
        self.max_num_batched_tokens = max_num_batched_tokens
        self.max_num_seqs = max_num_seqs
        self.waiting: deque[Sequence] = deque()
        self.running: list[Sequence] = []
        self.finished_seqs: list[Sequence] = []

    # ------------------------------------------------------------- lifecycle

    def _too_long(self, seq: Sequence, tokens: int) -> bool:
        kv = self.kv_cache_manager
        return tokens > self.max_num_batched_tokens or kv.num_blocks_needed(seq, tokens) > kv.num_blocks

    def add_seq(self, seq: Sequence) -> None:
        if self._too_long(seq, len(seq)):
            self._finish(seq, SequenceFinishReason.LENGTH)
            return
        seq.status = SequenceState.WAITING
        self.waiting.append(seq)

    def admit_seq(self, seq: Sequence) -> None:
        head = self.waiting.popleft()
        assert head is seq
        seq.status = SequenceState.RUNNING
        self.running.append(seq)

    def abort_seq(self, seq: Sequence) -> None:
        self._finish(seq, SequenceFinishReason.ABORT)

    def free_seq(self, seq: Sequence) -> None:
        if seq in self.running:
            self.running.remove(seq)
        elif seq in self.waiting:
            self.waiting.remove(seq)
        self.kv_cache_manager.free_if_allocated(seq)

    def _finish(self, seq: Sequence, reason: SequenceFinishReason) -> None:
        seq.finish(reason)
        self.free_seq(seq)
        self.finished_seqs.append(seq)

    def pop_finished(self) -> list[Sequence]:
        done, self.finished_seqs = self.finished_seqs, []
        return done

    def has_unfinished(self) -> bool:
        return bool(self.waiting or self.running)

    # ------------------------------------------------------------------ steps

    def _preempt(self, seq: Sequence, preempted: list[Sequence]) -> None:
        seq.reset_for_recompute()
        self.running.remove(seq)
        preempted.append(seq)
        self.kv_cache_manager.free_if_allocated(seq)

    def schedule(self) -> SchedulerOutput:
        kv = self.kv_cache_manager
        out = SchedulerOutput([], {}, {}, {}, [])
        budget = self.max_num_batched_tokens

        def take(seq: Sequence, n: int) -> None:
            out.scheduled_sequences.append(seq)
            out.num_scheduled_tokens[seq.seq_id] = n
            out.block_tables[seq.seq_id] = list(kv.get_block_table(seq))
            out.slot_mappings[seq.seq_id] = kv.get_slot_mapping(seq, n)

        for seq in list(self.running):
            if seq.status != SequenceState.RUNNING:
                continue  # preempted earlier in this loop
            n = seq.num_tokens_to_compute
            if n > budget or len(out.scheduled_sequences) >= self.max_num_seqs:
                break
            while not kv.can_allocate(seq, n):
                victim = self.running[-1]
                if victim is seq or len(self.running) <= 1:
                    self._preempt(seq, out.preempted_seqs)
                    break
                self._preempt(victim, out.preempted_seqs)
            else:
                kv.allocate_slots(seq, n)
                take(seq, n)
                budget -= n
        for seq in reversed(out.preempted_seqs):
            self.waiting.appendleft(seq)

        while self.waiting and len(out.scheduled_sequences) < self.max_num_seqs:
            seq = self.waiting[0]
            n = seq.num_tokens_to_compute
            if self._too_long(seq, n):
                self._finish(seq, SequenceFinishReason.LENGTH)
                continue
            hits = kv.get_computed_blocks(seq)
            n -= len(hits) * kv.block_size
            if n > budget or not kv.can_allocate(seq, n, hits):
                break
            kv.allocate_slots(seq, n, hits)
            seq.advance_computed(len(hits) * kv.block_size)
            self.admit_seq(seq)
            take(seq, n)
            budget -= n
        return out

    def update_from_output(self, scheduler_output: SchedulerOutput, model_output: dict[int, int]) -> None:
        for seq in scheduler_output.scheduled_sequences:
            seq.advance_computed(scheduler_output.num_scheduled_tokens[seq.seq_id])
            token = model_output.get(seq.seq_id)
            if token is None:
                continue
            if token in seq.sampling_params.stop_tokens:
                self._finish(seq, SequenceFinishReason.STOP)
                continue
            seq.append_token(token)
            if seq.generated_token_len >= seq.sampling_params.max_tokens:
                self._finish(seq, SequenceFinishReason.LENGTH)
