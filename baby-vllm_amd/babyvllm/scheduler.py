"""Continuous batching: which requests run in the next step, and how many tokens each computes.

Behaviour of the reference's Scheduler (babyvllm/scheduler.py:13-158), which
its tests pin: running requests go first, in order, each computing all its
uncached tokens (one token in steady decode, a whole prompt after a
recompute); when the pool cannot hold one of them, requests are preempted by
recompute from the back of the running list (their pages are released and
they wait again, ahead of newer requests), the request itself last. Then
waiting requests are admitted in arrival order, each with its whole prompt
minus the prefix-cache hits, while the step's token budget, its seat count
and the pool allow. A request whose prompt exceeds the token budget or the
whole pool finishes with reason LENGTH. The output carries each scheduled
request's block table and slot mapping, the inputs of the paged-KV kernels.

Design of this build: a step is assembled in a ``_StepBatch`` (budget, seats
and the per-request outputs in one place), and the two phases are separate
methods, ``_continue_running`` and ``_admit_waiting``; preemption is one
method that picks its victim and re-queues it.
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


class _StepBatch:
    """One step's batch while it is being assembled."""

    def __init__(self, kv: KVCacheManager, token_budget: int, seats: int):
        self.kv = kv
        self.tokens_left = token_budget
        self.seats_left = seats
        self.out = SchedulerOutput([], {}, {}, {}, [])

    def has_seat(self) -> bool:
        return self.seats_left > 0

    def fits(self, n_tokens: int) -> bool:
        return self.seats_left > 0 and n_tokens <= self.tokens_left

    def add(self, seq: Sequence, n_tokens: int) -> None:
        """Records a request whose pages for ``n_tokens`` more tokens are allocated."""
        o = self.out
        o.scheduled_sequences.append(seq)
        o.num_scheduled_tokens[seq.seq_id] = n_tokens
        o.block_tables[seq.seq_id] = list(self.kv.get_block_table(seq))
        o.slot_mappings[seq.seq_id] = self.kv.get_slot_mapping(seq, n_tokens)
        self.tokens_left -= n_tokens
        self.seats_left -= 1


class Scheduler:
    def __init__(self, kv_cache_manager: KVCacheManager, max_num_batched_tokens: int = 2048,
                 max_num_seqs: int = 256):
        self.kv_cache_manager = kv_cache_manager
        self.max_num_batched_tokens = max_num_batched_tokens
        self.max_num_seqs = max_num_seqs
        self.waiting: deque[Sequence] = deque()
        self.running: list[Sequence] = []
        self.finished_seqs: list[Sequence] = []

    # --------------------------------------------------------- requests

    def _never_fits(self, seq: Sequence, n_tokens: int) -> bool:
        kv = self.kv_cache_manager
        return n_tokens > self.max_num_batched_tokens or kv.num_blocks_needed(seq, n_tokens) > kv.num_blocks

    def add_seq(self, seq: Sequence) -> None:
        if self._never_fits(seq, len(seq)):
            self._retire(seq, SequenceFinishReason.LENGTH)
        else:
            seq.status = SequenceState.WAITING
            self.waiting.append(seq)

    def abort_seq(self, seq: Sequence) -> None:
        self._retire(seq, SequenceFinishReason.ABORT)

    def free_seq(self, seq: Sequence) -> None:
        """Drops a request from the queues and releases its pages."""
        if seq in self.running:
            self.running.remove(seq)
        elif seq in self.waiting:
            self.waiting.remove(seq)
        self.kv_cache_manager.free_if_allocated(seq)

    def _retire(self, seq: Sequence, reason: SequenceFinishReason) -> None:
        seq.finish(reason)
        self.free_seq(seq)
        self.finished_seqs.append(seq)

    def pop_finished(self) -> list[Sequence]:
        done = self.finished_seqs
        self.finished_seqs = []
        return done

    def has_unfinished(self) -> bool:
        return len(self.waiting) > 0 or len(self.running) > 0

    # ------------------------------------------------------------- steps

    def schedule(self) -> SchedulerOutput:
        batch = _StepBatch(self.kv_cache_manager, self.max_num_batched_tokens, self.max_num_seqs)
        self._continue_running(batch)
        self._admit_waiting(batch)
        return batch.out

    def _preempt_for(self, seq: Sequence, batch: _StepBatch) -> Sequence:
        """Preempts the newest running request, or ``seq`` itself when it is that one or alone; returns it."""
        victim = self.running[-1]
        if victim is seq or len(self.running) == 1:
            victim = seq
        victim.reset_for_recompute()
        self.running.remove(victim)
        self.kv_cache_manager.free_if_allocated(victim)
        batch.out.preempted_seqs.append(victim)
        return victim

    def _continue_running(self, batch: _StepBatch) -> None:
        kv = self.kv_cache_manager
        for seq in list(self.running):
            if seq.status is not SequenceState.RUNNING:
                continue  # preempted for an earlier request of this pass
            n = seq.num_tokens_to_compute
            if not batch.fits(n):
                break
            preempted_self = False
            while not kv.can_allocate(seq, n):
                if self._preempt_for(seq, batch) is seq:
                    preempted_self = True
                    break
            if not preempted_self:
                kv.allocate_slots(seq, n)
                batch.add(seq, n)
        # Preempted requests wait ahead of newer ones, in the order they were preempted.
        self.waiting.extendleft(reversed(batch.out.preempted_seqs))

    def _admit_waiting(self, batch: _StepBatch) -> None:
        kv = self.kv_cache_manager
        while self.waiting and batch.has_seat():
            seq = self.waiting[0]
            if self._never_fits(seq, seq.num_tokens_to_compute):
                self._retire(seq, SequenceFinishReason.LENGTH)
                continue
            hits = kv.get_computed_blocks(seq)
            n = seq.num_tokens_to_compute - len(hits) * kv.block_size
            if not batch.fits(n) or not kv.can_allocate(seq, n, hits):
                break
            kv.allocate_slots(seq, n, hits)
            seq.advance_computed(len(hits) * kv.block_size)
            self.waiting.popleft()
            seq.status = SequenceState.RUNNING
            self.running.append(seq)
            batch.add(seq, n)

    def update_from_output(self, scheduler_output: SchedulerOutput, model_output: dict[int, int]) -> None:
        """Advances every scheduled request and appends its sampled token (a stop token finishes it)."""
        for seq in scheduler_output.scheduled_sequences:
            seq.advance_computed(scheduler_output.num_scheduled_tokens[seq.seq_id])
            if seq.seq_id not in model_output:
                continue
            token = model_output[seq.seq_id]
            if token in seq.sampling_params.stop_tokens:
                self._retire(seq, SequenceFinishReason.STOP)
                continue
            seq.append_token(token)
            if seq.generated_token_len >= seq.sampling_params.max_tokens:
                self._retire(seq, SequenceFinishReason.LENGTH)
