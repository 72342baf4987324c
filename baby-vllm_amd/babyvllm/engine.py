"""The serving loop: schedule a step, run it on the model, feed the sampled tokens back.

Public surface of the reference's LLMEngine (babyvllm/engine.py:24-174):
``LLMEngine(model_runner, max_num_batched_tokens, max_num_seqs,
enable_prefix_caching)`` sizes the KV-cache manager from
``model_runner.allocate_kv_cache()`` and owns the scheduler; ``add_request``
returns a request id; ``step()`` returns one ``RequestOutput`` for every
request that received a token or finished in that step (a stop token is not
reported as a new token); ``run()`` steps until every request is done and
returns the accumulated output per request id; a step that can neither
schedule, preempt nor finish anything is an error.

Design of this build: ``step`` is three stages — ``_schedule_step`` (with the
progress check), ``_execute`` (the model call and the scheduler update) and
``_report`` (outputs for sampled and finished requests) — and ``run`` merges
step outputs with ``RequestOutput.merge``.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from babyvllm.kv_cache_manager import KVCacheManager
from babyvllm.scheduler import Scheduler, SchedulerOutput
from babyvllm.sequence import SamplingParams, Sequence, SequenceFinishReason


@dataclass
class RequestOutput:
    seq_id: int
    new_token_ids: list[int] = field(default_factory=list)
    finish_reason: SequenceFinishReason | None = None
    text: str = ""

    @property
    def finished(self) -> bool:
        return self.finish_reason is not None

    def merge(self, later: "RequestOutput") -> None:
        self.new_token_ids.extend(later.new_token_ids)
        if later.finished:
            self.finish_reason = later.finish_reason


class LLMEngine:
    def __init__(self, model_runner, max_num_batched_tokens: int = 8, max_num_seqs: int = 4,
                 enable_prefix_caching: bool = False):
        self.model_runner = model_runner
        self.block_size = model_runner.block_size
        self.kv_cache_manager = KVCacheManager(model_runner.allocate_kv_cache(), self.block_size,
                                               enable_prefix_caching=enable_prefix_caching)
        self.scheduler = Scheduler(self.kv_cache_manager, max_num_batched_tokens=max_num_batched_tokens,
                                   max_num_seqs=max_num_seqs)
        self.sequences: dict[int, Sequence] = {}

    # --------------------------------------------------------- requests

    def add_request(self, token_ids: list[int], sampling_params: SamplingParams | None = None) -> int:
        seq = Sequence(token_ids, sampling_params)
        self.sequences[seq.seq_id] = seq
        self.scheduler.add_seq(seq)
        return seq.seq_id

    def abort_request(self, seq_id: int) -> None:
        seq = self.sequences.get(seq_id)
        if seq is not None and not seq.is_finished:
            self.scheduler.abort_seq(seq)

    def has_unfinished_requests(self) -> bool:
        return self.scheduler.has_unfinished()

    # ------------------------------------------------------------- steps

    def _schedule_step(self) -> SchedulerOutput:
        out = self.scheduler.schedule()
        if not (out.scheduled_sequences or out.preempted_seqs or self.scheduler.finished_seqs):
            raise RuntimeError(
                f"no progress: {len(self.scheduler.waiting)} waiting and {len(self.scheduler.running)} running "
                f"requests, but the step scheduled, preempted and finished nothing")
        return out

    def _execute(self, out: SchedulerOutput) -> dict[int, int]:
        sampled = self.model_runner.execute_model(out)
        if not isinstance(sampled, dict):
            raise RuntimeError(f"the model runner returned {type(sampled).__name__}, expected {{seq_id: token}}")
        self.scheduler.update_from_output(out, sampled)
        return sampled

    def _report(self, out: SchedulerOutput | None, sampled: dict[int, int]) -> list[RequestOutput]:
        outputs: dict[int, RequestOutput] = {}
        if out is not None:
            for seq in out.scheduled_sequences:
                if seq.seq_id in sampled:
                    tok = sampled[seq.seq_id]
                    emitted = [] if tok in seq.sampling_params.stop_tokens else [tok]
                    outputs[seq.seq_id] = RequestOutput(seq.seq_id, emitted, seq.finish_reason)
        for seq in self.scheduler.pop_finished():
            outputs.setdefault(seq.seq_id, RequestOutput(seq.seq_id, [], seq.finish_reason))
            self.sequences.pop(seq.seq_id, None)
        return list(outputs.values())

    def step(self) -> list[RequestOutput]:
        out, sampled = None, {}
        if self.has_unfinished_requests():
            out = self._schedule_step()
            if out.scheduled_sequences:
                sampled = self._execute(out)
        return self._report(out, sampled)

    def run(self, max_steps: int = 100_000) -> dict[int, RequestOutput]:
        """Steps until every request is done (also reporting requests that finished on arrival)."""
        merged: dict[int, RequestOutput] = {}
        for _ in range(max_steps):
            if not (self.has_unfinished_requests() or self.scheduler.finished_seqs):
                return merged
            for o in self.step():
                merged.setdefault(o.seq_id, RequestOutput(o.seq_id)).merge(o)
        raise RuntimeError(f"requests still unfinished after {max_steps} steps")

    def reset(self) -> None:
        self.scheduler.waiting.clear()
        self.scheduler.running.clear()
        self.scheduler.finished_seqs.clear()
        self.kv_cache_manager.reset()
        self.sequences.clear()
