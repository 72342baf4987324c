"""The step loop: schedule, run the model, feed sampled tokens back (babyvllm/engine.py:24-174).

``LLMEngine(model_runner, max_num_batched_tokens, max_num_seqs,
enable_prefix_caching)`` owns the KV-cache manager (sized by
``model_runner.allocate_kv_cache()``) and the scheduler; ``step()`` returns one
``RequestOutput`` per sequence that got a token or finished, ``run()`` steps
until every request is done and returns the accumulated outputs per seq_id.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from babyvllm.kv_cache_manager import KVCacheManager
from babyvllm.scheduler import Scheduler
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

    def step(self) -> list[RequestOutput]:
        outputs: list[RequestOutput] = []
        reported: set[int] = set()
        if self.has_unfinished_requests():
            sched = self.scheduler.schedule()
            if not (sched.scheduled_sequences or sched.preempted_seqs or self.scheduler.finished_seqs):
                raise RuntimeError("Engine stalled: unfinished requests exist, but scheduler scheduled no "
                                   "work, preempted nothing, and no sequences finished.")
            if sched.scheduled_sequences:
                sampled = self.model_runner.execute_model(sched)
                if not isinstance(sampled, dict):
                    raise RuntimeError("ModelRunner returned incorrect type")
                self.scheduler.update_from_output(sched, sampled)
                for seq in sched.scheduled_sequences:
                    if seq.seq_id in sampled:
                        tok = sampled[seq.seq_id]
                        new = [] if tok in seq.sampling_params.stop_tokens else [tok]
                        outputs.append(RequestOutput(seq.seq_id, new, seq.finish_reason))
                        reported.add(seq.seq_id)
        for seq in self.scheduler.pop_finished():
            if seq.seq_id not in reported:
                outputs.append(RequestOutput(seq.seq_id, [], seq.finish_reason))
            self.sequences.pop(seq.seq_id, None)
        return outputs

    def run(self, max_steps: int = 100_000) -> dict[int, RequestOutput]:
        final: dict[int, RequestOutput] = {}
        steps = 0
        # Also drain sequences that finished when added (prompt too long), so
        # every request gets an output.
        while self.has_unfinished_requests() or self.scheduler.finished_seqs:
            for out in self.step():
                acc = final.setdefault(out.seq_id, RequestOutput(out.seq_id))
                acc.new_token_ids.extend(out.new_token_ids)
                if out.finished:
                    acc.finish_reason = out.finish_reason
            steps += 1
            if steps >= max_steps:
                raise RuntimeError(f"Engine.run() hit max_steps ({max_steps}). Possible livelock.")
        return final

    def reset(self) -> None:
        self.scheduler.waiting.clear()
        self.scheduler.running.clear()
        self.scheduler.finished_seqs.clear()
        self.kv_cache_manager.reset()
        self.sequences.clear()
