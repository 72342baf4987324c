"""One request: its token ids, how far its K/V is cached, and its lifecycle.

Public surface of the reference's Sequence (babyvllm/sequence.py:6-95), which
the scheduler, the engine and the tests address: ``Sequence(token_ids,
sampling_params)``, ``seq_id`` (from the class-level ``_counter``),
``token_ids`` (prompt then generated tokens), ``num_computed_tokens`` (tokens
whose K/V sit in the cache), ``num_preemptions`` (bumped by every recompute, so
(seq_id, num_preemptions) names one lifetime of a block table), ``status``,
``finish_reason``, the prompt / output views and the transitions below.

Design of this build: the lifecycle is a small state machine whose transitions
check their preconditions (a finished request cannot be re-queued, computed
tokens never pass the known tokens), and the prefix-cache identity of each full
page (a chained content digest, filled lazily by the KV-cache manager) lives on
the sequence as ``page_digests``, so it is computed once per page however many
times the request is scheduled.
"""

from __future__ import annotations

import itertools
from dataclasses import dataclass, field
from enum import Enum, auto


@dataclass
class SamplingParams:
    temperature: float = 1.0
    top_p: float = 1.0
    ignore_eos: bool = False
    max_tokens: int = 256
    stop_tokens: set[int] = field(default_factory=set)


class SequenceState(Enum):
    WAITING = auto()
    RUNNING = auto()
    DONE = auto()


class SequenceFinishReason(str, Enum):
    STOP = "stop"
    LENGTH = "length"
    ABORT = "abort"


class Sequence:
    _counter = itertools.count()

    __slots__ = ("seq_id", "token_ids", "sampling_params", "status", "finish_reason", "num_computed_tokens",
                 "num_preemptions", "page_digests", "_n_prompt")

    def __init__(self, token_ids: list[int], sampling_params: SamplingParams | None = None):
        if len(token_ids) == 0:
            raise ValueError("a request needs at least one prompt token")
        self.seq_id: int = next(Sequence._counter)
        self.token_ids: list[int] = list(token_ids)
        self.sampling_params = sampling_params if sampling_params is not None else SamplingParams()
        self.status = SequenceState.WAITING
        self.finish_reason: SequenceFinishReason | None = None
        self.num_computed_tokens = 0
        self.num_preemptions = 0
        self.page_digests: list[bytes] = []
        self._n_prompt = len(self.token_ids)

    # ------------------------------------------------------------ views

    def __len__(self) -> int:
        return len(self.token_ids)

    def __getitem__(self, index):
        return self.token_ids[index]

    def __repr__(self) -> str:
        return (f"Sequence(#{self.seq_id} {self.status.name.lower()}, {self.num_computed_tokens}/{len(self)} "
                f"tokens cached, prompt {self._n_prompt}, preempted {self.num_preemptions}x)")

    @property
    def prompt_len(self) -> int:
        return self._n_prompt

    @property
    def output_token_ids(self) -> list[int]:
        return self.token_ids[self._n_prompt:]

    @property
    def generated_token_len(self) -> int:
        return len(self.token_ids) - self._n_prompt

    @property
    def num_tokens_to_compute(self) -> int:
        return len(self.token_ids) - self.num_computed_tokens

    @property
    def is_finished(self) -> bool:
        return self.status is SequenceState.DONE

    @property
    def last_token_id(self) -> int:
        return self.token_ids[-1]

    # ------------------------------------------------------ transitions

    def append_token(self, token_id: int) -> None:
        self.token_ids.append(token_id)

    def advance_computed(self, n: int) -> None:
        """Marks ``n`` more tokens as cached (raises ValueError past the known tokens)."""
        target = self.num_computed_tokens + n
        if target > len(self.token_ids):
            raise ValueError(f"sequence {self.seq_id}: {target} tokens marked cached but only "
                             f"{len(self.token_ids)} exist")
        self.num_computed_tokens = target

    def finish(self, reason: SequenceFinishReason) -> None:
        self.status = SequenceState.DONE
        self.finish_reason = reason

    def reset_for_recompute(self) -> None:
        """Preemption by recompute: the cached K/V is dropped and the request waits again."""
        if self.status is SequenceState.DONE:
            raise ValueError(f"sequence {self.seq_id} is finished and cannot be recomputed")
        self.status = SequenceState.WAITING
        self.num_computed_tokens = 0
        self.num_preemptions += 1
