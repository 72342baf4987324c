"""Offline generation front end (babyvllm/llm.py:11-110) on token ids.

There is no network for tokenizers or checkpoints, so ``LLM`` takes a
``ModelConfig`` (e.g. ``babyvllm.config.qwen2_5_7b()``) and builds that
architecture with seeded random weights; ``generate`` takes prompts as lists
of token ids and returns one ``RequestOutput`` per prompt, in prompt order.
Greedy decoding (temperature 0) is the default, as in the reference.
"""

from __future__ import annotations

import copy

from babyvllm.config import CacheConfig, SchedulerConfig
from babyvllm.engine import LLMEngine
from babyvllm.sequence import SamplingParams
from babyvllm.worker.model_runner import ModelRunner


class LLM:
    def __init__(self, model_config, cache_config: CacheConfig | None = None,
                 scheduler_config: SchedulerConfig | None = None, device=None,
                 use_cuda_graphs: bool | None = None, seed: int = 0, eos_token_ids: set[int] | None = None,
                 init_std: float = 0.02):
        self.cache_config = cache_config or CacheConfig()
        self.scheduler_config = scheduler_config or SchedulerConfig()
        self.model_config = model_config
        self.eos_token_id = set(eos_token_ids or ())
        self.model_runner = ModelRunner(model_config, cache_config=self.cache_config,
                                        scheduler_config=self.scheduler_config, device=device,
                                        use_cuda_graphs=use_cuda_graphs, seed=seed, init_std=init_std)
        self.engine = LLMEngine(self.model_runner,
                                max_num_batched_tokens=self.scheduler_config.max_num_batched_tokens,
                                max_num_seqs=self.scheduler_config.max_num_seqs,
                                enable_prefix_caching=self.cache_config.enable_prefix_caching)

    def generate(self, prompts: list[list[int]], sampling_params: SamplingParams | None = None):
        params = sampling_params or SamplingParams(temperature=0.0)
        ids = []
        for prompt in prompts:
            p = copy.copy(params)
            if not p.ignore_eos:
                p.stop_tokens = set(p.stop_tokens) | self.eos_token_id
            ids.append(self.engine.add_request(list(prompt), p))
        done = self.engine.run()
        return [done[i] for i in ids]
