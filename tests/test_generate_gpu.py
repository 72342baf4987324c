"""End-to-end greedy generation through LLM.generate on the HIP kernels at a
small shape (2 layers, hidden 256, 4 / 2 heads of 64, vocabulary 512): the
model runner (eager prefill and mixed steps, hipGraph decode steps), the
KV-cache manager with prefix caching, the scheduler and preemption.

Checker: Hugging Face transformers' Qwen2ForCausalLM (an independent
implementation of the architecture) in fp32 on the GPU with the same random
weights, teacher-forced on our tokens (tests/_generate.py): every logits row
within the stated max-abs and mean-abs tolerances, every token the checker's
argmax except at near-ties the measured logit difference can decide. Runs
that differ only in how a step is executed (graph vs eager, prefix caching on vs off, a pool small enough to preempt)
must give identical tokens for every prompt up to its first near-tie.
"""

import pytest
import torch

from tests import _generate as G

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU"),
]

# Stated tolerances on each position's logits row (bf16 model vs fp32 checker;
# logits ~ N(0, 1.6^2) at this init, mean |logit| about 1.3): max-abs 0.2 and
# mean-abs 0.06 (measured 0.12-0.13 and 0.03-0.045 over runs whose decode
# arithmetic differed in rounding); LOGIT_TOL is the near-tie threshold of the
# run-vs-run comparisons.
LOGIT_MAX_TOL = 0.2
LOGIT_MEAN_TOL = 0.06
LOGIT_TOL = 0.05
NEW_TOKENS = 12


def _config():
    from babyvllm.config import ModelConfig
    return ModelConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, rms_norm_eps=1e-6,
                       max_position_embeddings=4096, rope_theta=10000.0, tie_word_embeddings=False)


def _prompts():
    g = torch.Generator().manual_seed(5)
    shared = torch.randint(0, 512, (40,), generator=g).tolist()
    out = []
    for i, n in enumerate([5, 17, 33, 70, 3, 16]):
        tail = torch.randint(0, 512, (n,), generator=g).tolist()
        out.append(shared + tail if i % 2 else tail)
    return out


def _llm(graphs=True, caching=False, blocks=256, max_seqs=8):
    from babyvllm.config import CacheConfig, SchedulerConfig
    from babyvllm.llm import LLM
    return LLM(_config(), cache_config=CacheConfig(num_gpu_blocks=blocks, enable_prefix_caching=caching),
               scheduler_config=SchedulerConfig(max_num_seqs=max_seqs, max_num_batched_tokens=512),
               use_cuda_graphs=graphs, seed=3, init_std=0.1)


@pytest.fixture(scope="module")
def base_run():
    llm = _llm(graphs=True)
    prompts = _prompts()
    toks, logits = G.generate_recording(llm, prompts, NEW_TOKENS)
    assert llm.model_runner.graph_replays > 0
    hf = G.hf_from(llm.model_runner.model, llm.model_config)
    checks = [G.checker_logits(hf, p, t) for p, t in zip(prompts, toks)]
    return prompts, toks, logits, checks


def test_greedy_tokens_match_an_independent_qwen2_implementation(base_run):
    prompts, toks, logits, checks = base_run
    assert all(len(t) == NEW_TOKENS for t in toks)
    exact, total, worst_max, worst_mean = G.compare_with_checker(toks, logits, checks, LOGIT_MAX_TOL,
                                                                 LOGIT_MEAN_TOL)
    print(f"small model: {exact}/{total} tokens equal the checker's argmax; worst logit diff "
          f"max-abs {worst_max:.4f}, mean-abs {worst_mean:.4f}")
    assert exact >= 0.9 * total, (exact, total)


@pytest.mark.parametrize("graphs,caching,blocks", [
    (False, False, 256), (True, True, 256), (False, True, 256), (True, False, 14), (True, True, 14)])
def test_runs_agree_up_to_the_first_near_tie(base_run, graphs, caching, blocks):
    """Eager vs graph decode, prefix caching on vs off, and a 14-page pool that
    forces preemption by recompute all give the base run's tokens."""
    prompts, toks, _, checks = base_run
    llm = _llm(graphs=graphs, caching=caching, blocks=blocks)
    other, _ = G.generate_recording(llm, prompts, NEW_TOKENS)
    assert (llm.model_runner.graph_replays > 0) == graphs
    if caching:
        assert llm.engine.kv_cache_manager.num_hit_tokens > 0
    for p, a, b, want in zip(prompts, toks, other, checks):
        clear = G.clear_prefix(want, LOGIT_TOL)
        assert len(b) == NEW_TOKENS
        assert a[:clear] == b[:clear], (len(p), clear, a, b)
