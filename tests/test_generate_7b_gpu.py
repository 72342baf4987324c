"""BASELINE config 5 on the HIP path: continuous-batching greedy generate at the
Qwen2.5-7B architecture through LLM.generate's engine.

* The full workload (28 layers, hidden 3584, 28 / 4 heads of 128, vocab
  152,064, random init N(0, 0.02), bf16): 64 prompts of 1920 token ids whose
  first 1536 are shared, 64 new tokens each, prefix caching on, 8192-token
  step budget, 64 sequences at most. Checks: every request gets 64 tokens;
  the prefix cache serves 63 · 1536 = 96,768 prompt tokens (the shared prefix
  of every prompt after the first); the KV pages in use never exceed the
  closed form 96 + 64 · (124 − 96) = 1,888; every logits row of every step is
  finite; the pure decode steps replay captured graphs.
* The same architecture cut to 2 layers (same widths, same vocabulary) against
  an independent implementation: Hugging Face transformers' Qwen2ForCausalLM
  in fp32 with the same weights, teacher-forced on our tokens so that every
  generated position is checked (tests/_generate.py): each position's logits
  row within the stated max-abs and mean-abs tolerances, and our token the
  checker's argmax except at near-ties that the measured logit difference can
  decide (at least 90% of positions exact). Graph vs eager decode and caching
  on vs off must give identical tokens for every prompt up to the first
  position whose checker margin is below 2 · LOGIT_TOL (GEMM shapes differ
  between those runs, so a near-tie may round either way).

* The full 28-layer model against the same checker, teacher-forced on six
  prompts (four on config 5's 1536-token shared prefix) for 16 tokens each:
  logits within stated tolerances at this depth; our tokens the checker's
  argmax except at measured near-ties, and at least as often as an
  independent bf16 implementation of the same design manages (transformers'
  model cast to bf16 on the host CPU); graph vs eager and caching on vs off
  compared logits row by row along each common token prefix.

Reference counterparts: tests/test_decode_graph.py:41-50 (graph tokens ==
eager tokens), tests/test_prefix_caching_e2e.py:33 (same outputs with and
without caching), tests/test_parity_7b.py (7B-shape parity with transformers).
"""

import gc

import pytest
import torch

from tests import _generate as G

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU"),
]

# bf16 activations through 2 layers and bf16 logits (ulp 2^-7 .. 2^-5 at the
# logits' magnitude; logits ~ N(0, 1.2^2), max |logit| about 6) against fp32:
# stated tolerances on each position's logits row (max-abs over the 152,064
# logits, and mean-abs; measured 0.10 and 0.017).
LOGIT_MAX_TOL = 0.15
LOGIT_MEAN_TOL = 0.025
# Near-tie threshold for the graph / eager / caching comparison.
LOGIT_TOL = 0.08
NEW_TOKENS = 16


def _cfg(layers):
    from babyvllm.config import qwen2_5_7b
    cfg = qwen2_5_7b()
    cfg.num_hidden_layers = layers
    return cfg


def _llm(cfg, graphs=True, caching=True, blocks=2048, max_seqs=64, budget=8192):
    from babyvllm.config import CacheConfig, SchedulerConfig
    from babyvllm.llm import LLM
    return LLM(cfg, cache_config=CacheConfig(num_gpu_blocks=blocks, enable_prefix_caching=caching),
               scheduler_config=SchedulerConfig(max_num_seqs=max_seqs, max_num_batched_tokens=budget),
               use_cuda_graphs=graphs, seed=0)


def test_config5_full_workload():
    cfg = _cfg(28)
    g = torch.Generator().manual_seed(0)
    shared = torch.randint(0, cfg.vocab_size, (1536,), generator=g).tolist()
    prompts = [shared + torch.randint(0, cfg.vocab_size, (384,), generator=g).tolist() for _ in range(64)]
    llm = _llm(cfg, blocks=9000)
    runner, engine = llm.model_runner, llm.engine
    bad_rows = []

    def observe(seqs, logits):
        finite = torch.isfinite(logits).all(dim=-1)
        if not bool(finite.all()):
            bad_rows.extend(s.seq_id for s, ok in zip(seqs, finite.tolist()) if not ok)

    runner.logits_observer = observe
    ids = [engine.add_request(p, G.greedy(64)) for p in prompts]
    got, peak, steps = {}, 0, 0
    while engine.has_unfinished_requests():
        for out in engine.step():
            got.setdefault(out.seq_id, []).extend(out.new_token_ids)
        peak = max(peak, engine.kv_cache_manager.num_used_blocks)
        steps += 1
        assert steps < 1000
    assert [len(got[i]) for i in ids] == [64] * 64
    assert engine.kv_cache_manager.num_hit_tokens == 63 * 1536
    assert peak <= 96 + 64 * (-(-(1920 + 64) // 16) - 96) == 1888, peak
    assert not bad_rows, f"non-finite logits for sequences {sorted(set(bad_rows))}"
    assert runner.graph_replays >= 60, runner.graph_replays
    assert engine.kv_cache_manager.num_free_blocks == 9000
    runner.logits_observer = None
    del llm, runner, engine
    gc.collect()
    torch.cuda.empty_cache()


def _prompts(vocab):
    g = torch.Generator().manual_seed(5)
    shared = torch.randint(0, vocab, (160,), generator=g).tolist()
    out = []
    for i, n in enumerate([7, 40, 95, 300, 3, 17]):
        tail = torch.randint(0, vocab, (n,), generator=g).tolist()
        out.append(shared + tail if i % 2 else tail)
    return out


@pytest.fixture(scope="module")
def two_layer_runs():
    cfg = _cfg(2)
    prompts = _prompts(cfg.vocab_size)
    base = _llm(cfg, graphs=True, caching=True, max_seqs=8, budget=1024)
    toks, logits = G.generate_recording(base, prompts, NEW_TOKENS)
    assert base.model_runner.graph_replays > 0
    assert base.engine.kv_cache_manager.num_hit_tokens > 0
    hf = G.hf_from(base.model_runner.model, cfg)
    checks = [G.checker_logits(hf, p, t) for p, t in zip(prompts, toks)]
    del hf, base
    gc.collect()
    torch.cuda.empty_cache()
    return cfg, prompts, toks, logits, checks


def test_7b_width_tokens_and_logits_match_transformers(two_layer_runs):
    cfg, prompts, toks, logits, checks = two_layer_runs
    assert all(len(t) == NEW_TOKENS for t in toks)
    exact, total, worst_max, worst_mean = G.compare_with_checker(toks, logits, checks, LOGIT_MAX_TOL,
                                                                 LOGIT_MEAN_TOL)
    print(f"7B-width 2-layer: {exact}/{total} tokens equal the checker's argmax; worst logit diff "
          f"max-abs {worst_max:.4f}, mean-abs {worst_mean:.4f}")
    assert exact >= 0.9 * total, (exact, total)


@pytest.mark.parametrize("graphs,caching", [(False, True), (True, False), (False, False)])
def test_7b_width_graph_eager_and_caching_agree(two_layer_runs, graphs, caching):
    cfg, prompts, toks, _, checks = two_layer_runs
    other = _llm(cfg, graphs=graphs, caching=caching, max_seqs=8, budget=1024)
    other_toks, _ = G.generate_recording(other, prompts, NEW_TOKENS)
    assert (other.model_runner.graph_replays > 0) == graphs
    for p, a, b, want in zip(prompts, toks, other_toks, checks):
        clear = G.clear_prefix(want, LOGIT_TOL)
        assert a[:clear] == b[:clear], (len(p), clear, a, b)
    del other
    gc.collect()
    torch.cuda.empty_cache()


# ------------------------------------------------ full depth: 28 layers (config 5's model)
#
# At 28 layers bf16 rounding moves logits by up to ~0.4 (mean-abs ~0.06) from
# the fp32 checker, while this random-init model's top-2 logit margins have a
# median of ~0.17, so some greedy tokens follow the rounding. The precision
# floor is measured rather than assumed: transformers' own model cast to bf16
# and run on the host CPU (a second, independent bf16 implementation of the
# same design) against the same fp32 checker. Measured on MI355X: ours 83/96
# tokens equal to the fp32 argmax, max-abs 0.388, mean-abs 0.062; transformers
# bf16 83/96, max-abs 0.398, mean-abs 0.062; ours vs transformers bf16 90/96.

FULL_NEW_TOKENS = 16
FULL_MAX_TOL = 0.6     # stated max-abs logit tolerance at 28 layers (measured 0.39)
FULL_MEAN_TOL = 0.09   # stated mean-abs logit tolerance at 28 layers (measured 0.062)
RUN_MAX_TOL = 0.6      # two bf16 runs of our engine (graph / eager, caching on / off)


def _full_prompts(vocab):
    """Four prompts on config 5's 1536-token shared prefix (tails of 7 to 300
    tokens) and two short distinct ones."""
    g = torch.Generator().manual_seed(0)
    shared = torch.randint(0, vocab, (1536,), generator=g).tolist()
    out = [shared + torch.randint(0, vocab, (n,), generator=g).tolist() for n in (7, 40, 95, 300)]
    out += [torch.randint(0, vocab, (n,), generator=g).tolist() for n in (3, 17)]
    return out


def _full_llm(cfg, graphs=True, caching=True):
    return _llm(cfg, graphs=graphs, caching=caching, max_seqs=8, budget=8192, blocks=1024)


@pytest.fixture(scope="module")
def full_depth_runs():
    cfg = _cfg(28)
    prompts = _full_prompts(cfg.vocab_size)
    base = _full_llm(cfg)
    toks, logits = G.generate_recording(base, prompts, FULL_NEW_TOKENS)
    assert base.model_runner.graph_replays > 0
    assert base.engine.kv_cache_manager.num_hit_tokens == 3 * 1536
    hf = G.hf_from(base.model_runner.model, cfg)
    checks = [G.checker_logits(hf, p, t) for p, t in zip(prompts, toks)]
    del base
    gc.collect()
    torch.cuda.empty_cache()
    bf16_checks = G.bf16_cpu_checker_logits(hf, prompts, toks)
    del hf
    gc.collect()
    torch.cuda.empty_cache()
    return cfg, prompts, toks, logits, checks, bf16_checks


def test_full_depth_tokens_and_logits_against_transformers(full_depth_runs):
    cfg, prompts, toks, logits, checks, bf16_checks = full_depth_runs
    assert all(len(t) == FULL_NEW_TOKENS for t in toks)
    exact, total, worst_max, worst_mean = G.compare_with_checker(toks, logits, checks, FULL_MAX_TOL,
                                                                 FULL_MEAN_TOL)
    floor, _ = G.argmax_agreement(bf16_checks, checks)
    with_bf16, _ = G.argmax_agreement(logits, bf16_checks)
    print(f"28-layer 7B: {exact}/{total} tokens equal the fp32 checker's argmax (transformers bf16: "
          f"{floor}/{total}; ours vs transformers bf16: {with_bf16}/{total}); worst logit diff max-abs "
          f"{worst_max:.4f}, mean-abs {worst_mean:.4f}")
    # At least as many exact tokens as the independent bf16 implementation, up
    # to 3 positions of sampling noise, and never below 80%.
    assert exact >= floor - 3 and exact >= 0.8 * total, (exact, floor, total)
    # Against the bf16 checker, tokens differ only at its measured near-ties too.
    G.compare_with_checker(toks, logits, bf16_checks, FULL_MAX_TOL, FULL_MEAN_TOL)


@pytest.mark.parametrize("graphs,caching", [(False, True), (True, False)])
def test_full_depth_graph_eager_and_caching_agree(full_depth_runs, graphs, caching):
    cfg, prompts, toks, logits, _, _ = full_depth_runs
    other = _full_llm(cfg, graphs=graphs, caching=caching)
    other_toks, other_logits = G.generate_recording(other, prompts, FULL_NEW_TOKENS)
    assert (other.model_runner.graph_replays > 0) == graphs
    compared, worst, diverged = G.compare_runs(toks, logits, other_toks, other_logits, RUN_MAX_TOL)
    print(f"28-layer graphs={graphs} caching={caching}: {compared} positions compared, worst max-abs "
          f"{worst:.4f}, {diverged} of {len(prompts)} prompts diverged at a near-tie")
    assert compared >= len(prompts)
    del other
    gc.collect()
    torch.cuda.empty_cache()
