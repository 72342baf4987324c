"""End-to-end greedy generation through LLM.generate on the HIP kernels
(BASELINE config 5's path at a small shape): the model runner (eager prefill
and mixed steps, hipGraph decode steps), the KV-cache manager with prefix
caching and the scheduler.

Checker: Hugging Face transformers' Qwen2ForCausalLM (an independent
implementation of the architecture) in fp32 on the GPU, loaded with the same
random weights, decoding greedily by full recomputation. Our model runs in
bf16, so tokens are compared while the checker's top-2 logit margin exceeds
MARGIN (a near-tie can flip under bf16 rounding, and every later token depends
on it); the test requires most tokens to be compared.
"""

import pytest
import torch

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU"),
]

MARGIN = 0.05
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


def _llm(graphs=True, caching=False, max_seqs=8):
    from babyvllm.config import CacheConfig, SchedulerConfig
    from babyvllm.llm import LLM
    return LLM(_config(), cache_config=CacheConfig(num_gpu_blocks=256, enable_prefix_caching=caching),
               scheduler_config=SchedulerConfig(max_num_seqs=max_seqs, max_num_batched_tokens=512),
               use_cuda_graphs=graphs, seed=3, init_std=0.1)


def _hf_from(runner_model, cfg):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    hf = Qwen2ForCausalLM(Qwen2Config(
        vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
        num_hidden_layers=cfg.num_hidden_layers, num_attention_heads=cfg.num_attention_heads,
        num_key_value_heads=cfg.num_key_value_heads, rms_norm_eps=cfg.rms_norm_eps,
        max_position_embeddings=cfg.max_position_embeddings, rope_theta=cfg.rope_theta,
        tie_word_embeddings=False)).float().cuda().eval()
    ours = {k: v.float() for k, v in runner_model.state_dict().items()}
    q, kv = cfg.num_attention_heads * cfg.head_dim, cfg.num_key_value_heads * cfg.head_dim
    sd = {"model.embed_tokens.weight": ours["model.embed_tokens.weight"],
          "model.norm.weight": ours["model.norm.weight"], "lm_head.weight": ours["lm_head.weight"]}
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        w, b = ours[p + "self_attn.qkv_proj.weight"], ours[p + "self_attn.qkv_proj.bias"]
        for name, lo, hi in (("q", 0, q), ("k", q, q + kv), ("v", q + kv, q + 2 * kv)):
            sd[p + f"self_attn.{name}_proj.weight"] = w[lo:hi]
            sd[p + f"self_attn.{name}_proj.bias"] = b[lo:hi]
        sd[p + "self_attn.o_proj.weight"] = ours[p + "self_attn.o_proj.weight"]
        gu = ours[p + "mlp.gate_up_proj.weight"]
        sd[p + "mlp.gate_proj.weight"] = gu[: cfg.intermediate_size]
        sd[p + "mlp.up_proj.weight"] = gu[cfg.intermediate_size:]
        sd[p + "mlp.down_proj.weight"] = ours[p + "mlp.down_proj.weight"]
        sd[p + "input_layernorm.weight"] = ours[p + "input_layernorm.weight"]
        sd[p + "post_attention_layernorm.weight"] = ours[p + "post_attention_layernorm.weight"]
    missing, unexpected = hf.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    return hf


@torch.no_grad()
def _checker_tokens(hf, prompt, n):
    """Greedy tokens and the top-2 margin at each step, by full recomputation in fp32."""
    ids, toks, margins = list(prompt), [], []
    for _ in range(n):
        logits = hf(torch.tensor([ids], device="cuda")).logits[0, -1].float()
        top = torch.topk(logits, 2)
        toks.append(int(top.indices[0]))
        margins.append(float(top.values[0] - top.values[1]))
        ids.append(toks[-1])
    return toks, margins


def _compare(outputs, prompts, hf):
    compared = total = 0
    for out, prompt in zip(outputs, prompts):
        want, margins = _checker_tokens(hf, prompt, NEW_TOKENS)
        assert len(out.new_token_ids) == NEW_TOKENS
        for got, exp, m in zip(out.new_token_ids, want, margins):
            total += 1
            if m < MARGIN:
                break
            assert got == exp, (prompt[:4], out.new_token_ids, want, margins)
            compared += 1
    return compared, total


def _generate(llm, prompts):
    from babyvllm.sequence import SamplingParams
    return llm.generate(prompts, SamplingParams(temperature=0.0, max_tokens=NEW_TOKENS, ignore_eos=True))


def test_greedy_tokens_match_an_independent_qwen2_implementation():
    llm = _llm(graphs=True)
    prompts = _prompts()
    outs = _generate(llm, prompts)
    hf = _hf_from(llm.model_runner.model, llm.model_config)
    compared, total = _compare(outs, prompts, hf)
    assert compared >= total * 0.6, (compared, total)
    # The decode steps ran on captured graphs.
    assert llm.model_runner._graphs


@pytest.mark.parametrize("graphs,caching", [(False, False), (True, True)])
def test_eager_and_prefix_cached_runs_give_the_same_tokens(graphs, caching):
    prompts = _prompts()
    base = _generate(_llm(graphs=True), prompts)
    other_llm = _llm(graphs=graphs, caching=caching)
    other = _generate(other_llm, prompts)
    hf = _hf_from(other_llm.model_runner.model, other_llm.model_config)
    compared, total = _compare(other, prompts, hf)
    assert compared >= total * 0.6
    same = sum(a.new_token_ids == b.new_token_ids for a, b in zip(base, other))
    assert same >= len(prompts) - 1
    if caching:
        assert other_llm.engine.kv_cache_manager.num_hit_tokens > 0


def test_preemption_under_a_small_pool_keeps_tokens():
    from babyvllm.config import CacheConfig, SchedulerConfig
    from babyvllm.llm import LLM
    prompts = _prompts()
    roomy = _generate(_llm(graphs=True), prompts)
    tight = LLM(_config(), cache_config=CacheConfig(num_gpu_blocks=14),
                scheduler_config=SchedulerConfig(max_num_seqs=8, max_num_batched_tokens=512),
                use_cuda_graphs=True, seed=3, init_std=0.1)
    outs = _generate(tight, prompts)
    same = sum(a.new_token_ids == b.new_token_ids for a, b in zip(roomy, outs))
    assert same >= len(prompts) - 1
