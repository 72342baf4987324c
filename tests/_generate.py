"""Helpers of the end-to-end generation tests: the independent checker
(Hugging Face transformers' Qwen2ForCausalLM in fp32 with our weights),
greedy generation that records the logits row behind every sampled token, and
the teacher-forced comparison against the checker.

The checker is fed our own tokens (teacher forcing), so every generated
position is compared, and one near-tie that rounds differently in bf16 does
not hide the positions after it. Logits are compared within a stated
tolerance, and tokens must be the checker's argmax except at near-ties that
the measured logit difference can decide.
"""

from __future__ import annotations

import torch


def hf_from(runner_model, cfg):
    """transformers' Qwen2ForCausalLM (fp32, on the GPU) loaded with our model's weights."""
    from transformers import Qwen2Config, Qwen2ForCausalLM
    # Built on the GPU (its own random init is overwritten below): building a
    # 7B-size fp32 model on the CPU first takes minutes.
    with torch.device("cuda"):
        hf = Qwen2ForCausalLM(Qwen2Config(
            vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
            num_hidden_layers=cfg.num_hidden_layers, num_attention_heads=cfg.num_attention_heads,
            num_key_value_heads=cfg.num_key_value_heads, rms_norm_eps=cfg.rms_norm_eps,
            max_position_embeddings=cfg.max_position_embeddings, rope_theta=cfg.rope_theta,
            tie_word_embeddings=False)).float().eval()
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
    del ours, sd
    return hf


def greedy(n):
    from babyvllm.sequence import SamplingParams
    return SamplingParams(temperature=0.0, max_tokens=n, ignore_eos=True)


def generate_recording(llm, prompts, new_tokens):
    """Greedy tokens per prompt, and the logits rows (fp32 copies) they were sampled from."""
    rows = {}

    def observe(seqs, logits):
        for s, row in zip(seqs, logits.float().cpu()):
            rows.setdefault(s.seq_id, []).append(row)

    llm.model_runner.logits_observer = observe
    ids = [llm.engine.add_request(list(p), greedy(new_tokens)) for p in prompts]
    done = llm.engine.run()
    llm.model_runner.logits_observer = None
    return [done[i].new_token_ids for i in ids], [torch.stack(rows[i]) for i in ids]


@torch.no_grad()
def checker_logits(hf, prompt, tokens):
    """The checker's fp32 logits at every generated position, teacher-forced on `tokens`."""
    ids = torch.tensor([list(prompt) + list(tokens[:-1])], device="cuda")
    return hf(ids).logits[0, len(prompt) - 1:].float().cpu()


def clear_prefix(want_logits, tol):
    """Number of leading positions whose checker top-2 margin exceeds 2 · tol."""
    top = torch.topk(want_logits, 2, dim=-1).values
    low = ((top[:, 0] - top[:, 1]) <= 2 * tol).nonzero()
    return int(low[0]) if len(low) else want_logits.shape[0]


def compare_with_checker(tokens, our_logits, want_logits, max_tol, mean_tol):
    """Logits and tokens against the checker, position by position.

    Every position's logits row must be within max_tol (max-abs) and mean_tol
    (mean-abs) of the checker's. Our token (the argmax of our row) may differ
    from the checker's argmax only where the checker's margin between the two
    is at most twice that position's max-abs logit difference, i.e. where the
    measured rounding difference can decide it. Returns (exact, total, worst
    max-abs, worst mean-abs): `exact` counts positions whose token is the
    checker's argmax.
    """
    exact = total = 0
    worst_max = worst_mean = 0.0
    for toks, ours, want in zip(tokens, our_logits, want_logits):
        assert ours.shape == want.shape, (ours.shape, want.shape)
        diff = (ours - want).abs()
        row_max, row_mean = diff.max(dim=-1).values, diff.mean(dim=-1)
        worst_max = max(worst_max, row_max.max().item())
        worst_mean = max(worst_mean, row_mean.max().item())
        assert row_max.max().item() <= max_tol, f"logits differ by {row_max.max().item():.4f} > {max_tol}"
        assert row_mean.max().item() <= mean_tol, f"mean logit diff {row_mean.max().item():.4f} > {mean_tol}"
        best = want.argmax(dim=-1)
        for pos, tok in enumerate(toks):
            total += 1
            assert tok == int(ours[pos].argmax()), "sampled token is not the argmax of its logits"
            if tok == int(best[pos]):
                exact += 1
            else:
                gap = float(want[pos, best[pos]] - want[pos, tok])
                assert gap <= 2 * float(row_max[pos]), (pos, tok, int(best[pos]), gap, float(row_max[pos]))
    return exact, total, worst_max, worst_mean


@torch.no_grad()
def bf16_cpu_checker_logits(hf_fp32, prompts, tokens):
    """A second, bf16 checker: the same transformers model cast to bf16 and run
    on the host CPU (oneDNN bf16 GEMMs with fp32 accumulation; bf16 activations,
    residual and logits, as the reference's design), teacher-forced on `tokens`.
    Its disagreement with the fp32 checker is the precision floor of bf16
    arithmetic on the model. The rotary frequencies stay fp32, as both
    implementations compute them. Moves the model to the CPU."""
    inv = hf_fp32.model.rotary_emb.inv_freq.detach().clone().cpu()
    hf = hf_fp32.to(torch.bfloat16).to("cpu")
    hf.model.rotary_emb.inv_freq = inv
    out = []
    for p, t in zip(prompts, tokens):
        ids = torch.tensor([list(p) + list(t[:-1])])
        out.append(hf(ids).logits[0, len(p) - 1:].float())
    return out


def argmax_agreement(a_logits, b_logits):
    """Positions where the two logits rows have the same argmax, and the total."""
    same = sum(int((a.argmax(-1) == b.argmax(-1)).sum()) for a, b in zip(a_logits, b_logits))
    return same, sum(a.shape[0] for a in a_logits)


def compare_runs(tokens_a, logits_a, tokens_b, logits_b, max_tol):
    """Two greedy runs of our engine on the same prompts (different launch
    choices). Up to and including the first position where their tokens
    differ, both runs saw the same inputs: there each pair of logits rows must
    agree within max_tol (max-abs), and at that first differing position each
    run's token must lead the other's by at most twice the rows' measured
    difference (a near-tie). Returns (positions compared, worst max-abs,
    prompts that diverged)."""
    compared, worst, diverged = 0, 0.0, 0
    for ta, la, tb, lb in zip(tokens_a, logits_a, tokens_b, logits_b):
        n = next((i for i, (x, y) in enumerate(zip(ta, tb)) if x != y), len(ta))
        for pos in range(min(n + 1, len(ta))):
            d = float((la[pos] - lb[pos]).abs().max())
            worst = max(worst, d)
            compared += 1
            assert d <= max_tol, (pos, d)
        if n < len(ta):
            diverged += 1
            d = float((la[n] - lb[n]).abs().max())
            lead_a = float(la[n][ta[n]] - la[n][tb[n]])
            lead_b = float(lb[n][tb[n]] - lb[n][ta[n]])
            assert 0 <= lead_a <= 2 * d and 0 <= lead_b <= 2 * d, (n, lead_a, lead_b, d)
    return compared, worst, diverged
