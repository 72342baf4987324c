"""CPU oracle for the paged-KV hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in plain torch on the CPU, the reference's own torch
path for the three hot-path operations:

* RoPE + KV-store append: ``apply_rope`` (babyvllm/layers/rotary.py:4-15),
  the ``RotaryEmbedding`` tables (rotary.py:17-32) and ``store_kvcache``
  (babyvllm/layers/attention.py:24-32).
* Paged decode attention: ``gather_kv_batched`` + ``make_decode_mask`` +
  ``_static_decode_attention`` (attention.py:71-134), and the split/LSE merge
  semantics of the flash-decoding reduce (babyvllm/kernels/paged_attn.py:216-251).
* Varlen paged prefill attention: ``_paged_attention_torch`` + ``_causal_sdpa``
  (attention.py:137-196).

* The decode step's other kernels (the next row of the path): greedy argmax,
  residual add + RMSNorm and SiLU·mul (``decode_step.py``; the reference's
  Triton kernel math, babyvllm/kernels/argmax.py, layernorm.py, activation.py).

It also holds independent float64 brute-force restatements used to pin the
torch restatement (see tests/test_oracle.py).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker or as the timed CPU
baseline. The product path (``baby-vllm_amd/babyvllm``) never imports it.

Parity status per function (pins live in tests/test_oracle.py):
  rope_tables, apply_rope, apply_rope_bf16_explicit, store_kvcache,
  gather_kv_batched, make_decode_mask, static_decode_attention,
  paged_attention_torch, causal_sdpa, naive_causal_attention,
  brute_decode, brute_prefill, lse_merge,
  decode_step.greedy_argmax, decode_step.fused_add_rms_norm,
  decode_step.silu_mul                             -- all pinned.
"""
