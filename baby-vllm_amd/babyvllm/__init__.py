"""babyvllm (MI355X build): the paged-KV hot path of baby-vLLM on hand-written gfx950 HIP kernels.

Importable names mirror the reference package's kernel layer:
``babyvllm.kernels.rope.fused_rope_and_cache``,
``babyvllm.kernels.paged_attn.paged_decode_attention``,
``babyvllm.kernels.paged_prefill.paged_prefill_attention`` and
``babyvllm.kernels.decode_split`` (pure Python), plus the boundary types
``babyvllm.worker.context.AttentionMetadata`` and the dispatching
``babyvllm.layers.attention.Attention`` module.
"""
