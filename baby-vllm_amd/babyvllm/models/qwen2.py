"""Qwen2 decoder for the paged-KV path (babyvllm/models/qwen2.py:17-137).

Same module tree and parameter names as the reference (``model.layers[i].
self_attn.qkv_proj`` with bias, ``o_proj``, ``mlp.gate_up_proj``,
``down_proj``, ``input_layernorm``, ``post_attention_layernorm``,
``model.norm``, ``lm_head`` unless embeddings are tied). Per layer a step runs:
add + RMSNorm (HIP), the QKV GEMM (hipBLASLt through torch), fused RoPE + KV
append (HIP, straight into the paged cache through the step's slot_mapping),
paged attention (HIP decode or prefill kernel), the output GEMM, add + RMSNorm,
the gate/up GEMM, SiLU·mul (HIP) and the down GEMM.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from babyvllm.kernels.activation import fused_silu_mul
from babyvllm.kernels.rope import fused_rope_and_cache
from babyvllm.layers.attention import Attention
from babyvllm.layers.layernorm import RMSNorm
from babyvllm.layers.rotary import RotaryEmbedding
from babyvllm.worker.context import get_forward_context


class Qwen2MLP(nn.Module):
    def __init__(self, hidden_size: int, intermediate_size: int):
        super().__init__()
        self.gate_up_proj = nn.Linear(hidden_size, 2 * intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x):
        return self.down_proj(fused_silu_mul(self.gate_up_proj(x)))


class Qwen2Attention(nn.Module):
    def __init__(self, cfg, layer_idx: int):
        super().__init__()
        self.layer_idx = layer_idx
        self.num_heads = cfg.num_attention_heads
        self.num_kv_heads = cfg.num_key_value_heads
        self.head_dim = cfg.head_dim
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim
        self.qkv_proj = nn.Linear(cfg.hidden_size, self.q_size + 2 * self.kv_size, bias=True)
        self.o_proj = nn.Linear(self.q_size, cfg.hidden_size, bias=False)
        self.attn = Attention(self.num_heads, self.head_dim, self.num_kv_heads)

    def forward(self, x, cos, sin):
        qkv = self.qkv_proj(x)
        q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
        q = q.view(-1, self.num_heads, self.head_dim)
        k = k.view(-1, self.num_kv_heads, self.head_dim)
        v = v.view(-1, self.num_kv_heads, self.head_dim)
        ctx = get_forward_context()
        if ctx is None or self.attn.kv_cache is None:
            raise RuntimeError("Qwen2Attention needs a KV cache and a forward context")
        q, k = fused_rope_and_cache(q, k, v, cos, sin, kv_cache=self.attn.kv_cache,
                                    slot_mapping=ctx.attn_metadata.slot_mapping)
        o = self.attn(q, k, v)
        return self.o_proj(o.reshape(-1, self.q_size))


class Qwen2DecoderLayer(nn.Module):
    def __init__(self, cfg, layer_idx: int):
        super().__init__()
        self.self_attn = Qwen2Attention(cfg, layer_idx)
        self.mlp = Qwen2MLP(cfg.hidden_size, cfg.intermediate_size)
        self.input_layernorm = RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps)

    def forward(self, hidden_states, residual, cos, sin):
        normed, residual = self.input_layernorm(hidden_states, residual)
        hidden_states = self.self_attn(normed, cos, sin)
        normed, residual = self.post_attention_layernorm(hidden_states, residual)
        return self.mlp(normed), residual


class Qwen2Model(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList([Qwen2DecoderLayer(cfg, i) for i in range(cfg.num_hidden_layers)])
        self.norm = RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps)
        self.rotary_emb = RotaryEmbedding(cfg.head_dim, max_position_embeddings=cfg.max_position_embeddings,
                                          base=cfg.rope_theta)

    def forward(self, input_ids, positions):
        hidden = self.embed_tokens(input_ids)
        cos, sin = self.rotary_emb(positions, hidden.dtype)
        residual = None
        for layer in self.layers:
            hidden, residual = layer(hidden, residual, cos, sin)
        hidden, _ = self.norm(hidden, residual)
        return hidden


class Qwen2ForCausalLM(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.config = cfg
        self.model = Qwen2Model(cfg)
        self.lm_head = None if cfg.tie_word_embeddings else nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)

    def compute_logits(self, hidden, out=None):
        w = self.model.embed_tokens.weight if self.lm_head is None else self.lm_head.weight
        if out is None:
            return F.linear(hidden, w)
        return torch.mm(hidden, w.t(), out=out)

    def forward(self, input_ids, positions):
        return self.model(input_ids, positions)

    @torch.no_grad()
    def init_random(self, seed: int, std: float = 0.02) -> None:
        """Seeded N(0, std) weights and zero biases; norm weights stay 1 (random-init benchmark model)."""
        g = torch.Generator(device=next(self.parameters()).device).manual_seed(seed)
        for name, p in self.named_parameters():
            if name.endswith("layernorm.weight") or name.endswith("norm.weight"):
                p.fill_(1.0)
            elif name.endswith(".bias"):
                p.zero_()
            else:
                p.normal_(0.0, std, generator=g)
