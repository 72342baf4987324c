"""BASELINE config 1 as one whole step on the HIP path: a single-layer paged
decode step at the Qwen2.5-0.5B shape.

14 query / 2 KV heads, head_dim 64, block 16, batch 8, lengths U[100, 512]
(seeded), a 512-block pool whose rows are a seeded permutation (width 32),
q/k/v ~ N(0, 1) in bf16. RotaryEmbedding(θ = 1e6) gives cos/sin at each
sequence's last position (seq_len − 1); the fused RoPE + append rotates q and
k and writes the new token's K/V through slot_mapping; then the Attention
layer's decode dispatch attends with max_seq_len = 512 (the bucket).

Checked against the oracle (the reference's torch path restated on the CPU):
q, k and the whole pool bit for bit, the attention output within max-abs 2e-2
and mean-abs 2e-3 of fp32. The same step captured in a hipGraph and replayed
with the next token of every sequence is checked the same way.
"""

import pytest
import torch

from oracle import attention as oa
from oracle import rope as orope
from tests._cases import assert_attn_close

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU"),
]

H, HKV, D, BS, B = 14, 2, 64, 16, 8
POOL, WIDTH, BUCKET, THETA = 512, 32, 512, 1e6


def _case(seed):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(100, 513, (B,), generator=g)
    cache = torch.randn(2, POOL, BS, HKV, D, generator=g).bfloat16()
    bt = torch.randperm(POOL, generator=g)[: B * WIDTH].view(B, WIDTH).int()
    qkv = torch.randn(B, (H + 2 * HKV) * D, generator=g).bfloat16()
    return lens, cache, bt, qkv


def _views(qkv):
    q = qkv[:, : H * D].view(-1, H, D)
    k = qkv[:, H * D:(H + HKV) * D].view(-1, HKV, D)
    v = qkv[:, (H + HKV) * D:].view(-1, HKV, D)
    return q, k, v


def _slots(bt, pos):
    return bt[torch.arange(len(pos)), pos // BS].long() * BS + pos % BS


def _oracle_step(lens, cache, bt, qkv):
    """RoPE + store + decode on the CPU (fp32 attention of the rotated bf16 q)."""
    pos = lens - 1
    ct, st = orope.rope_tables(D, 4096, THETA)
    q, k, v = _views(qkv)
    q_ref, k_ref = orope.apply_rope(q, k, ct[pos].bfloat16(), st[pos].bfloat16())
    cache_ref = cache.clone()
    orope.store_kvcache(k_ref, v, cache_ref, _slots(bt, pos))
    out = oa.static_decode_attention(q_ref.float(), cache_ref.float(), bt, lens.int(), BUCKET, D ** -0.5)
    return q_ref, k_ref, cache_ref, out


class _Step:
    """The product's step: RotaryEmbedding → fused_rope_and_cache → Attention."""

    def __init__(self, lens, cache, bt):
        from babyvllm.layers.attention import Attention
        from babyvllm.layers.rotary import RotaryEmbedding

        dev = torch.device("cuda")
        self.rotary = RotaryEmbedding(D, 4096, THETA).to(dev)
        self.attn = Attention(H, D, HKV)
        self.attn.kv_cache = cache.to(dev)
        self.bt = bt.to(dev)
        self.lens = lens.int().to(dev)
        self.positions = (lens - 1).to(dev)
        self.slots = _slots(bt, lens - 1).to(dev)
        self.qkv = torch.empty(B, (H + 2 * HKV) * D, device=dev, dtype=torch.bfloat16)

    def run(self):
        from babyvllm.kernels.rope import fused_rope_and_cache
        from babyvllm.worker.context import AttentionMetadata, set_forward_context

        q, k, v = _views(self.qkv)
        cos, sin = self.rotary(self.positions, torch.bfloat16)
        q, k = fused_rope_and_cache(q, k, v, cos, sin, kv_cache=self.attn.kv_cache, slot_mapping=self.slots)
        md = AttentionMetadata(
            slot_mapping=self.slots, block_tables=self.bt,
            query_start_loc=torch.arange(B + 1, dtype=torch.int32, device=q.device),
            seq_lens=self.lens, context_lens=self.lens - 1,
            query_start_loc_cpu=list(range(B + 1)), seq_lens_cpu=[BUCKET] * B,
            context_lens_cpu=[BUCKET - 1] * B, max_query_len=1, max_seq_len=BUCKET)
        with set_forward_context(md):
            return self.attn(q, k, v)

    def load(self, lens, qkv, bt):
        self.lens.copy_(lens.int())
        self.positions.copy_(lens - 1)
        self.slots.copy_(_slots(bt, lens - 1))
        self.qkv.copy_(qkv)


def _check(step, out, lens, cache, bt, qkv):
    q_ref, k_ref, cache_ref, want = _oracle_step(lens, cache, bt, qkv)
    q, k, _ = _views(step.qkv)
    assert torch.equal(q.cpu(), q_ref), "rotated q differs from the oracle"
    assert torch.equal(k.cpu(), k_ref), "rotated k differs from the oracle"
    assert torch.equal(step.attn.kv_cache.cpu().view(torch.int16), cache_ref.view(torch.int16)), \
        "KV pool differs from the oracle"
    assert_attn_close(out, want)
    return cache_ref


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config1_step_matches_the_oracle(seed):
    lens, cache, bt, qkv = _case(seed)
    step = _Step(lens, cache, bt)
    step.load(lens, qkv, bt)
    out = step.run()
    torch.cuda.synchronize()
    _check(step, out, lens, cache, bt, qkv)


def test_config1_step_in_a_graph_over_consecutive_tokens():
    lens, cache, bt, qkv = _case(7)
    step = _Step(lens, cache, bt)
    step.load(lens, qkv, bt)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step.run()  # warm-up writes the first token's K/V, as the first replay will again
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step.run()
    g = torch.Generator().manual_seed(8)
    ref_cache = cache
    for t in range(3):
        cur = torch.clamp(lens + t, max=BUCKET)
        new_qkv = torch.randn(B, (H + 2 * HKV) * D, generator=g).bfloat16()
        step.load(cur, new_qkv, bt)
        graph.replay()
        torch.cuda.synchronize()
        ref_cache = _check(step, out, cur, ref_cache, bt, new_qkv)
