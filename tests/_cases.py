"""Seeded inputs shared by the GPU parity tests, and the attention tolerance.

Builders follow the reference's fixtures: ``make_decode_inputs`` is
``_make_inputs`` (tests/test_paged_attn.py:77-90) and ``build_prefill_case`` is
``build_case`` (tests/test_paged_prefill.py:24-67, unwritten slots NaN).
"""

from __future__ import annotations

from contextlib import contextmanager

import torch

from babyvllm.worker.context import AttentionMetadata

BLOCK_SIZE = 16
# Tolerance stated for the attention outputs: bf16 with fp32 accumulation.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


def assert_attn_close(actual: torch.Tensor, expected: torch.Tensor, rows=None):
    """max |a − e| ≤ 2e-2 and mean |a − e| ≤ 2e-3, on the given rows (default: all)."""
    a = actual.float().cpu()
    e = expected.float().cpu()
    if rows is not None:
        a, e = a[rows], e[rows]
    assert not torch.isnan(a).any(), "NaN in kernel output"
    diff = (a - e).abs()
    assert diff.max().item() <= MAX_ABS, f"max abs diff {diff.max().item():.4g} > {MAX_ABS}"
    assert diff.mean().item() <= MEAN_ABS, f"mean abs diff {diff.mean().item():.4g} > {MEAN_ABS}"


def make_decode_inputs(lens, hkv=4, group=7, d=128, width=None, seed=0, device="cuda"):
    """Ragged decode batch with a shuffled block table; a length of 0 is a padded row."""
    g = torch.Generator(device=device).manual_seed(seed)
    B = len(lens)
    width = width or cdiv(max(max(lens), 1), BLOCK_SIZE) + 2
    total = B * width + 1
    q = torch.randn(B, hkv * group, d, device=device, dtype=torch.bfloat16, generator=g)
    kv_cache = torch.randn(2, total, BLOCK_SIZE, hkv, d, device=device, dtype=torch.bfloat16,
                           generator=g)
    perm = torch.randperm(total, device=device, generator=g)[: B * width]
    block_tables = perm.view(B, width).to(torch.int32)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=device)
    return q, kv_cache, block_tables, seq_lens


def build_prefill_case(specs, hkv, group, d, seed=0, nan_fill=True, device="cuda"):
    """specs: list of (context_len, query_len). Unwritten cache slots are NaN."""
    g = torch.Generator(device=device).manual_seed(seed)
    H = hkv * group
    seq_lens = [c + n for c, n in specs]
    blocks_per_seq = [cdiv(s, BLOCK_SIZE) for s in seq_lens]
    total = sum(blocks_per_seq) + 3
    width = max(blocks_per_seq)
    fill = float("nan") if nan_fill else 0.0
    kv_cache = torch.full((2, total, BLOCK_SIZE, hkv, d), fill, device=device, dtype=torch.bfloat16)
    perm = torch.randperm(total, device=device, generator=g).tolist()
    tables, written = [], []
    for n, s in zip(blocks_per_seq, seq_lens):
        table = [perm.pop() for _ in range(n)]
        written.extend(table[p // BLOCK_SIZE] * BLOCK_SIZE + p % BLOCK_SIZE for p in range(s))
        tables.append(table + [0] * (width - n))
    flat = kv_cache.view(2, -1, hkv, d)
    flat[:, torch.tensor(written, device=device)] = torch.randn(
        2, len(written), hkv, d, device=device, dtype=torch.bfloat16, generator=g)
    q_lens = [n for _, n in specs]
    q = torch.randn(sum(q_lens), H, d, device=device, dtype=torch.bfloat16, generator=g)
    qsl = [0]
    for n in q_lens:
        qsl.append(qsl[-1] + n)
    ctx = [c for c, _ in specs]
    md = AttentionMetadata(
        slot_mapping=torch.zeros(sum(q_lens), dtype=torch.int64, device=device),
        block_tables=torch.tensor(tables, dtype=torch.int32, device=device),
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=device),
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=device),
        context_lens=torch.tensor(ctx, dtype=torch.int32, device=device),
        query_start_loc_cpu=qsl,
        seq_lens_cpu=seq_lens,
        context_lens_cpu=ctx,
        max_query_len=max(q_lens),
        max_seq_len=max(seq_lens),
    )
    return q, kv_cache, md


def scale_keys_by_position(kv_cache, block_tables, seq_lens, factor):
    """Multiplies the key at position p of every row by factor(p), in place:
    with growing factors a row's later scores exceed its running max many
    times over, which drives the kernels' rescale paths."""
    bs = kv_cache.shape[2]
    bt = block_tables.cpu()
    for row, n in enumerate(int(x) for x in seq_lens):
        if n == 0:
            continue
        pos = torch.arange(n)
        blocks = bt[row, pos // bs].long().to(kv_cache.device)
        offs = (pos % bs).to(kv_cache.device)
        f = torch.tensor([factor(int(p)) for p in pos], dtype=torch.float32, device=kv_cache.device)
        k = kv_cache[0, blocks, offs].float() * f[:, None, None]
        kv_cache[0, blocks, offs] = k.to(kv_cache.dtype)


def md_to_cpu(md):
    return AttentionMetadata(
        slot_mapping=md.slot_mapping.cpu(), block_tables=md.block_tables.cpu(),
        query_start_loc=md.query_start_loc.cpu(), seq_lens=md.seq_lens.cpu(),
        context_lens=md.context_lens.cpu(), query_start_loc_cpu=md.query_start_loc_cpu,
        seq_lens_cpu=md.seq_lens_cpu, context_lens_cpu=md.context_lens_cpu,
        max_query_len=md.max_query_len, max_seq_len=md.max_seq_len,
    )


@contextmanager
def tuned(knob: int, value: int):
    """Sets a library tuning knob (bvllm_set_tuning) for the block, then restores it."""
    from babyvllm.kernels import _lib
    prev = _lib.set_tuning(knob, value)
    try:
        yield
    finally:
        _lib.set_tuning(knob, prev)
