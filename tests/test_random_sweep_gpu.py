"""Seeded random sweeps over the attention kernels' launch choices.

Decode: random batches (padded rows, ragged lengths up to 9,000 tokens, buckets
and table widths above the longest row, every partition size the reference's
split plan takes, GQA groups 1 to 64) run under every decode launch choice
(default, split mode 1/2/3, split-major wave order, cached page loads); all
must give the same bits, and one case in five is checked against the oracle
(oracle.attention.static_decode_attention, the reference's
babyvllm/layers/attention.py:71-134).

Prefill: random varlen batches (cached prefixes, ragged query lengths,
single-token decode rows in the same launch, NaN in unwritten cache slots) are
checked against oracle.attention.paged_attention_torch (the reference's
babyvllm/layers/attention.py:137-175); the blocks-per-work-group switch must
give the default's bits and the short-grid switch the oracle's values.
"""

import random

import pytest
import torch

from oracle import attention as oa
from tests._cases import assert_attn_close, build_prefill_case, make_decode_inputs, md_to_cpu, tuned

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU"),
]

_SPLIT_MODE, _BPW, _ORDER, _CACHED, _SHORT_GRID = 0, 1, 2, 4, 6  # bvllm_set_tuning knobs

_DECODE_HEADS = [(4, 7, 128), (2, 7, 64), (8, 4, 128), (1, 16, 128), (4, 1, 64), (1, 32, 128), (2, 24, 64),
                 (1, 64, 128)]
_DECODE_CHOICES = [None, (_SPLIT_MODE, 1), (_SPLIT_MODE, 2), (_SPLIT_MODE, 3), (_SPLIT_MODE, 4), (_ORDER, 1),
                   (_CACHED, 1)]


def _decode_case(rng):
    hkv, group, d = rng.choice(_DECODE_HEADS)
    B = rng.choice([1, 2, 3, 4, 5, 8, 13, 16, 33])
    maxlen = rng.choice([64, 700, 2000, 5000, 9000])
    lens = [rng.randint(0, maxlen) for _ in range(B)]
    if rng.random() < 0.3:
        lens[rng.randrange(B)] = 0
    bucket = max(max(lens), 1) + rng.choice([0, 0, 15, 300, 4000])
    width = (bucket + 15) // 16 + rng.choice([0, 1, 7])
    partition = rng.choice([None, None, 0, 1, 2, 3, 4, 5, 8, 16, 32])
    return dict(hkv=hkv, group=group, d=d, lens=lens, bucket=bucket, width=width, partition=partition)


@pytest.mark.parametrize("block", range(4))
def test_decode_launch_choices_agree_on_random_batches(block):
    from babyvllm.kernels.paged_attn import paged_decode_attention
    rng = random.Random(1000 + block)
    for case in range(30):
        c = _decode_case(rng)
        print("decode sweep", block, case, c, flush=True)
        q, kv, bt, sl = make_decode_inputs(c["lens"], hkv=c["hkv"], group=c["group"], d=c["d"], width=c["width"],
                                           seed=100 * block + case)
        scale = c["d"] ** -0.5
        outs = []
        for choice in _DECODE_CHOICES:
            run = lambda: paged_decode_attention(q, kv, bt, sl, scale, max_seq_len=c["bucket"],
                                                 partition_blocks=c["partition"])
            if choice is None:
                outs.append(run())
            else:
                with tuned(*choice):
                    outs.append(run())
        for choice, o in zip(_DECODE_CHOICES[1:], outs[1:]):
            assert torch.equal(o, outs[0]), f"launch choice {choice} differs from the default on {c}"
        live = [i for i, n in enumerate(c["lens"]) if n > 0]
        if case % 5 == 0 and live:
            ref = oa.static_decode_attention(q.float().cpu(), kv.float().cpu(), bt.cpu(),
                                             torch.tensor(c["lens"], dtype=torch.int32), max(c["lens"]), scale)
            assert_attn_close(outs[0], ref, rows=live)


_PREFILL_HEADS = [(4, 7, 128), (2, 7, 64), (4, 1, 64), (1, 32, 128), (2, 24, 64), (8, 2, 128)]


def _prefill_specs(rng):
    short = rng.random() < 0.3  # every row within 8 pages: several column blocks per work-group
    specs = []
    for _ in range(rng.choice([1, 1, 2, 3, 5, 8, 12])):
        if short:
            ctx = rng.choice([0, 0, 5, 16, 40, 64])
            specs.append((ctx, rng.randint(1, 128 - ctx)))
        else:
            specs.append((rng.choice([0, 0, 17, 64, 300, 1024, 2000]), rng.choice([1, 1, 2, 15, 64, 129, 300])))
    return short, specs


@pytest.mark.parametrize("block", range(3))
def test_prefill_on_random_varlen_batches(block):
    from babyvllm.kernels.paged_prefill import paged_prefill_attention
    rng = random.Random(2000 + block)
    for case in range(20):
        hkv, group, d = rng.choice(_PREFILL_HEADS)
        short, specs = _prefill_specs(rng)
        if sum(n for _, n in specs) * max(c + n for c, n in specs) * hkv * group > 6e7:
            specs = specs[:2]  # keeps the CPU oracle within seconds
        print("prefill sweep", block, case, dict(hkv=hkv, group=group, d=d, specs=specs), flush=True)
        q, kv, md = build_prefill_case(specs, hkv, group, d, seed=100 * block + case)
        scale = d ** -0.5
        out = paged_prefill_attention(q, kv, md, scale)
        if short:
            for bpw in (2, 3):
                with tuned(_BPW, bpw):
                    assert torch.equal(paged_prefill_attention(q, kv, md, scale), out), f"{bpw} blocks per work-group"
        with tuned(_SHORT_GRID, 1):
            out_sg = paged_prefill_attention(q, kv, md, scale)
        cache = torch.nan_to_num(kv.float().cpu(), nan=0.0)
        ref = oa.paged_attention_torch(q.float().cpu(), cache, md_to_cpu(md), scale, group)
        assert_attn_close(out, ref)
        assert_attn_close(out_sg, ref)
