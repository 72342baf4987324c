"""Paged decode attention: HIP kernel vs the CPU oracle (ports tests/test_paged_attn.py).

Oracle: oracle.attention.static_decode_attention (the reference's gather + SDPA
decode, babyvllm/layers/attention.py:113-134) in float32 on the CPU, and the
float64 split/LSE restatement for the split invariants.
"""

import pytest
import torch

from oracle import attention as oa
from tests._cases import BLOCK_SIZE, assert_attn_close, cdiv, make_decode_inputs, scale_keys_by_position, tuned

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU"),
]

HEAD_DIM = 128
GRAPH_TABLE_WIDTH = 129  # 2048 / 16 + 1


def _kernel():
    from babyvllm.kernels.paged_attn import paged_decode_attention
    return paged_decode_attention


def _oracle(q, kv_cache, bt, lens, scale, bucket=None):
    lens_t = torch.tensor(lens, dtype=torch.int32)
    bucket = bucket or max(max(lens), 1)
    out = oa.static_decode_attention(q.float().cpu(), kv_cache.float().cpu(), bt.cpu(), lens_t,
                                     bucket, scale)
    return out


def _live(lens):
    return [i for i, n in enumerate(lens) if n > 0]


@pytest.mark.parametrize("B", [1, 2, 7, 64])
@pytest.mark.parametrize("seq_len", [1, 15, 16, 17, 31, 32, 127, 128, 2048])
def test_paged_decode_parity(B, seq_len):
    scale = HEAD_DIM ** -0.5
    q, kv_cache, bt, seq_lens = make_decode_inputs([seq_len] * B, seed=B * 10000 + seq_len)
    actual = _kernel()(q, kv_cache, bt, seq_lens, scale)
    assert_attn_close(actual, _oracle(q, kv_cache, bt, [seq_len] * B, scale))


RAGGED = [1, 17, 300, 2048, 0, 64, 1000, 16]


@pytest.mark.parametrize("partition", [0, 1, 2, 3, 7, 8, 64])
def test_split_decode_matches_reference_on_ragged_batch(partition):
    scale = HEAD_DIM ** -0.5
    q, kv_cache, bt, seq_lens = make_decode_inputs(RAGGED, width=GRAPH_TABLE_WIDTH)
    actual = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=2048, partition_blocks=partition)
    assert_attn_close(actual, _oracle(q, kv_cache, bt, RAGGED, scale), rows=_live(RAGGED))
    assert actual[RAGGED.index(0)].abs().max() == 0


@pytest.mark.parametrize("n", [1, 15, 16, 17, 127, 128, 129, 255, 256, 1023, 2047, 2048])
def test_auto_split_with_bucket_wider_than_live_length(n, monkeypatch):
    from babyvllm.kernels.decode_split import DECODE_PARTITION_ENV, decode_split_plan

    monkeypatch.delenv(DECODE_PARTITION_ENV, raising=False)
    scale = HEAD_DIM ** -0.5
    q, kv_cache, bt, seq_lens = make_decode_inputs([n], width=GRAPH_TABLE_WIDTH, seed=n)
    sms = torch.cuda.get_device_properties(0).multi_processor_count
    splits, _ = decode_split_plan(1, 4, BLOCK_SIZE, GRAPH_TABLE_WIDTH, 2048, sms)
    assert splits > 1
    actual = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=2048)
    assert_attn_close(actual, _oracle(q, kv_cache, bt, [n], scale))


def test_live_length_and_graph_bucket_give_identical_bits(monkeypatch):
    from babyvllm.kernels.decode_split import DECODE_PARTITION_ENV

    monkeypatch.delenv(DECODE_PARTITION_ENV, raising=False)
    scale = HEAD_DIM ** -0.5
    lens = [300, 17, 129, 0, 5]
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, width=GRAPH_TABLE_WIDTH)
    eager = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=max(lens))
    graph = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=2048)
    assert torch.equal(eager, graph)


@pytest.mark.parametrize("n", [1, 17, 63, 64])
def test_row_within_one_partition_matches_single_pass_bits(n):
    from babyvllm.kernels.decode_split import auto_partition_blocks

    partition = auto_partition_blocks(2)
    assert n <= partition * BLOCK_SIZE
    scale = HEAD_DIM ** -0.5
    q, kv_cache, bt, seq_lens = make_decode_inputs([n, n], width=GRAPH_TABLE_WIDTH, seed=n)
    single = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=2048, partition_blocks=0)
    split = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=2048, partition_blocks=partition)
    assert torch.equal(single, split)


def test_row_longer_than_the_bucket_is_attended_in_full():
    scale = HEAD_DIM ** -0.5
    lens = [1000, 40]
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens)
    actual = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=256, partition_blocks=4)
    assert_attn_close(actual, _oracle(q, kv_cache, bt, lens, scale))


@pytest.mark.parametrize("partition_env", ["0", "auto"])
def test_decode_attention_replays_in_a_hip_graph(partition_env, monkeypatch):
    """Grid frozen at capture; lengths, tables and q change between replays."""
    from babyvllm.kernels.decode_split import DECODE_PARTITION_ENV

    monkeypatch.setenv(DECODE_PARTITION_ENV, partition_env)
    scale = HEAD_DIM ** -0.5
    q, kv_cache, bt, seq_lens = make_decode_inputs([2048, 2048, 0, 0], width=GRAPH_TABLE_WIDTH)
    run = lambda: _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=2048)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()

    g = torch.Generator(device="cuda").manual_seed(7)
    for lens in ([5, 2048, 0, 0], [1999, 33, 129, 0], [1, 1, 1, 1], [5, 2048, 0, 0]):
        seq_lens.copy_(torch.tensor(lens, dtype=torch.int32))
        bt.copy_(torch.randperm(bt.numel(), device="cuda", generator=g).view_as(bt).to(torch.int32))
        q.copy_(torch.randn(q.shape, device="cuda", dtype=q.dtype, generator=g))
        graph.replay()
        torch.cuda.synchronize()
        eager = run()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert_attn_close(out, _oracle(q, kv_cache, bt, lens, scale), rows=_live(lens))
        for i, n in enumerate(lens):
            if n == 0:
                assert out[i].abs().max() == 0


def test_unwritten_nan_slots_past_seq_len_do_not_leak():
    scale = HEAD_DIM ** -0.5
    lens = [17, 33, 5]
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, seed=3)
    clean = kv_cache.clone()
    for i, n in enumerate(lens):
        page = bt[i, (n - 1) // BLOCK_SIZE].item()
        kv_cache[:, page, n % BLOCK_SIZE or BLOCK_SIZE:] = float("nan")
        clean[:, page, n % BLOCK_SIZE or BLOCK_SIZE:] = 0
    for part in (0, 1):
        actual = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=64, partition_blocks=part)
        assert_attn_close(actual, _oracle(q, clean, bt, lens, scale))


@pytest.mark.parametrize("hkv,group,d", [(2, 7, 64), (4, 1, 64), (1, 16, 128), (8, 4, 128)])
def test_other_head_configs(hkv, group, d):
    lens = [1, 40, 200, 513]
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, hkv=hkv, group=group, d=d, seed=11)
    for part in (0, None, 3):
        actual = _kernel()(q, kv_cache, bt, seq_lens, d ** -0.5, max_seq_len=520, partition_blocks=part)
        assert_attn_close(actual, _oracle(q, kv_cache, bt, lens, d ** -0.5))


# GQA groups above one 16-column MFMA tile (MQA-style layouts): the group is cut
# into 16-head column groups; the reference pads any group
# (babyvllm/kernels/paged_attn.py:275).
_WIDE_GROUPS = [(1, 32, 128), (1, 64, 128), (2, 24, 64), (1, 17, 64), (3, 20, 128)]


@pytest.mark.parametrize("hkv,group,d", _WIDE_GROUPS)
def test_gqa_groups_above_16(hkv, group, d):
    lens = [1, 40, 200, 513, 0, 1100]
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, hkv=hkv, group=group, d=d, seed=group)
    want = _oracle(q, kv_cache, bt, lens, d ** -0.5)
    for part in (0, None, 3, 8):
        actual = _kernel()(q, kv_cache, bt, seq_lens, d ** -0.5, max_seq_len=1200, partition_blocks=part)
        assert_attn_close(actual, want, rows=_live(lens))
        assert actual[4].abs().max() == 0


@pytest.mark.parametrize("hkv,group,d", _WIDE_GROUPS[:3])
def test_gqa_groups_above_16_launch_choices_agree(hkv, group, d):
    lens = [700, 33, 0, 1500]
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, width=128, seed=7 * group, hkv=hkv, group=group, d=d)
    scale = d ** -0.5
    for partition in (4, 0, 2):
        outs = _modes(q, kv_cache, bt, seq_lens, scale, 2048, partition)
        for name, out in outs.items():
            assert torch.equal(out, outs["auto"]), name
        assert_attn_close(outs["auto"], _oracle(q, kv_cache, bt, lens, scale), rows=_live(lens))


def test_strided_q_view_into_fused_qkv():
    lens = [100, 7]
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, seed=5)
    B, H, D = q.shape
    qkv = torch.randn(B, (H + 8) * D, device="cuda", dtype=q.dtype)
    view = qkv[:, : H * D].view(B, H, D)
    view.copy_(q)
    assert not view.is_contiguous()
    assert torch.equal(_kernel()(view, kv_cache, bt, seq_lens, D ** -0.5),
                       _kernel()(q, kv_cache, bt, seq_lens, D ** -0.5))


# ---------------------------------------------------- BASELINE config 3 shapes

@pytest.mark.parametrize("batch,ctx", [(64, 1920), (8, 1920), (1, 32768)])
def test_baseline_decode_configs(batch, ctx):
    scale = HEAD_DIM ** -0.5
    lens = [ctx] * batch
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, width=cdiv(ctx, BLOCK_SIZE), seed=ctx + batch)
    actual = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=ctx)
    assert_attn_close(actual, _oracle(q, kv_cache, bt, lens, scale))


@pytest.mark.parametrize("n", [600, 130, 2047])
def test_reduce_bits_do_not_depend_on_the_split_count(n, monkeypatch):
    """A row's bits depend only on its non-empty splits: an eager launch with
    few splits (one reduce group) and a graph-bucket launch with more than 32
    splits (several groups) agree bit for bit."""
    from babyvllm.kernels.decode_split import DECODE_PARTITION_ENV, decode_split_plan

    monkeypatch.delenv(DECODE_PARTITION_ENV, raising=False)
    scale = HEAD_DIM ** -0.5
    q, kv_cache, bt, seq_lens = make_decode_inputs([n], width=520, seed=n)
    sms = torch.cuda.get_device_properties(0).multi_processor_count
    s_eager, _ = decode_split_plan(1, 4, BLOCK_SIZE, 520, n, sms)
    s_graph, _ = decode_split_plan(1, 4, BLOCK_SIZE, 520, 8192, sms)
    assert s_eager <= 32 < s_graph or n > 32 * 4 * BLOCK_SIZE
    eager = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=n)
    graph = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=8192)
    assert torch.equal(eager, graph)
    assert_attn_close(graph, _oracle(q, kv_cache, bt, [n], scale))


def _modes(q, kv_cache, bt, seq_lens, scale, bucket, partition):
    """Outputs of every launch choice that must give the same bits: split mode
    (four waves per split of at most 32 pages and two per longer split by
    default, two waves per split throughout, one wave per split, one or two
    waves per group of 4 splits), wave order, nontemporal page loads, single
    pass on streaming waves."""
    from babyvllm.kernels import _lib

    outs = {}
    choices = [("auto", None, 0), ("per_split", _lib.TUNE_DECODE_SPLIT_MODE, 1),
               ("per_group", _lib.TUNE_DECODE_SPLIT_MODE, 2), ("pair_group", _lib.TUNE_DECODE_SPLIT_MODE, 3),
               ("pair_split", _lib.TUNE_DECODE_SPLIT_MODE, 4),
               ("order1", _lib.TUNE_DECODE_ORDER, 1), ("cached", _lib.TUNE_DECODE_CACHED, 1),
               ("stream_single", _lib.TUNE_DECODE_SINGLE_PASS_STREAM, 1)]
    for name, knob, value in choices:
        if knob is None:
            outs[name] = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=bucket, partition_blocks=partition)
            continue
        with tuned(knob, value):
            outs[name] = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=bucket,
                                   partition_blocks=partition)
    return outs


@pytest.mark.parametrize("partition", [None, 0, 1, 2, 3, 4, 7, 8, 16])
@pytest.mark.parametrize("lens", [[600, 37, 0, 1], [2047, 16, 64, 300], [5000, 129], [130, 129, 128, 127]])
def test_launch_choices_do_not_change_bits(partition, lens, monkeypatch):
    """Every launch choice of one plan gives identical bits: two waves or one
    wave per split (groups of 4 splits folded in the reduce) or one or two per
    group (folded in the wave, the two waves handing states over at every
    split's end), either wave order, with or without the nontemporal hint, and
    the single pass on work-groups or streaming waves.
    Rows longer than the bucket and rows ending inside a group are covered."""
    from babyvllm.kernels.decode_split import DECODE_PARTITION_ENV

    monkeypatch.delenv(DECODE_PARTITION_ENV, raising=False)
    scale = HEAD_DIM ** -0.5
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, width=330, seed=len(lens) + (partition or 0))
    outs = _modes(q, kv_cache, bt, seq_lens, scale, 4096, partition)
    for name, out in outs.items():
        assert torch.equal(out, outs["auto"]), name
    assert not torch.isnan(outs["auto"]).any()
    assert_attn_close(outs["auto"], _oracle(q, kv_cache, bt, lens, scale), rows=_live(lens))


@pytest.mark.parametrize("hkv,group,d", [(2, 7, 64), (4, 7, 128), (1, 32, 128), (2, 24, 64)])
@pytest.mark.parametrize("partition,bucket", [(8, 512), (4, 192), (5, 150), (4, 128), (16, 512), (4, 256)])
def test_plans_of_two_to_four_splits(hkv, group, d, partition, bucket):
    """Plans of 2-4 splits (the reduce folds groups of 4 splits when the pages
    per split are a multiple of 4, not at 5): every launch choice gives the
    same bits and the oracle's values, on rows of the bucket's length, of 0 and
    1 tokens, and rows ending inside a split."""
    lens = [bucket, 1, 0, bucket - 37, 17]
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, width=cdiv(bucket, BLOCK_SIZE) + 1, seed=partition + bucket,
                                                   hkv=hkv, group=group, d=d)
    scale = d ** -0.5
    outs = _modes(q, kv_cache, bt, seq_lens, scale, bucket, partition)
    for name, out in outs.items():
        assert torch.equal(out, outs["auto"]), name
    assert_attn_close(outs["auto"], _oracle(q, kv_cache, bt, lens, scale), rows=_live(lens))


@pytest.mark.parametrize("hkv,group,d", [(2, 7, 64), (1, 16, 128), (8, 4, 128), (4, 1, 64)])
def test_launch_choices_other_head_configs(hkv, group, d):
    lens = [700, 33, 0, 1500]
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, width=128, seed=hkv * 10 + group, hkv=hkv, group=group,
                                                   d=d)
    scale = d ** -0.5
    for partition in (4, 0):
        outs = _modes(q, kv_cache, bt, seq_lens, scale, 2048, partition)
        for name, out in outs.items():
            assert torch.equal(out, outs["auto"]), name
        assert_attn_close(outs["auto"], _oracle(q, kv_cache, bt, lens, scale), rows=_live(lens))


def test_single_pass_walk_lengths_around_the_table_slices():
    """The single pass's page walk (wave w of 4 takes pages w, w+4, ...; one page
    in flight, none requested past the wave's last page; the row's table entries
    come in slices of 64 per wave) on rows whose per-wave page counts sit at and
    just past a slice (4096 tokens: 64 pages per wave; 4097: 65 for wave 0) and on
    rows of one to five pages (waves with no page or one): the same bits as the
    single pass on streaming waves, and the oracle's values."""
    lens = [4096, 4097, 4112, 4113, 1, 17, 33, 49, 65, 0]
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, seed=41)
    scale = HEAD_DIM ** -0.5
    from babyvllm.kernels import _lib

    wg = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=max(lens), partition_blocks=0)
    with tuned(_lib.TUNE_DECODE_SINGLE_PASS_STREAM, 1):
        st = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=max(lens), partition_blocks=0)
    assert torch.equal(wg, st)
    assert wg[len(lens) - 1].abs().max() == 0
    assert_attn_close(wg, _oracle(q, kv_cache, bt, lens, scale), rows=_live(lens))


@pytest.mark.parametrize("partition", [0, 1, 4])
def test_scores_rising_along_the_row(partition):
    """Key norms growing with position: the running max of every split is
    raised page after page (the online-softmax rescale path)."""
    scale = HEAD_DIM ** -0.5
    lens = [3000, 1, 700, 0, 2048]
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, width=GRAPH_TABLE_WIDTH + 60, seed=3)
    scale_keys_by_position(kv_cache, bt, lens, lambda p: 1.0 + p / 64.0)
    actual = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=3000, partition_blocks=partition)
    assert_attn_close(actual, _oracle(q, kv_cache, bt, lens, scale), rows=_live(lens))


# ------------------------------------------------------- seeded random batches

_HEAD_CONFIGS = [(4, 7, 128), (2, 7, 64), (1, 16, 128), (8, 4, 128), (4, 1, 64), (2, 3, 64)]


@pytest.mark.parametrize("seed", range(24))
def test_random_ragged_batches(seed):
    """Seeded random batches: 1-40 rows of 0-3000 tokens (a tenth of them
    padded, length 0), a bucket at or above the longest row, random head
    configurations and partition sizes (auto, single pass, 1-16 pages)."""
    g = torch.Generator().manual_seed(3000 + seed)
    hkv, group, d = _HEAD_CONFIGS[int(torch.randint(len(_HEAD_CONFIGS), (1,), generator=g))]
    B = int(torch.randint(1, 41, (1,), generator=g))
    lens = [0 if int(torch.randint(10, (1,), generator=g)) == 0 else int(torch.randint(1, 3001, (1,), generator=g))
            for _ in range(B)]
    if max(lens) == 0:
        lens[0] = 1
    bucket = max(lens) + int(torch.randint(0, 65, (1,), generator=g))
    choice = int(torch.randint(18, (1,), generator=g))
    partition = None if choice == 17 else choice  # 0 = single pass
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, hkv=hkv, group=group, d=d,
                                                   width=cdiv(bucket, BLOCK_SIZE) + 1, seed=seed)
    scale = d ** -0.5
    actual = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=bucket, partition_blocks=partition)
    assert_attn_close(actual, _oracle(q, kv_cache, bt, lens, scale), rows=_live(lens))
    for row in range(B):
        if lens[row] == 0:
            assert actual[row].abs().max() == 0


@pytest.mark.parametrize("seed", range(16))
def test_random_batches_launch_choices_agree(seed):
    """Seeded random batches (1-16 rows of 0-5000 tokens, buckets up to 4096
    tokens past the longest row, partitions from 1 page to auto): every launch
    choice of the plan gives the same bits, including the split-mode and
    group-mode kernels on one or two waves."""
    g = torch.Generator().manual_seed(5000 + seed)
    hkv, group, d = _HEAD_CONFIGS[int(torch.randint(len(_HEAD_CONFIGS), (1,), generator=g))]
    B = int(torch.randint(1, 17, (1,), generator=g))
    lens = [0 if int(torch.randint(8, (1,), generator=g)) == 0 else int(torch.randint(1, 5001, (1,), generator=g))
            for _ in range(B)]
    bucket = max(max(lens), 1) + int(torch.randint(0, 4097, (1,), generator=g))
    partition = [None, 1, 2, 4, 8, 16][int(torch.randint(6, (1,), generator=g))]
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, hkv=hkv, group=group, d=d,
                                                   width=cdiv(bucket, BLOCK_SIZE) + 1, seed=seed)
    outs = _modes(q, kv_cache, bt, seq_lens, d ** -0.5, bucket, partition)
    for name, out in outs.items():
        assert torch.equal(out, outs["auto"]), name


# ------------------------------------------- reduce over more than one set of groups

def test_more_splits_than_one_reduce_set():
    """Partition 1 over rows of 20000 and 17001 tokens: 1250 splits, more
    than the 32 x 32 that one reduce pass holds, so the reduce takes the max
    in a pass of its own and adds the sets' group sums in order."""
    lens = [20000, 17001, 0]
    scale = HEAD_DIM ** -0.5
    q, kv_cache, bt, seq_lens = make_decode_inputs(lens, seed=21)
    assert cdiv(max(lens), BLOCK_SIZE) > 32 * 32
    actual = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=max(lens), partition_blocks=1)
    assert_attn_close(actual, _oracle(q, kv_cache, bt, lens, scale), rows=_live(lens))
    assert actual[2].abs().max() == 0


def test_reduce_sets_do_not_change_bits():
    """A 600-token row with partition 1: 38 splits eagerly, 1100 under a wide
    graph bucket (several reduce sets, trailing splits empty); same bits."""
    scale = HEAD_DIM ** -0.5
    q, kv_cache, bt, seq_lens = make_decode_inputs([600], width=1102, seed=22)
    eager = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=600, partition_blocks=1)
    graph = _kernel()(q, kv_cache, bt, seq_lens, scale, max_seq_len=1100 * BLOCK_SIZE, partition_blocks=1)
    assert torch.equal(eager, graph)
    assert_attn_close(graph, _oracle(q, kv_cache, bt, [600], scale))
