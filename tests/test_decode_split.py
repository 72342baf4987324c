"""The flash-decoding split plan (pure Python, CPU).

The plan's integer rules are part of the drop-in boundary (they fix where a
row is cut into splits, so the output bits of eager and graph launches), so
they are checked against known answers — the reference's, stated for a
132-SM H100 (tests/test_decode_split.py:12-109 of the reference), and this
build's at MI355X's 256 compute units for the BASELINE configurations — and
against properties that any correct plan has: the splits tile the context
exactly, the pages per split depend only on the batch's power-of-two bucket,
and every live batch gets the plan of its graph bucket.
"""

import pytest

from babyvllm.kernels.decode_split import (
    DECODE_PARTITION_ENV,
    MIN_PARTITION_BLOCKS,
    auto_partition_blocks,
    decode_split_plan,
    grid_fills_gpu,
)

BLOCK = 16
WIDTH_2048 = 129  # table width of the 2048-token graph bucket

# (batch, kv_heads, compute units, table width, context bucket, override, env, expected plan)
KNOWN = [
    # H100 (132 SMs), the reference's answers
    (1, 4, 132, WIDTH_2048, 2048, None, None, (32, 4)),
    (2, 4, 132, WIDTH_2048, 2048, None, None, (32, 4)),
    (4, 4, 132, WIDTH_2048, 2048, None, None, (32, 4)),
    (8, 4, 132, WIDTH_2048, 2048, None, None, (16, 8)),
    (16, 4, 132, WIDTH_2048, 2048, None, None, (8, 16)),
    (32, 4, 132, WIDTH_2048, 2048, None, None, (4, 32)),
    (64, 4, 132, WIDTH_2048, 2048, None, None, (1, 128)),
    (64, 4, 132, WIDTH_2048, 256, None, None, (1, 16)),
    (1, 4, 132, WIDTH_2048, 64, None, None, (1, 4)),
    (1, 4, 132, WIDTH_2048, None, None, None, (33, 4)),
    (1, 4, 132, WIDTH_2048, 8192, None, None, (33, 4)),
    (1, 4, 132, WIDTH_2048, 2048, None, "0", (1, 128)),
    (64, 4, 132, WIDTH_2048, 2048, None, "32", (4, 32)),
    (1, 4, 132, WIDTH_2048, 2048, None, "8", (16, 8)),
    (1, 4, 132, WIDTH_2048, 2048, 7, None, (19, 7)),
    (1, 4, 132, WIDTH_2048, 2048, 16, "0", (8, 16)),
    (64, 3, 132, WIDTH_2048, 2048, None, None, (1, 128)),
    # MI355X (256 CUs), the BASELINE configurations
    (64, 4, 256, 121, 1920, None, None, (1, 120)),
    (8, 4, 256, 121, 1920, None, None, (15, 8)),
    (1, 4, 256, 2049, 32768, None, None, (512, 4)),
    (32, 4, 256, WIDTH_2048, 2048, None, None, (4, 32)),
    (64, 3, 256, WIDTH_2048, 2048, None, None, (2, 64)),
    (8, 2, 256, 32, 512, None, None, (4, 8)),
]


@pytest.mark.parametrize("batch, kv, units, width, ctx, override, env, expect", KNOWN)
def test_known_plans(batch, kv, units, width, ctx, override, env, expect, monkeypatch):
    if env is None:
        monkeypatch.delenv(DECODE_PARTITION_ENV, raising=False)
    else:
        monkeypatch.setenv(DECODE_PARTITION_ENV, env)
    assert decode_split_plan(batch, kv, BLOCK, width, ctx, units, override) == expect


@pytest.mark.parametrize("units", [132, 256])
@pytest.mark.parametrize("kv", [1, 2, 4, 8])
def test_every_plan_tiles_the_context_exactly(units, kv, monkeypatch):
    """Splits of `per` pages cover the bucket's pages with the last one non-empty."""
    monkeypatch.delenv(DECODE_PARTITION_ENV, raising=False)
    for batch in range(1, 70):
        for ctx in (1, 15, 16, 17, 100, 128, 129, 1000, 2048, 4095):
            width = ctx // BLOCK + 2
            splits, per = decode_split_plan(batch, kv, BLOCK, width, ctx, units)
            pages = -(-ctx // BLOCK)
            assert splits >= 1 and per >= 1
            if splits == 1:
                assert per >= pages or per >= MIN_PARTITION_BLOCKS
            assert (splits - 1) * per < pages <= splits * per


def test_single_pass_when_the_bucketed_grid_fills_the_chip(monkeypatch):
    """A grid of bucket · kv_heads work-groups that covers every CU takes the
    whole context in one pass; otherwise splits follow the bucket's size."""
    monkeypatch.delenv(DECODE_PARTITION_ENV, raising=False)
    for units in (132, 256, 304):
        for kv in (1, 2, 4, 8):
            for batch in range(1, 130):
                bucket = 1 << (batch - 1).bit_length()
                splits, per = decode_split_plan(batch, kv, BLOCK, WIDTH_2048, 2048, units)
                fills = bucket * kv >= units
                assert grid_fills_gpu(batch, kv, units) == fills
                if fills:
                    assert (splits, per) == (1, 2048 // BLOCK)
                else:
                    assert per == max(MIN_PARTITION_BLOCKS, bucket)


def test_pages_per_split_follow_the_bucket_and_never_drop_below_the_floor():
    previous = 0
    for batch in range(1, 200):
        per = auto_partition_blocks(batch)
        assert per >= MIN_PARTITION_BLOCKS and per >= previous
        assert per == max(MIN_PARTITION_BLOCKS, 1 << (batch - 1).bit_length())
        previous = per


@pytest.mark.parametrize("units", [132, 256])
def test_live_batches_share_their_graph_bucket_plan(units, monkeypatch):
    """Eager decode plans from the live batch, the captured graph from its bucket:
    for every live batch in (bucket/2, bucket] the plans must cut rows at the
    same pages (so the outputs have the same bits)."""
    monkeypatch.delenv(DECODE_PARTITION_ENV, raising=False)
    for bucket in (1, 2, 4, 8, 16, 32, 64):
        for live in range(bucket // 2 + 1, bucket + 1):
            for kv in (2, 4):
                _, per_live = decode_split_plan(live, kv, BLOCK, WIDTH_2048, 2048, units)
                _, per_graph = decode_split_plan(bucket, kv, BLOCK, WIDTH_2048, 2048, units)
                assert per_live == per_graph


def test_the_bucket_only_adds_empty_splits(monkeypatch):
    """A longer context bucket keeps the pages per split and only appends splits."""
    monkeypatch.delenv(DECODE_PARTITION_ENV, raising=False)
    for batch in (1, 3, 8, 20):
        short = decode_split_plan(batch, 4, BLOCK, 2049, 600, 256)
        long = decode_split_plan(batch, 4, BLOCK, 2049, 32768, 256)
        assert short[1] == long[1] and long[0] >= short[0]


def test_invalid_partitions_are_rejected(monkeypatch):
    monkeypatch.setenv(DECODE_PARTITION_ENV, "-3")
    with pytest.raises(ValueError):
        decode_split_plan(1, 4, BLOCK, WIDTH_2048, 2048, 132)
    monkeypatch.delenv(DECODE_PARTITION_ENV)
    with pytest.raises(ValueError):
        decode_split_plan(1, 4, BLOCK, WIDTH_2048, 2048, 132, partition_blocks=-1)
