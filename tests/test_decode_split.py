"""Flash-decoding split plan: known answers (pure Python, CPU).

Ports the reference's plan tests (tests/test_decode_split.py:12-109), whose
known answers are stated for 132 SMs, and adds the answers at MI355X's 256
compute units for the BASELINE configurations.
"""

import pytest

from babyvllm.kernels.decode_split import (
    DECODE_PARTITION_ENV,
    MIN_PARTITION_BLOCKS,
    auto_partition_blocks,
    decode_split_plan,
    grid_fills_gpu,
)

H100_SMS = 132
MI355X_CUS = 256
BLOCK = 16
MAX_BLOCKS = 129  # table width of the 2048 graph bucket: 2048 / 16 + 1
GRAPH_BATCHES = [1, 2, 4, 8, 16, 32, 64]


@pytest.fixture(autouse=True)
def _auto(monkeypatch):
    monkeypatch.delenv(DECODE_PARTITION_ENV, raising=False)


def plan(batch, ctx, n_kv=4, sms=H100_SMS, **kw):
    return decode_split_plan(batch, n_kv, BLOCK, MAX_BLOCKS, ctx, sms, **kw)


def test_batch_one_long_context_splits_at_the_floor():
    assert plan(1, 2048) == (2048 // BLOCK // MIN_PARTITION_BLOCKS, MIN_PARTITION_BLOCKS)


@pytest.mark.parametrize("batch, per", [(1, 4), (2, 4), (4, 4), (8, 8), (16, 16), (32, 32)])
def test_partition_grows_with_the_batch_bucket(batch, per):
    splits, got = plan(batch, 2048)
    assert got == per
    assert splits == 128 // per


def test_full_batch_keeps_the_single_pass_kernel():
    assert plan(64, 2048) == (1, 128)
    assert plan(64, 256) == (1, 16)


def test_threshold_uses_the_batch_bucket():
    assert not grid_fills_gpu(32, 4, H100_SMS)
    assert grid_fills_gpu(33, 4, H100_SMS)


@pytest.mark.parametrize("bucket", GRAPH_BATCHES)
def test_eager_batch_and_its_graph_bucket_get_the_same_plan(bucket):
    lo = bucket // 2 + 1 if bucket > 1 else 1
    for live in range(lo, bucket + 1):
        assert auto_partition_blocks(live) == auto_partition_blocks(bucket)
        for sms in (H100_SMS, MI355X_CUS):
            assert grid_fills_gpu(live, 4, sms) == grid_fills_gpu(bucket, 4, sms)
            assert grid_fills_gpu(live, 2, sms) == grid_fills_gpu(bucket, 2, sms)


@pytest.mark.parametrize("batch", [1, 2, 4, 8, 16, 32])
@pytest.mark.parametrize("ctx", [17, 128, 129, 256, 2048])
def test_partition_does_not_depend_on_the_context(batch, ctx):
    splits, per = plan(batch, ctx)
    assert per == auto_partition_blocks(batch)
    ctx_blocks = -(-ctx // BLOCK)
    assert (splits - 1) * per < ctx_blocks <= splits * per


def test_context_within_one_partition_is_one_split():
    assert plan(1, MIN_PARTITION_BLOCKS * BLOCK) == (1, MIN_PARTITION_BLOCKS)


def test_no_bucket_uses_the_block_table_width():
    assert decode_split_plan(1, 4, BLOCK, MAX_BLOCKS, None, H100_SMS) == (
        -(-MAX_BLOCKS // MIN_PARTITION_BLOCKS), MIN_PARTITION_BLOCKS,
    )


def test_bucket_wider_than_table_is_clamped():
    assert plan(1, 8192) == (-(-MAX_BLOCKS // MIN_PARTITION_BLOCKS), MIN_PARTITION_BLOCKS)


def test_env_zero_is_the_single_pass_kernel(monkeypatch):
    monkeypatch.setenv(DECODE_PARTITION_ENV, "0")
    assert plan(1, 2048) == (1, 128)


def test_env_count_forces_splits_even_at_full_batch(monkeypatch):
    monkeypatch.setenv(DECODE_PARTITION_ENV, "32")
    assert plan(64, 2048) == (4, 32)
    monkeypatch.setenv(DECODE_PARTITION_ENV, "8")
    assert plan(1, 2048) == (16, 8)


def test_partition_that_does_not_divide_rounds_up():
    assert plan(1, 2048, partition_blocks=7) == (19, 7)


def test_explicit_partition_overrides_env(monkeypatch):
    monkeypatch.setenv(DECODE_PARTITION_ENV, "0")
    assert plan(1, 2048, partition_blocks=16) == (8, 16)


def test_negative_partition_is_rejected(monkeypatch):
    monkeypatch.setenv(DECODE_PARTITION_ENV, "-3")
    with pytest.raises(ValueError):
        plan(1, 2048)


# Known answers at 256 compute units (MI355X) for the BASELINE decode configs.
@pytest.mark.parametrize("batch, ctx, width, expect", [
    (64, 1920, 121, (1, 120)),      # 64·4 = 256 work-groups fill the chip: single pass
    (8, 1920, 121, (15, 8)),        # 8 pages per split
    (1, 32768, 2049, (512, 4)),     # the floor: 4 pages per split
    (32, 2048, 129, (4, 32)),       # 32·4 = 128 < 256: splits on MI355X (not on 132 SMs)
    (8, 512, 32, (4, 8)),           # the 0.5B config: 8 rows, 2 KV heads, 512-token bucket
])
def test_mi355x_plans_for_the_baseline_configs(batch, ctx, width, expect):
    n_kv = 2 if ctx == 512 else 4
    assert decode_split_plan(batch, n_kv, BLOCK, width, ctx, MI355X_CUS) == expect


def test_132_and_256_units_differ_only_in_the_fill_threshold():
    # 64 rows × 3 KV heads = 192 work-groups: enough for 132 SMs, not for 256 CUs.
    assert plan(64, 2048, n_kv=3, sms=H100_SMS) == (1, 128)
    assert plan(64, 2048, n_kv=3, sms=MI355X_CUS) == (2, 64)
    # With 4 KV heads the bucketed grid is 128 or 256: both counts agree.
    for b in GRAPH_BATCHES:
        assert plan(b, 2048, sms=H100_SMS) == plan(b, 2048, sms=MI355X_CUS)
