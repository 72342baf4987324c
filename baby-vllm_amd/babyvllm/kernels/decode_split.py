"""Flash-decoding split plan for paged decode attention (pure Python, no device needed).

Mirrors the interface and the integer rules of the reference plan,
babyvllm/kernels/decode_split.py:18-79, so callers and tests that import
``decode_split_plan``, ``auto_partition_blocks``, ``grid_fills_gpu``,
``DECODE_PARTITION_ENV`` and ``MIN_PARTITION_BLOCKS`` see the same values.

Rules (each a pure function of its integer arguments):

* ``ctx_blocks`` = pages of the context bucket (``max_seq_len``), or the table
  width when no bucket is given, clamped to ``[1, max_blocks]``.
* "auto": one split whenever ``next_pow2(batch) · n_kv_heads`` work-groups
  already cover every compute unit; otherwise ``auto_partition_blocks(batch)``
  pages per split.
* an explicit page count (argument, else the environment) always splits with
  that many pages; 0 means one split; a negative count raises ``ValueError``.

The page count per split depends only on the batch rounded up to a power of
two, and the split count only on the context bucket. An eager step (live
lengths) and a graph step (bucket) therefore cut every row at the same pages,
which is what lets the decode kernel return identical bits for both.
"""

from __future__ import annotations

import os

# "auto" | "0" (single pass) | a positive page count per split.
DECODE_PARTITION_ENV = "BABYVLLM_DECODE_PARTITION"
# Smallest number of pages a split may hold under "auto".
MIN_PARTITION_BLOCKS = 4


def _ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def _pow2_at_least(n: int) -> int:
    p = 1
    while p < n:
        p <<= 1
    return p


def auto_partition_blocks(batch: int) -> int:
    """Pages per split under "auto": ``max(MIN_PARTITION_BLOCKS, next_pow2(batch))``.

    A function of the batch's power-of-two bucket only, so every live batch
    size inside one graph bucket gets the same partition.
    """
    return max(MIN_PARTITION_BLOCKS, _pow2_at_least(batch))


def grid_fills_gpu(batch: int, n_kv_heads: int, num_sms: int) -> bool:
    """True when one work-group per (bucketed row, KV head) already covers ``num_sms`` units."""
    return _pow2_at_least(batch) * n_kv_heads >= num_sms


def decode_split_plan(
    batch: int,
    n_kv_heads: int,
    block_size: int,
    max_blocks: int,
    max_seq_len: int | None,
    num_sms: int,
    partition_blocks: int | None = None,
) -> tuple[int, int]:
    """``(num_splits, blocks_per_split)`` for one decode launch.

    ``max_seq_len`` is the context bucket the launch is sized for (under a
    captured graph, the bucket, never the live lengths). ``partition_blocks``
    overrides the environment switch and has the same meaning.
    """
    if max_seq_len is None:
        ctx_blocks = max_blocks
    else:
        ctx_blocks = _ceil_div(max_seq_len, block_size)
    ctx_blocks = min(max(ctx_blocks, 1), max_blocks) if max_blocks >= 1 else 1

    if partition_blocks is None:
        setting = os.environ.get(DECODE_PARTITION_ENV, "auto")
        if setting == "auto":
            if grid_fills_gpu(batch, n_kv_heads, num_sms):
                return 1, ctx_blocks
            partition_blocks = auto_partition_blocks(batch)
        else:
            partition_blocks = int(setting)

    if partition_blocks < 0:
        raise ValueError(
            f"{DECODE_PARTITION_ENV} must be 'auto', 0 or a page count, got {partition_blocks}"
        )
    if partition_blocks == 0:
        return 1, ctx_blocks
    return _ceil_div(ctx_blocks, partition_blocks), partition_blocks
