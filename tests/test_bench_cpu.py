"""bench.py's measurement arithmetic, on the CPU: the algorithmic flop and byte
counts behind every roofline fraction (checked against brute-force counts, not
the same formula), the choice of the binding roof, the traffic figure read
from the committed counter summary, and the one-GPU contract of the command
line."""

import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)

import bench  # noqa: E402


def _visible_pairs(specs):
    """Brute force: (query, key) pairs a causal prefill with a cached prefix sees."""
    n = 0
    for ctx, q_len in specs:
        for i in range(q_len):
            for k in range(ctx + q_len):
                if k <= ctx + i:
                    n += 1
    return n


@pytest.mark.parametrize("specs", [[(0, 5)], [(3, 4), (0, 1)], [(16, 16), (7, 0), (100, 3)]])
def test_prefill_flops_count_visible_pairs(specs):
    # QK^T and PV: 2 flop per multiply-add, D = 128 each, for every head.
    assert bench.prefill_flops(specs) == _visible_pairs(specs) * bench.H * 2 * 2 * bench.D


def test_baseline_prefill_shapes_flops_and_bytes():
    shapes = bench.PREFILL_SHAPES
    # 8 sequences: each query i of 128 sees the 1024 cached keys and i + 1 new ones.
    pairs = 8 * (128 * 1024 + 128 * 129 // 2)
    assert bench.prefill_flops(shapes["8x(1024+128)"]) == pairs * 28 * 512 == 15_979_249_664
    assert round(bench.prefill_flops(shapes["1x(2048+4096)"]) / 1e9, 3) == 240.548
    # q read + output written (bf16, 28 heads x 128) + K/V of every sequence once per KV head.
    q_out = 2 * 64 * 128 * 28 * 128 * 2
    kv = 64 * 128 * 4 * 128 * 2 * 2
    assert bench.prefill_bytes(shapes["64x128_fresh"]) == q_out + kv == 134_217_728
    mixed = shapes["1x512+63x(1000+1)"]
    assert bench.prefill_bytes(mixed) == 2 * (512 + 63) * 28 * 128 * 2 + (512 + 63 * 1001) * 4 * 128 * 4


def test_binding_roof_picks_the_longer_time_at_peak():
    shapes = bench.PREFILL_SHAPES
    for name, bound in [("1x(2048+4096)", "mfma"), ("8x(1024+128)", "mfma"),
                        ("64x128_fresh", "hbm"), ("1x512+63x(1000+1)", "hbm")]:
        specs = shapes[name]
        flops, nbytes = bench.prefill_flops(specs), bench.prefill_bytes(specs)
        roof = bench.binding_roof(flops, nbytes, 1e-3)
        assert roof["bound"] == bound, name
        t_roof = max(flops / 2.5e15, nbytes / 8e12)
        assert abs(roof["roof_us"] - t_roof * 1e6) < 0.01
        assert abs(roof["frac"] - t_roof / 1e-3) < 1e-4   # a 1 ms launch
    # 64 x 128: 16.78 us at the HBM roof (134.2 MB at 8 TB/s).
    assert bench.binding_roof(bench.prefill_flops(shapes["64x128_fresh"]),
                              bench.prefill_bytes(shapes["64x128_fresh"]), 1.0)["roof_us"] == 16.78


def test_hbm_roof_fraction():
    r = bench.hbm_roof(251_658_240, 44e-6)
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert abs(r["achieved"] - 251_658_240 / 44e-6 / 1e9) < 0.01
    assert abs(r["frac"] - 251_658_240 / 44e-6 / 8e12) < 1e-4


def test_traffic_is_read_from_the_committed_summary():
    t = bench.read_traffic()
    assert t is not None and 251_658_240 < t < 1.1 * 251_658_240


def test_more_than_one_gpu_is_refused_with_a_message():
    p = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert p.returncode == 2
    assert "one GPU" in p.stderr
