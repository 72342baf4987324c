"""Varlen paged prefill attention: HIP kernel vs the CPU oracle (ports tests/test_paged_prefill.py).

Oracle: oracle.attention.paged_attention_torch (the reference's per-sequence
SDPA loop, babyvllm/layers/attention.py:137-175) in float32 on the CPU, with
the NaN-filled unwritten slots replaced by zeros for the oracle only.
"""

import pytest
import torch

from oracle import attention as oa
from tests._cases import assert_attn_close, build_prefill_case, md_to_cpu, scale_keys_by_position, tuned

_BPW = 1  # tuning knob: prefill column blocks per work-group (bvllm_set_tuning)
_SHORT_GRID = 6  # tuning knob: 1 = short grids on the single key walk instead of the key split

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU"),
]


def _kernel():
    from babyvllm.kernels.paged_prefill import paged_prefill_attention
    return paged_prefill_attention


def _oracle(q, kv_cache, md, group):
    scale = q.shape[-1] ** -0.5
    cache = torch.nan_to_num(kv_cache.float().cpu(), nan=0.0)
    return oa.paged_attention_torch(q.float().cpu(), cache, md_to_cpu(md), scale, group)


CASES = {
    "fresh_prefill": [(0, 128)],
    "fresh_prefill_ragged": [(0, 1), (0, 17), (0, 100), (0, 64)],
    "prefix_hit_aligned": [(32, 5), (48, 77), (16, 2)],
    "prefix_unaligned": [(37, 20), (5, 3), (100, 130)],
    "mixed_prefill_and_decode": [(0, 40), (200, 1), (63, 1), (500, 1)],
    "long_tail_after_prefix": [(1024, 1024)],
    "batch64_fresh": [(0, 128)] * 64,
}


@pytest.mark.parametrize("case", list(CASES))
@pytest.mark.parametrize("hkv,group,d", [(4, 7, 128), (2, 7, 64), (4, 1, 64)])
def test_paged_prefill_matches_oracle(case, hkv, group, d):
    q, kv_cache, md = build_prefill_case(CASES[case], hkv, group, d)
    expected = _oracle(q, kv_cache, md, group)
    actual = _kernel()(q, kv_cache, md, d ** -0.5)
    assert not torch.isnan(actual).any()
    assert_attn_close(actual, expected)


def test_non_contiguous_query_view():
    hkv, group, d = 4, 7, 128
    q, kv_cache, md = build_prefill_case([(16, 33), (0, 70)], hkv, group, d)
    H = hkv * group
    qkv = torch.randn(q.shape[0], (H + 2 * hkv) * d, device="cuda", dtype=q.dtype)
    view = qkv[:, : H * d].view(-1, H, d)
    view.copy_(q)
    assert not view.is_contiguous()
    assert_attn_close(_kernel()(view, kv_cache, md, d ** -0.5), _oracle(q, kv_cache, md, group))


def test_attention_layer_routes_to_the_hip_kernels(monkeypatch):
    from babyvllm.layers.attention import Attention
    from babyvllm.worker.context import set_forward_context
    import babyvllm.kernels.paged_attn as pa
    import babyvllm.kernels.paged_prefill as pp

    hkv, group, d = 4, 7, 128
    q, kv_cache, md = build_prefill_case([(32, 9), (0, 20)], hkv, group, d)
    attn = Attention(hkv * group, d, hkv)
    attn.kv_cache = kv_cache
    calls = []
    real_p, real_d = pp.paged_prefill_attention, pa.paged_decode_attention
    monkeypatch.setattr(pp, "paged_prefill_attention", lambda *a: calls.append("prefill") or real_p(*a))
    monkeypatch.setattr(pa, "paged_decode_attention",
                        lambda *a, **kw: calls.append("decode") or real_d(*a, **kw))
    with set_forward_context(md):
        out = attn(q, q, q)
    assert calls == ["prefill"]
    assert_attn_close(out, _oracle(q, kv_cache, md, group))

    q1, kv1, md1 = build_prefill_case([(40, 1), (7, 1)], hkv, group, d, nan_fill=False)
    attn.kv_cache = kv1
    with set_forward_context(md1):
        out1 = attn(q1, q1, q1)
    assert calls == ["prefill", "decode"]
    assert_attn_close(out1, _oracle(q1, kv1, md1, group))


def test_prefill_backend_switch(monkeypatch):
    """The reference's BABYVLLM_PREFILL_ATTN switch (tests/test_paged_prefill.py:110-130 of
    the reference): "triton" (the default) and "hip" run the HIP prefill kernel; "torch",
    the reference's SDPA loop, is not part of this build and raises instead of falling back."""
    import babyvllm.layers.attention as attn_mod
    import babyvllm.kernels.paged_prefill as pp
    from babyvllm.layers.attention import Attention
    from babyvllm.worker.context import set_forward_context

    assert attn_mod._PREFILL_BACKEND == "triton"
    hkv, group, d = 4, 7, 128
    q, kv_cache, md = build_prefill_case([(32, 9), (0, 20)], hkv, group, d)
    attn = Attention(hkv * group, d, hkv)
    attn.kv_cache = kv_cache
    calls = []
    real = pp.paged_prefill_attention
    monkeypatch.setattr(pp, "paged_prefill_attention", lambda *a: calls.append(1) or real(*a))
    for backend in ("triton", "hip"):
        monkeypatch.setattr(attn_mod, "_PREFILL_BACKEND", backend)
        with set_forward_context(md):
            out = attn(q, q, q)
        assert_attn_close(out, _oracle(q, kv_cache, md, group))
    assert calls == [1, 1]
    monkeypatch.setattr(attn_mod, "_PREFILL_BACKEND", "torch")
    with set_forward_context(md), pytest.raises(RuntimeError, match="BABYVLLM_PREFILL_ATTN"):
        attn(q, q, q)
    assert calls == [1, 1]


def test_empty_step_returns_empty():
    q, kv_cache, md = build_prefill_case([(0, 3)], 4, 7, 128)
    out = _kernel()(q[:0], kv_cache, md, 0.1)
    assert out.shape == (0, 28, 128)


# ---------------------------------------------------- BASELINE config 4 shapes

@pytest.mark.parametrize("name,specs", [
    ("64x128_fresh", [(0, 128)] * 64),
    ("8x(1024+128)", [(1024, 128)] * 8),
    ("1x(2048+4096)", [(2048, 4096)]),
    ("1x512+63x(1000+1)", [(0, 512)] + [(1000, 1)] * 63),
])
def test_baseline_prefill_configs(name, specs):
    q, kv_cache, md = build_prefill_case(specs, 4, 7, 128, seed=len(specs))
    actual = _kernel()(q, kv_cache, md, 128 ** -0.5)
    assert_attn_close(actual, _oracle(q, kv_cache, md, 7))


# ------------------------------------- single-query sequences on the decode kernel

SINGLE_MIX = [(0, 40), (200, 1), (63, 1), (0, 1), (500, 1), (16, 16), (31, 1)]


@pytest.mark.parametrize("hkv,group,d", [(4, 7, 128), (2, 7, 64)])
def test_single_query_rows_whatever_the_host_hint(hkv, group, d, monkeypatch):
    """Decode rows of a mixed step give oracle results whether the host passes
    their count (decode kernel), -1 (decode kernel, rows found on the device)
    or 0 (everything on the prefill kernel); the first two give the same bits."""
    import babyvllm.kernels.paged_prefill as pp

    q, kv_cache, md = build_prefill_case(SINGLE_MIX, hkv, group, d, seed=7)
    expected = _oracle(q, kv_cache, md, group)
    assert pp._single_query_seqs(md, len(SINGLE_MIX)) == 5
    counted = _kernel()(q, kv_cache, md, d ** -0.5)
    monkeypatch.setattr(pp, "_single_query_seqs", lambda md, n: -1)
    unknown = _kernel()(q, kv_cache, md, d ** -0.5)
    monkeypatch.setattr(pp, "_single_query_seqs", lambda md, n: 0)
    prefill_only = _kernel()(q, kv_cache, md, d ** -0.5)
    assert torch.equal(counted, unknown)
    for out in (counted, prefill_only):
        assert not torch.isnan(out).any()
        assert_attn_close(out, expected)


def test_step_of_only_single_query_rows():
    q, kv_cache, md = build_prefill_case([(40, 1), (7, 1), (0, 1), (1000, 1)], 4, 7, 128, seed=3)
    actual = _kernel()(q, kv_cache, md, 128 ** -0.5)
    assert_attn_close(actual, _oracle(q, kv_cache, md, 7))


def test_single_query_row_matches_paged_decode():
    """A one-token sequence of a prefill step is the decode of that token."""
    from babyvllm.kernels.paged_attn import paged_decode_attention

    specs = [(300, 1), (0, 50), (129, 1)]
    q, kv_cache, md = build_prefill_case(specs, 4, 7, 128, seed=11, nan_fill=False)
    out = _kernel()(q, kv_cache, md, 128 ** -0.5)
    rows = [0, 51]
    dec = paged_decode_attention(q[rows].contiguous(), kv_cache, md.block_tables[[0, 2]].contiguous(),
                                 md.seq_lens[[0, 2]].contiguous(), 128 ** -0.5, partition_blocks=0)
    assert torch.equal(out[rows], dec)


# ------------------------------------------- work-group mapping (query-block list)

def _many_seqs(n, seed):
    g = torch.Generator().manual_seed(seed)
    specs = []
    for i in range(n):
        kind = i % 4
        ctx = int(torch.randint(0, 200, (1,), generator=g))
        q_len = [1, 2, int(torch.randint(3, 40, (1,), generator=g)), 0][kind]
        specs.append((ctx, q_len))
    return specs


@pytest.mark.parametrize("n_seqs", [63, 64, 65, 300])
def test_many_sequences_of_mixed_lengths(n_seqs):
    """Covers the block-list scan across several 64-sequence slices, empty
    sequences and single-query sequences between prefill ones."""
    specs = _many_seqs(n_seqs, seed=n_seqs)
    q, kv_cache, md = build_prefill_case(specs, 4, 7, 128, seed=n_seqs)
    actual = _kernel()(q, kv_cache, md, 128 ** -0.5)
    assert not torch.isnan(actual).any()
    assert_attn_close(actual, _oracle(q, kv_cache, md, 7))


@pytest.mark.parametrize("hkv,group,d", [(8, 2, 128), (1, 8, 128), (3, 2, 64), (16, 1, 64),
                                         (2, 3, 128), (1, 5, 64), (2, 6, 128), (1, 16, 64)])
def test_kv_head_counts_and_xcd_groups(hkv, group, d):
    """Group sizes that do not divide 16 put the heads of one query in two
    16-column tiles (and the queries of one tile in two work-groups)."""
    specs = [(0, 70), (130, 1), (33, 45), (7, 1), (0, 16)]
    q, kv_cache, md = build_prefill_case(specs, hkv, group, d, seed=hkv)
    actual = _kernel()(q, kv_cache, md, d ** -0.5)
    assert_attn_close(actual, _oracle(q, kv_cache, md, group))


@pytest.mark.parametrize("growth", [128.0, 24.0])
@pytest.mark.parametrize("hkv,group,d", [(4, 7, 128), (2, 7, 64)])
def test_scores_rising_along_the_sequence(growth, hkv, group, d):
    """Key norms growing with position (factor 1 + p / growth): each row's
    scores keep exceeding the running max by more than 8 in log2 units, so the
    kernel raises its max, rescales its accumulators and forms P again many
    times; growth 24 makes the softmax nearly one-hot at the far end."""
    specs = [(0, 300), (500, 200), (37, 1), (1000, 64), (0, 5)]
    q, kv_cache, md = build_prefill_case(specs, hkv, group, d, seed=11)
    scale_keys_by_position(kv_cache, md.block_tables, md.seq_lens_cpu, lambda p: 1.0 + p / growth)
    actual = _kernel()(q, kv_cache, md, d ** -0.5)
    assert_attn_close(actual, _oracle(q, kv_cache, md, group))


@pytest.mark.parametrize("bpw", [2, 3, 4, 7, 64])
@pytest.mark.parametrize("hkv,group,d", [(4, 7, 128), (8, 3, 64), (1, 16, 128)])
def test_blocks_per_work_group_do_not_change_bits(bpw, hkv, group, d):
    """When every sequence fits two 64-key tiles (table width ≤ 8 pages), a
    work-group may compute several column blocks of one (sequence, KV head)
    over tiles staged once; any number of blocks per work-group gives the
    bits of one block per work-group. (Both head configurations give a grid
    of at least two work-groups per CU, where the override applies.)"""
    specs = [(0, 128)] * (20 if hkv > 1 else 40) + [(0, 77), (37, 90), (100, 28), (0, 1), (5, 3), (64, 64),
                                                    (127, 1)]
    q, kv_cache, md = build_prefill_case(specs, hkv, group, d, seed=bpw)
    assert md.block_tables.shape[1] <= 8
    with tuned(_BPW, 1):
        one = _kernel()(q, kv_cache, md, d ** -0.5)
    with tuned(_BPW, bpw):
        many = _kernel()(q, kv_cache, md, d ** -0.5)
    assert torch.equal(one, many)
    assert_attn_close(many, _oracle(q, kv_cache, md, group))


def test_scores_rising_with_blocks_per_work_group():
    """The rescale path on the multi-block kernel: every sequence within two
    64-key tiles, a grid large enough for several blocks per work-group, key
    norms growing with position; same bits as one block per work-group."""
    specs = [(0, 128)] * 40 + [(60, 60)] * 10 + [(5, 1)]
    q, kv_cache, md = build_prefill_case(specs, 4, 7, 128, seed=17)
    assert md.block_tables.shape[1] <= 8
    scale_keys_by_position(kv_cache, md.block_tables, md.seq_lens_cpu, lambda p: 1.0 + p / 12.0)
    many = _kernel()(q, kv_cache, md, 128 ** -0.5)
    with tuned(_BPW, 1):
        one = _kernel()(q, kv_cache, md, 128 ** -0.5)
    assert torch.equal(one, many)
    assert_attn_close(many, _oracle(q, kv_cache, md, 7))


# ------------------------------------------------------- seeded random batches

_HEAD_CONFIGS = [(4, 7, 128), (2, 7, 64), (1, 16, 128), (8, 4, 128), (4, 1, 64), (2, 3, 64)]


@pytest.mark.parametrize("seed", range(24))
def test_random_varlen_batches(seed):
    """Seeded random steps: 1-12 sequences, each with a cached prefix of 0-700
    tokens and 0-300 new queries (a quarter of them single-query rows), over
    random head configurations."""
    g = torch.Generator().manual_seed(1000 + seed)
    hkv, group, d = _HEAD_CONFIGS[int(torch.randint(len(_HEAD_CONFIGS), (1,), generator=g))]
    specs = []
    for _ in range(int(torch.randint(1, 13, (1,), generator=g))):
        ctx = int(torch.randint(0, 701, (1,), generator=g))
        kind = int(torch.randint(4, (1,), generator=g))
        q_len = 1 if kind == 0 else int(torch.randint(0, 301, (1,), generator=g))
        specs.append((ctx, q_len))
    if max(n for _, n in specs) == 0:
        specs[0] = (specs[0][0], 1)
    q, kv_cache, md = build_prefill_case(specs, hkv, group, d, seed=seed)
    actual = _kernel()(q, kv_cache, md, d ** -0.5)
    assert_attn_close(actual, _oracle(q, kv_cache, md, group))


@pytest.mark.parametrize("seed", range(8))
def test_random_short_batches_against_one_block_per_work_group(seed):
    """Seeded random steps of 24-80 sequences that all fit two 64-key tiles,
    where the host gives a work-group several column blocks whenever the grid
    allows it: within tolerance of the oracle and bit-equal to one block per
    work-group."""
    g = torch.Generator().manual_seed(2000 + seed)
    hkv, group, d = _HEAD_CONFIGS[seed % len(_HEAD_CONFIGS)]
    specs = []
    for _ in range(int(torch.randint(24, 81, (1,), generator=g))):
        q_len = int(torch.randint(1, 129, (1,), generator=g))
        ctx = int(torch.randint(0, 129 - q_len, (1,), generator=g))
        specs.append((ctx, q_len))
    q, kv_cache, md = build_prefill_case(specs, hkv, group, d, seed=seed)
    assert md.block_tables.shape[1] <= 8
    auto = _kernel()(q, kv_cache, md, d ** -0.5)
    with tuned(_BPW, 1):
        one = _kernel()(q, kv_cache, md, d ** -0.5)
    assert torch.equal(auto, one)
    assert_attn_close(auto, _oracle(q, kv_cache, md, group))


# ------------------------------------------------- beyond the oracle's sizes

@pytest.mark.parametrize("hkv,group,d", [(4, 7, 128), (2, 7, 64)])
def test_long_sequence_with_one_key_repeated(hkv, group, d):
    """1 x (8192 cached + 8192 new) tokens, every key the same vector: each
    query's scores are equal, so its output is the mean of the values it sees
    (keys 0 .. ctx + i), a closed form checked at a size where the CPU oracle
    would take minutes. The scores are not zero, so the QKᵀ path and the max
    reference still run."""
    ctx, n = 8192, 8192
    q, kv_cache, md = build_prefill_case([(ctx, n)], hkv, group, d, seed=5, nan_fill=False)
    key = torch.randn(hkv, d, device="cuda", dtype=torch.bfloat16)
    kv_cache[0] = key
    pages = md.block_tables[0].long()
    v = kv_cache[1, pages].reshape(-1, hkv, d)[: ctx + n].double()  # [keys, Hkv, D] in order
    prefix_mean = v.cumsum(0) / torch.arange(1, ctx + n + 1, device="cuda", dtype=torch.float64)[:, None, None]
    expected = prefix_mean[ctx:].repeat_interleave(group, dim=1)  # [n, H, D]
    actual = _kernel()(q, kv_cache, md, d ** -0.5)
    assert_attn_close(actual, expected)


# ------------------------------------------ in-work-group key split (short grids)

KEY_SPLIT_CASES = {
    "8x(1024+128)": [(1024, 128)] * 8,
    "one tile, both halves": [(0, 40), (10, 50)],
    "first half only": [(0, 20), (5, 9), (0, 1)],
    "odd tile counts": [(100, 91), (0, 193), (311, 2)],
    "long prefix few queries": [(3000, 5), (1500, 17)],
}


@pytest.mark.parametrize("name", list(KEY_SPLIT_CASES))
@pytest.mark.parametrize("hkv,group,d", [(4, 7, 128), (2, 7, 64), (1, 16, 128)])
def test_short_grid_kernels_match_the_oracle(name, hkv, group, d):
    """Grids too small for two work-groups per CU at 128 columns run 64-column
    work-groups whose two waves per column group take the two halves of every
    key tile and merge at the end; the single key walk (one wave per column
    tile over every key) stays behind a tuning knob. Both within tolerance of
    the oracle, with edge cases: a sequence inside one tile, columns whose keys
    all lie in a first half, odd tile counts, long prefixes with few queries."""
    specs = KEY_SPLIT_CASES[name]
    q, kv_cache, md = build_prefill_case(specs, hkv, group, d, seed=len(specs) + d)
    expected = _oracle(q, kv_cache, md, group)
    split = _kernel()(q, kv_cache, md, d ** -0.5)
    with tuned(_SHORT_GRID, 1):
        walk = _kernel()(q, kv_cache, md, d ** -0.5)
    for out in (split, walk):
        assert not torch.isnan(out).any()
        assert_attn_close(out, expected)


@pytest.mark.parametrize("growth", [6.0, 40.0])
def test_key_split_with_rising_scores(growth):
    """The rescale path on both halves: key norms growing with position, so the
    two waves of a column group raise their reference maxima at different tiles
    and the merge rescales the two partial states by different factors."""
    specs = [(700, 60), (0, 300), (129, 2), (64, 64)]
    q, kv_cache, md = build_prefill_case(specs, 4, 7, 128, seed=int(growth))
    scale_keys_by_position(kv_cache, md.block_tables, md.seq_lens_cpu, lambda p: 1.0 + p / growth)
    expected = _oracle(q, kv_cache, md, 7)
    assert_attn_close(_kernel()(q, kv_cache, md, 128 ** -0.5), expected)
    with tuned(_SHORT_GRID, 1):
        assert_attn_close(_kernel()(q, kv_cache, md, 128 ** -0.5), expected)


# ------------------------------------------ GQA groups above 16 query heads per KV head

# The reference's prefill takes any H % Hkv == 0 (babyvllm/kernels/paged_prefill.py:114-115):
# fresh, prefix and mixed steps (the decode rows of a mixed step run on the decode
# work-groups, cut into 16-head column groups).
WIDE_GROUP_CASES = {
    "fresh": [(0, 128), (0, 17), (0, 1)],
    "prefix": [(37, 20), (100, 130), (16, 2)],
    "mixed": [(0, 40), (200, 1), (63, 1), (500, 1), (16, 16)],
    "short grid": [(1024, 128)] * 2,
}


@pytest.mark.parametrize("name", list(WIDE_GROUP_CASES))
@pytest.mark.parametrize("hkv,group,d", [(1, 32, 128), (1, 64, 128), (2, 24, 64), (1, 17, 64)])
def test_gqa_groups_above_16(name, hkv, group, d):
    specs = WIDE_GROUP_CASES[name]
    q, kv_cache, md = build_prefill_case(specs, hkv, group, d, seed=group + len(specs))
    expected = _oracle(q, kv_cache, md, group)
    actual = _kernel()(q, kv_cache, md, d ** -0.5)
    assert not torch.isnan(actual).any()
    assert_attn_close(actual, expected)
    with tuned(_SHORT_GRID, 1):
        walk = _kernel()(q, kv_cache, md, d ** -0.5)
    assert_attn_close(walk, expected)
