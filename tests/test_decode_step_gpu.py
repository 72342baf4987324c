"""The decode step's other kernels on the GPU: greedy argmax, residual add +
RMSNorm and SiLU·mul (ports tests/test_argmax_kernel.py and covers
babyvllm/kernels/layernorm.py, activation.py).

Oracle: oracle/decode_step.py on the CPU. Argmax and the residual update are
bit-exact; normalised and activated outputs are within one bf16 ulp of the
oracle (the fp32 sums of squares and exp differ from torch's in the last bits,
which moves a value across a bf16 rounding boundary only rarely).
"""

import pytest
import torch

from oracle import decode_step as ds

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU"),
]


def _argmax():
    from babyvllm.kernels.argmax import greedy_argmax
    return greedy_argmax


def _ulps(a, b):
    """Distance in bf16 ulps of two bf16 tensors (same sign assumed near equality)."""
    ai = a.view(torch.int16).to(torch.int32)
    bi = b.view(torch.int16).to(torch.int32)
    ai = torch.where(ai < 0, -32768 - ai, ai)
    bi = torch.where(bi < 0, -32768 - bi, bi)
    return (ai - bi).abs()


# --------------------------------------------------------------------- argmax

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,vocab", [(1, 151936), (64, 152064), (7, 4097), (3, 100)])
def test_matches_torch_argmax(rows, vocab, dtype):
    g = torch.Generator(device="cuda").manual_seed(rows + vocab)
    x = torch.randn(rows, vocab, device="cuda", dtype=dtype, generator=g) * 4
    out = torch.empty(rows, dtype=torch.int64, device="cuda")
    _argmax()(x, out)
    assert torch.equal(out, x.argmax(-1))
    assert torch.equal(out.cpu(), ds.greedy_argmax(x.cpu()))


def test_ties_go_to_the_lowest_index_across_chunks():
    vocab = 20000
    x = torch.zeros(6, vocab, device="cuda", dtype=torch.bfloat16)
    x[0, [5, 9000, 19999]] = 3.0            # first chunk wins
    x[1, [8191, 8192]] = 3.0                # straddles the kernel's chunk boundary
    x[2, [12000, 8200]] = 3.0               # later chunk listed first
    x[3, 19999] = 3.0                       # last, partial chunk
    x[5, [4095, 4096]] = 3.0                # straddles the reference's block boundary
    # row 4 all equal: index 0
    out = torch.empty(6, dtype=torch.int64, device="cuda")
    _argmax()(x, out, block=4096)
    assert out.tolist() == [5, 8191, 8200, 19999, 0, 4095]
    assert torch.equal(out, x.argmax(-1))


def test_row_slice_of_a_larger_buffer():
    buf = torch.randn(64, 152064, device="cuda", dtype=torch.bfloat16)
    out = torch.full((64,), -1, dtype=torch.int64, device="cuda")
    _argmax()(buf[:5], out[:5])
    assert torch.equal(out[:5], buf[:5].argmax(-1))
    assert (out[5:] == -1).all()


def test_column_slice_and_unaligned_rows():
    buf = torch.randn(9, 5003, device="cuda", dtype=torch.bfloat16)
    view = buf[:, 1:5001]                    # row stride 5003, unaligned start
    out = torch.empty(9, dtype=torch.int64, device="cuda")
    _argmax()(view, out)
    assert torch.equal(out, view.argmax(-1))


def test_nan_is_the_maximum_and_the_first_nan_wins():
    x = torch.randn(3, 9000, device="cuda", dtype=torch.float32)
    x[0, [8500, 17]] = float("nan")
    x[1, 8999] = float("nan")
    out = torch.empty(3, dtype=torch.int64, device="cuda")
    _argmax()(x, out)
    assert out.tolist()[:2] == [17, 8999]
    assert torch.equal(out.cpu(), ds.greedy_argmax(x.cpu()))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_ties_nan_and_infinities_across_batches(dtype):
    """Full-width rows: ties in different chunks go to the lowest column, a NaN
    in a later chunk beats a larger number earlier, a negative NaN counts as
    NaN, an all -inf row gives 0, -0.0 ties +0.0, and maxima straddling
    power-of-two column boundaries resolve to the lower column."""
    vocab = 152064
    x = torch.randn(8, vocab, device="cuda", dtype=dtype)
    x[0, [140000, 70000, 65535]] = 50.0                 # three chunks; the first wins
    x[1, 3] = 60.0
    x[1, 150000] = float("nan")                         # NaN in the last chunk beats 60
    x[2, [65536, 100]] = -float("nan")                  # negative NaNs: the first wins
    x[3] = -float("inf")                                # all -inf: column 0
    x[4] = -1.0
    x[4, [99999, 7]] = -0.0
    x[4, 50000] = 0.0                                   # -0.0 ties +0.0: the lowest column
    x[5, vocab - 1] = 70.0                              # last column
    x[6, [32767, 32768]] = 80.0
    x[7, [65535, 65536]] = 90.0
    out = torch.empty(8, dtype=torch.int64, device="cuda")
    _argmax()(x, out)
    assert out.tolist() == [65535, 150000, 100, 0, 7, vocab - 1, 32767, 65535]
    assert torch.equal(out.cpu(), ds.greedy_argmax(x.cpu()))


def test_fp32_ties_and_nan_around_the_chunk_boundaries():
    """fp32 rows are cut into 2,048-column chunks (bf16 rows into 4,096): ties
    straddling those boundaries go to the lower column, -0.0 ties +0.0 across
    chunks, and a NaN in the partial last chunk beats every number."""
    vocab = 3 * 2048 + 40                              # a partial last chunk
    x = torch.randn(6, vocab, device="cuda", dtype=torch.float32)
    x[0, [2047, 2048]] = 9.0                           # straddles the first boundary
    x[1, [4100, 4095]] = 9.0                           # later chunk first in the list
    x[2] = -1.0
    x[2, 5000] = 0.0
    x[2, 300] = -0.0                                   # -0.0 ties +0.0, lower column
    x[3, vocab - 1] = float("nan")                     # NaN in the partial chunk
    x[3, 10] = 100.0
    x[4] = -float("inf")
    x[4, vocab - 3] = -1e30                            # the only finite value, last chunk
    x[5, [6143, 6144, 6150]] = 7.0                     # the last full chunk and the partial one
    out = torch.empty(6, dtype=torch.int64, device="cuda")
    _argmax()(x, out)
    assert out.tolist() == [2047, 4095, 300, vocab - 1, vocab - 3, 6143]
    assert torch.equal(out.cpu(), ds.greedy_argmax(x.cpu()))


def test_more_rows_than_one_launch_takes():
    """Rows beyond the 65,535 of one launch's grid continue in a second launch."""
    rows, vocab = 70_000, 24
    g = torch.Generator().manual_seed(5)
    x = torch.randn(rows, vocab, generator=g).to(torch.bfloat16)
    x[65_535, [3, 17]] = 50.0                           # first row of the second launch
    x[65_534, 23] = float("nan")                        # last row of the first launch
    xd = x.to("cuda")
    out = torch.full((rows,), -1, dtype=torch.int64, device="cuda")
    _argmax()(xd, out)
    exp = ds.greedy_argmax(x)
    assert int(exp[65_535]) == 3 and int(exp[65_534]) == 23
    assert torch.equal(out.cpu(), exp)


def test_unaligned_rows_take_the_two_stage_path_with_the_same_answers():
    vocab = 20001                                       # 40,002 bytes per row: not 16-byte aligned
    x = torch.zeros(4, vocab, device="cuda", dtype=torch.bfloat16)
    x[0, [8191, 8192]] = 3.0
    x[1, [12000, 8200]] = 3.0
    x[2, 20000] = float("nan")
    out = torch.empty(4, dtype=torch.int64, device="cuda")
    _argmax()(x, out)
    assert out.tolist() == [8191, 8200, 20000, 0]
    assert torch.equal(out.cpu(), ds.greedy_argmax(x.cpu()))


# -------------------------------------------------------------------- RMSNorm

def _rms():
    from babyvllm.kernels.layernorm import fused_add_rms_norm
    return fused_add_rms_norm


@pytest.mark.parametrize("rows,hidden", [(64, 3584), (1024, 3584), (7, 896), (3, 100), (5, 4104), (2, 20000)])
@pytest.mark.parametrize("with_residual", [True, False])
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_rms_norm_matches_oracle(rows, hidden, with_residual, wdtype):
    g = torch.Generator(device="cuda").manual_seed(rows * 7 + hidden)
    x = (torch.randn(rows, hidden, device="cuda", generator=g) * 2).to(torch.bfloat16)
    res = torch.randn(rows, hidden, device="cuda", generator=g).to(torch.bfloat16) if with_residual else None
    w = (torch.rand(hidden, device="cuda", generator=g) + 0.5).to(wdtype)
    eps = 1e-6
    exp_out, exp_res = ds.fused_add_rms_norm(x.cpu(), None if res is None else res.cpu(), w.cpu(), eps)
    x_before = x.clone()
    out = _rms()(x, res, w, eps)
    assert out.shape == x.shape and out.dtype == torch.bfloat16
    if with_residual:
        assert torch.equal(res.cpu(), exp_res)
    assert torch.equal(x, x_before)
    d = _ulps(out.cpu(), exp_out)
    assert int(d.max()) <= 1
    assert float((d > 0).float().mean()) < 1e-3


def _weighted_neighbours(x, res, w, eps):
    """bf16(n·w) for n the oracle's bf16 normalized value and its two bf16
    neighbours. The normalized value is rounded to bf16 before the weight
    multiplies it, so a kernel whose normalized value is within one ulp (a
    different summation order of the variance) gives one of these three; a
    weight below 1 can carry that one ulp into a lower binade, where it is two
    ulps of the output."""
    normed, _ = ds.fused_add_rms_norm(x, res, torch.ones(x.shape[-1], dtype=torch.float32), eps)
    bits = normed.view(torch.int16)
    out = []
    for step in (-1, 0, 1):
        nb = (bits.to(torch.int32) + step).to(torch.int16).view(torch.bfloat16)
        out.append((nb.float() * w.float()).to(torch.bfloat16))
    return out


def test_rms_norm_of_a_strided_view_and_3d_input():
    g = torch.Generator().manual_seed(5)
    big = torch.randn(6, 4000, generator=g).to("cuda", torch.bfloat16)
    view = big[:, :3584]
    w = torch.ones(3584, device="cuda", dtype=torch.bfloat16)
    out = _rms()(view, None, w, 1e-6)
    exp, _ = ds.fused_add_rms_norm(view.cpu(), None, w.cpu(), 1e-6)
    assert int(_ulps(out.cpu(), exp).max()) <= 1
    for seed in range(4):
        g = torch.Generator().manual_seed(100 + seed)
        x3 = torch.randn(2, 3, 896, generator=g).to("cuda", torch.bfloat16)
        r3 = torch.randn(2, 3, 896, generator=g).to("cuda", torch.bfloat16)
        w3 = torch.rand(896, generator=g).to("cuda")  # fp32 weights in [0, 1)
        _, er3 = ds.fused_add_rms_norm(x3.cpu(), r3.cpu(), w3.cpu(), 1e-5)
        cands = _weighted_neighbours(x3.cpu(), r3.cpu(), w3.cpu(), 1e-5)
        o3 = _rms()(x3, r3, w3, 1e-5)
        assert o3.shape == (2, 3, 896) and torch.equal(r3.cpu(), er3)
        oc = o3.cpu()
        hit = torch.zeros(oc.shape, dtype=torch.bool)
        for c in cands:
            hit |= oc.view(torch.int16) == c.view(torch.int16)
        assert bool(hit.all()), (seed, int((~hit).sum()))


def test_rms_norm_refuses_a_non_viewable_residual():
    x = torch.randn(4, 64, device="cuda").to(torch.bfloat16)
    res = torch.randn(64, 4, device="cuda").to(torch.bfloat16).t()
    with pytest.raises(AssertionError):
        _rms()(x, res, torch.ones(64, device="cuda", dtype=torch.bfloat16), 1e-6)


# ------------------------------------------------------------------- SiLU·mul

def _silu():
    from babyvllm.kernels.activation import fused_silu_mul
    return fused_silu_mul


@pytest.mark.parametrize("shape", [(64, 2 * 18944), (8192, 2 * 1024), (7, 2 * 100), (2, 5, 2 * 64)])
def test_silu_mul_matches_oracle(shape):
    g = torch.Generator(device="cuda").manual_seed(sum(shape))
    gu = (torch.randn(*shape, device="cuda", generator=g) * 3).to(torch.bfloat16)
    out = _silu()(gu)
    exp = ds.silu_mul(gu.cpu())
    assert out.shape == exp.shape
    d = _ulps(out.cpu(), exp)
    assert int(d.max()) <= 1
    assert float((d > 0).float().mean()) < 1e-3


# ------------------------------------------------------------- in a hip graph

def test_decode_step_tail_replays_in_a_hip_graph():
    """norm -> (stand-in LM head) -> argmax, and SiLU·mul, captured once and
    replayed with new inputs: every replay equals the eager result."""
    rows, hidden, vocab = 64, 896, 5000
    x = torch.randn(rows, hidden, device="cuda").to(torch.bfloat16)
    res = torch.randn(rows, hidden, device="cuda").to(torch.bfloat16)
    w = torch.rand(hidden, device="cuda").to(torch.bfloat16)
    head = (torch.randn(vocab, hidden, device="cuda") * 0.05).to(torch.bfloat16)
    gu = torch.randn(rows, 2 * 256, device="cuda").to(torch.bfloat16)
    tokens = torch.empty(rows, dtype=torch.int64, device="cuda")

    def step():
        h = _rms()(x, res, w, 1e-6)
        logits = h @ head.t().contiguous()
        _argmax()(logits, tokens)
        return _silu()(gu), logits

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    res0 = res.clone()
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    res.copy_(res0)
    with torch.cuda.graph(graph):
        act, logits = step()
    for seed in range(3):
        g = torch.Generator(device="cuda").manual_seed(seed)
        x.copy_(torch.randn(rows, hidden, device="cuda", generator=g).to(torch.bfloat16))
        res.copy_(res0)
        gu.copy_(torch.randn(rows, 2 * 256, device="cuda", generator=g).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        g_tokens, g_act, g_res = tokens.clone(), act.clone(), res.clone()
        res.copy_(res0)
        e_act, e_logits = step()
        torch.cuda.synchronize()
        assert torch.equal(g_act, e_act)
        assert torch.equal(g_res, res)
        assert torch.equal(g_tokens, tokens)
        assert torch.equal(tokens, e_logits.argmax(-1))
