"""bvllm_paged_decode_noalloc (the decode entry point that allocates nothing)
against bvllm_paged_decode, through the C ABI.

Both entry points run the same kernels on the same plan; the allocation-free
one keeps the split partials in the library's static per-GPU scratch array
instead of a caller workspace. Outputs must be bit-identical, on two calls in
a row where the second is smaller (the array then still holds the first call's
partials, which the second must not read), and on a single-pass plan (no
scratch). A plan whose scratch exceeds the array is refused on the host.
"""

import ctypes

import pytest
import torch

from tests._cases import BLOCK_SIZE, assert_attn_close, make_decode_inputs

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU"),
]

HEADER_LIMIT = 32 << 20  # BVLLM_NOALLOC_SCRATCH_BYTES
SCRATCH_LIMIT_ERROR = 10001  # BVLLM_ERROR_SCRATCH_LIMIT


def _lib():
    from babyvllm.kernels import _lib
    return _lib


def _plan(batch, width, ctx_bucket, partition=None):
    from babyvllm.kernels.decode_split import decode_split_plan
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    return decode_split_plan(batch, 4, BLOCK_SIZE, width, ctx_bucket, cus, partition)


def _call(name, q, kv_cache, bt, lens, scale, plan, workspace=None):
    L = _lib()
    B, H, D = q.shape
    _, nb, bs, hkv, _ = kv_cache.shape
    k, v = kv_cache[0], kv_cache[1]
    out = torch.full_like(q, float("nan"))
    args = [q.data_ptr(), q.stride(0), q.stride(1),
            k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), k.stride(2), nb,
            bt.data_ptr(), bt.stride(0), bt.shape[1], lens.data_ptr(), ctypes.c_float(scale),
            out.data_ptr(), out.stride(0), out.stride(1)]
    if name == "bvllm_paged_decode":
        args.append(None if workspace is None else workspace.data_ptr())
    args += [plan[0], plan[1], B, H, hkv, D, bs, 0, L.stream_handle(q.device)]
    rc = getattr(L.lib(), name)(*args)
    return rc, out


def _with_workspace(q, kv_cache, bt, lens, scale, plan):
    L = _lib()
    B, H, D = q.shape
    nbytes = L.lib().bvllm_decode_workspace_bytes(B, H, kv_cache.shape[3], D, plan[0], plan[1])
    ws = torch.empty(max(nbytes, 4) // 4, device=q.device, dtype=torch.float32) if nbytes > 0 else None
    rc, out = _call("bvllm_paged_decode", q, kv_cache, bt, lens, scale, plan, ws)
    L.check(rc, "bvllm_paged_decode")
    return out, nbytes


def _oracle(q, kv_cache, bt, lens, scale):
    from oracle import attention as oa
    return oa.static_decode_attention(q.float().cpu(), kv_cache.float().cpu(), bt.cpu(),
                                      torch.tensor(lens, dtype=torch.int32), max(max(lens), 1), scale)


def test_noalloc_matches_workspace_entry_point_on_two_calls_in_a_row():
    scale = 128 ** -0.5
    g = torch.Generator().manual_seed(11)
    # First call: batch 8 at context up to 1920 (15 splits of 8 pages).
    lens1 = torch.randint(1500, 1921, (8,), generator=g).tolist()
    q1, kv1, bt1, sl1 = make_decode_inputs(lens1, width=120, seed=1)
    plan1 = _plan(8, 120, 1920)
    assert plan1[0] > 1
    want1, ws1 = _with_workspace(q1, kv1, bt1, sl1, scale, plan1)
    rc, got1 = _call("bvllm_paged_decode_noalloc", q1, kv1, bt1, sl1, scale, plan1)
    _lib().check(rc, "bvllm_paged_decode_noalloc")
    torch.cuda.synchronize()
    assert ws1 > 0
    assert torch.equal(got1, want1)
    assert_attn_close(got1, _oracle(q1, kv1, bt1, lens1, scale))

    # Second call, smaller: batch 2 with a padded row at context up to 600.
    lens2 = [600, 0]
    q2, kv2, bt2, sl2 = make_decode_inputs(lens2, width=40, seed=2)
    plan2 = _plan(2, 40, 640)
    assert plan2[0] > 1
    want2, ws2 = _with_workspace(q2, kv2, bt2, sl2, scale, plan2)
    rc, got2 = _call("bvllm_paged_decode_noalloc", q2, kv2, bt2, sl2, scale, plan2)
    _lib().check(rc, "bvllm_paged_decode_noalloc")
    torch.cuda.synchronize()
    assert 0 < ws2 < ws1
    assert torch.equal(got2, want2)
    assert got2[1].abs().max() == 0
    assert_attn_close(got2[:1], _oracle(q2, kv2, bt2, lens2, scale)[:1])


def test_noalloc_single_pass_and_batch_one_long_context():
    scale = 128 ** -0.5
    # Single pass (no scratch needed at all).
    lens = [1920] * 64
    q, kv, bt, sl = make_decode_inputs(lens, width=120, seed=3)
    plan = _plan(64, 120, 1920)
    assert plan[0] == 1
    want, ws = _with_workspace(q, kv, bt, sl, scale, plan)
    rc, got = _call("bvllm_paged_decode_noalloc", q, kv, bt, sl, scale, plan)
    _lib().check(rc, "bvllm_paged_decode_noalloc")
    assert ws == 0 and torch.equal(got, want)
    # Batch 1 at context 32768: the largest plan of the benchmark (512 splits of 4 pages).
    lens = [32768]
    q, kv, bt, sl = make_decode_inputs(lens, width=2048, seed=4)
    plan = _plan(1, 2048, 32768)
    want, ws = _with_workspace(q, kv, bt, sl, scale, plan)
    rc, got = _call("bvllm_paged_decode_noalloc", q, kv, bt, sl, scale, plan)
    _lib().check(rc, "bvllm_paged_decode_noalloc")
    torch.cuda.synchronize()
    assert 0 < ws <= HEADER_LIMIT and torch.equal(got, want)


def test_noalloc_refuses_a_plan_beyond_its_scratch():
    L = _lib()
    B, H, D = 64, 28, 128
    splits, bps = 4096, 1
    need = L.lib().bvllm_decode_workspace_bytes(B, H, 4, D, splits, bps)
    assert need > HEADER_LIMIT
    q, kv, bt, sl = make_decode_inputs([16] * B, width=4, seed=5)
    rc, out = _call("bvllm_paged_decode_noalloc", q, kv, bt, sl, 0.1, (splits, bps))
    assert rc == SCRATCH_LIMIT_ERROR
    assert b"BVLLM_NOALLOC_SCRATCH_BYTES" in L.lib().bvllm_error_string(rc)
    torch.cuda.synchronize()
    assert torch.isnan(out).all()  # nothing was launched


_CAPTURE_FIRST_CALL = r"""
import sys
sys.path[:0] = [{repo!r}, {repo!r} + "/baby-vllm_amd", {repo!r} + "/tests"]
import torch
from tests import test_zz_no_alloc as t
from tests._cases import make_decode_inputs

scale = 128 ** -0.5
lens = [1900, 1500, 1920, 700, 1920, 33, 1800, 1024]
q, kv, bt, sl = make_decode_inputs(lens, width=120, seed=21)
plan = t._plan(8, 120, 1920)
assert plan[0] > 1
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(side):
    with torch.cuda.graph(graph, stream=side):
        # The process's first call of the entry point: its scratch lookup
        # happens inside the capture.
        rc, out = t._call("bvllm_paged_decode_noalloc", q, kv, bt, sl, scale, plan)
torch.cuda.current_stream().wait_stream(side)
torch.cuda.synchronize()
t._lib().check(rc, "bvllm_paged_decode_noalloc under capture")
g = torch.Generator(device="cuda").manual_seed(5)
for replay in range(4):
    q.copy_(torch.randn(q.shape, device="cuda", dtype=q.dtype, generator=g))
    if replay == 2:
        sl.copy_(torch.tensor([16, 1920, 1, 0, 500, 1919, 64, 1234], dtype=torch.int32))
    graph.replay()
    torch.cuda.synchronize()
    want, _ = t._with_workspace(q, kv, bt, sl, scale, plan)  # eager, between replays
    torch.cuda.synchronize()
    assert torch.equal(out, want), f"replay {{replay}} differs from the workspace entry point"
print("CAPTURE_OK", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture_then_replays():
    # A fresh process, so that the capture holds the first call (and the
    # scratch address lookup); every replay is compared bit for bit with the
    # workspace entry point run eagerly between replays.
    import os
    import subprocess
    import sys

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = _CAPTURE_FIRST_CALL.format(repo=repo)
    p = subprocess.run([sys.executable, "-c", code], cwd=repo, capture_output=True, text=True, timeout=300)
    assert p.returncode == 0 and "CAPTURE_OK" in p.stdout, p.stdout[-2000:] + p.stderr[-4000:]
