"""C-ABI library checks that need no GPU: it loads, exports every symbol the
header declares with the argument counts the binding uses, rejects bad
arguments on the host, and the Python layer never falls back to a non-HIP path.
"""

import os
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "babyvllm_amd.h"


def _lib():
    from babyvllm.kernels import _lib

    if not _lib.LIB_PATH.exists():
        sys.path.insert(0, str(REPO / "baby-vllm_amd"))
        import build_lib

        build_lib.build()
    return _lib


def _declared():
    text = HEADER.read_text()
    decls = {}
    for m in re.finditer(r"BVLLM_API\s+[\w\s\*]+?\b(bvllm_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        decls[m.group(1)] = len(params)
    return decls


def test_header_declares_the_three_ops_and_helpers():
    names = set(_declared())
    assert {"bvllm_rope_kv_append", "bvllm_paged_decode", "bvllm_paged_prefill",
            "bvllm_decode_workspace_bytes", "bvllm_abi_version", "bvllm_error_string"} <= names


def test_library_exports_every_declared_symbol_with_matching_arity():
    mod = _lib()
    handle = mod.lib()
    for name, nparams in _declared().items():
        assert hasattr(handle, name), f"{name} not exported"
        assert name in mod.SIGNATURES, f"{name} has no ctypes binding"
        assert len(mod.SIGNATURES[name][1]) == nparams, f"{name}: binding arity != header"
    exported = subprocess.run(["nm", "-D", "--defined-only", str(mod.LIB_PATH)],
                              capture_output=True, text=True, check=True).stdout
    ours = set(re.findall(r"\b(bvllm_\w+)\b", exported))
    assert ours == set(_declared()), f"exported {ours ^ set(_declared())} not in the header"


def test_abi_version_matches_header():
    mod = _lib()
    want = int(re.search(r"#define BVLLM_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert mod.lib().bvllm_abi_version() == want == mod.ABI_VERSION


def test_workspace_bytes_formula():
    h = _lib().lib()
    # B8: 15 splits -> 15 partial states per (row, head).
    assert h.bvllm_decode_workspace_bytes(8, 28, 4, 128, 15, 8) == 8 * 28 * 15 * (128 + 1) * 4
    # Single pass: no scratch.
    assert h.bvllm_decode_workspace_bytes(64, 28, 4, 128, 1, 120) == 0
    # B1 x 32768: 512 splits of 4 pages fold into 128 groups of 4 splits.
    assert h.bvllm_decode_workspace_bytes(1, 28, 4, 128, 512, 4) == 28 * 128 * 129 * 4
    # 512 splits of 6 pages cannot fold: one partial per split.
    assert h.bvllm_decode_workspace_bytes(1, 28, 4, 128, 512, 6) == 28 * 512 * 129 * 4


def test_workspace_bytes_ignore_the_split_mode_knob():
    # The size (and the place of part_lse inside it) must not follow knob 0:
    # a knob changed between the size query and the launch would otherwise make
    # the kernels write past the workspace.
    mod = _lib()
    h = mod.lib()
    plans = [(8, 15, 8), (64, 2, 60), (16, 8, 16), (1, 512, 4), (2, 40, 8), (4, 20, 4), (1, 7, 5)]
    want = {p: h.bvllm_decode_workspace_bytes(p[0], 28, 4, 128, p[1], p[2]) for p in plans}
    try:
        for knob_value in (1, 2, 3, 4):
            mod.set_tuning(mod.TUNE_DECODE_SPLIT_MODE, knob_value)
            for p in plans:
                assert h.bvllm_decode_workspace_bytes(p[0], 28, 4, 128, p[1], p[2]) == want[p], (knob_value, p)
    finally:
        mod.set_tuning(mod.TUNE_DECODE_SPLIT_MODE, 0)


def test_host_side_argument_rejection():
    h = _lib().lib()
    bad = 1  # hipErrorInvalidValue
    # block_size 15
    assert h.bvllm_paged_decode(None, 0, 0, None, None, 0, 0, 0, 0, None, 0, 0, None, 1.0,
                                None, 0, 0, None, 1, 1, 1, 28, 4, 128, 15, 0, None) == bad
    # head_dim 96
    assert h.bvllm_paged_prefill(None, 0, 0, None, None, 0, 0, 0, 0, None, 0, 0, None, None, None,
                                 1.0, None, 0, 0, 1, 1, 1, -1, 28, 4, 96, 16, None) == bad
    # single_query_seqs above num_seqs
    assert h.bvllm_paged_prefill(None, 0, 0, None, None, 0, 0, 0, 0, None, 0, 0, None, None, None,
                                 1.0, None, 0, 0, 1, 1, 1, 2, 28, 4, 128, 16, None) == bad
    # 28 heads over 5 KV heads
    assert h.bvllm_rope_kv_append(None, 0, 0, None, 0, 0, None, 0, 0, None, 0, None, 0,
                                  None, None, 0, 0, 0, None, 1, 28, 5, 128, None) == bad
    # 34 query heads over 4 KV heads (GQA groups above 16 are accepted: 34 over 2 is)
    assert h.bvllm_paged_decode(None, 0, 0, None, None, 0, 0, 0, 0, None, 0, 0, None, 1.0,
                                None, 0, 0, None, 1, 1, 1, 34, 4, 128, 16, 0, None) == bad
    assert b"invalid argument" in h.bvllm_error_string(bad)
    # waves must be 0 or 4 (8 was accepted by an earlier ABI and is refused now)
    for waves in (5, 8):
        assert h.bvllm_paged_decode(None, 0, 0, None, None, 0, 0, 0, 0, None, 0, 0, None, 1.0,
                                    None, 0, 0, None, 1, 1, 1, 28, 4, 128, 16, waves, None) == bad
    # Nothing to do is a success that launches nothing.
    assert h.bvllm_paged_decode(None, 0, 0, None, None, 0, 0, 0, 0, None, 0, 0, None, 1.0,
                                None, 0, 0, None, 1, 1, 0, 28, 4, 128, 16, 0, None) == 0


def test_python_ops_refuse_cpu_tensors():
    from babyvllm.kernels.paged_attn import paged_decode_attention
    from babyvllm.kernels.rope import fused_rope_and_cache

    q = torch.zeros(2, 28, 128, dtype=torch.bfloat16)
    cache = torch.zeros(2, 4, 16, 4, 128, dtype=torch.bfloat16)
    bt = torch.zeros(2, 2, dtype=torch.int32)
    lens = torch.ones(2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="ROCm"):
        paged_decode_attention(q, cache, bt, lens, 0.1)
    with pytest.raises(RuntimeError, match="ROCm"):
        fused_rope_and_cache(q, q[:, :4], q[:, :4], q[:, 0], q[:, 0])


def test_attention_layer_has_no_cpu_path():
    from babyvllm.layers.attention import Attention
    from babyvllm.worker.context import AttentionMetadata, set_forward_context

    attn = Attention(4, 16, 2)
    q = torch.zeros(1, 4, 16)
    with pytest.raises(RuntimeError):
        attn(q, q[:, :2], q[:, :2])  # no cache / context
    attn.kv_cache = torch.zeros(2, 1, 16, 2, 16)
    md = AttentionMetadata(torch.zeros(1, dtype=torch.int64), torch.zeros(1, 1, dtype=torch.int32),
                           torch.tensor([0, 1], dtype=torch.int32), torch.ones(1, dtype=torch.int32),
                           torch.zeros(1, dtype=torch.int32), [0, 1], [1], [0], 1, 1)
    with set_forward_context(md):
        with pytest.raises(RuntimeError, match="ROCm"):
            attn(q, q[:, :2], q[:, :2])


def test_missing_library_fails_loudly():
    code = (
        "import sys; sys.path.insert(0, 'baby-vllm_amd')\n"
        "from babyvllm.kernels import _lib\n"
        "try:\n    _lib.lib()\nexcept _lib.KernelLibraryError as e:\n    print('LOUD', e)\n"
    )
    env = dict(os.environ, BVLLM_LIB="/nonexistent/libbvllm_amd.so")
    out = subprocess.run([sys.executable, "-c", code], cwd=REPO, env=env, capture_output=True,
                         text=True, timeout=120)
    assert "LOUD" in out.stdout and "no non-HIP fallback" in out.stdout


def test_product_package_never_imports_the_oracle():
    pkg = REPO / "baby-vllm_amd"
    for f in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.h")):
        text = f.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", text, re.M), f"{f} imports the oracle"
