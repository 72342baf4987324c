"""ctypes binding of libbvllm_amd.so, the C-ABI HIP library (include/babyvllm_amd.h).

The library is built in-tree by ``baby-vllm_amd/build_lib.py`` (or
``__graft_entry__.build()``). There is no fallback: if the library is missing
or fails to load, every kernel entry point raises, so a run can never silently
take a CPU or eager-PyTorch path instead of the HIP kernels.
"""

from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get(
    "BVLLM_LIB", Path(__file__).resolve().parent.parent / "libbvllm_amd.so"))

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# Signatures, in header order. Every entry point returns int (a hipError_t).
SIGNATURES = {
    "bvllm_abi_version": (ctypes.c_int, []),
    "bvllm_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "bvllm_rope_kv_append": (ctypes.c_int, [
        _p, _i64, _i64,             # q, strides t, h
        _p, _i64, _i64,             # k
        _p, _i64, _i64,             # v
        _p, _i64,                   # cos
        _p, _i64,                   # sin
        _p, _p, _i64, _i64,         # k_cache, v_cache, slot stride, head stride
        _i64, _p,                   # num_slots, slot_mapping
        _i32, _i32, _i32, _i32,     # T, H, Hkv, D
        _p,                         # stream
    ]),
    "bvllm_decode_workspace_bytes": (ctypes.c_int64, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "bvllm_paged_decode": (ctypes.c_int, [
        _p, _i64, _i64,             # q
        _p, _p, _i64, _i64, _i64,   # caches + strides
        _i32,                       # num_blocks
        _p, _i64, _i32,             # block_tables, bt_stride, max_blocks
        _p, _f32,                   # seq_lens, scale
        _p, _i64, _i64,             # out
        _p, _i32, _i32,             # workspace, num_splits, blocks_per_split
        _i32, _i32, _i32, _i32, _i32, _i32,  # B, H, Hkv, D, block_size, waves
        _p,                         # stream
    ]),
    "bvllm_paged_decode_noalloc": (ctypes.c_int, [
        _p, _i64, _i64,             # q
        _p, _p, _i64, _i64, _i64,   # caches + strides
        _i32,                       # num_blocks
        _p, _i64, _i32,             # block_tables, bt_stride, max_blocks
        _p, _f32,                   # seq_lens, scale
        _p, _i64, _i64,             # out
        _i32, _i32,                 # num_splits, blocks_per_split
        _i32, _i32, _i32, _i32, _i32, _i32,  # B, H, Hkv, D, block_size, waves
        _p,                         # stream
    ]),
    "bvllm_paged_prefill": (ctypes.c_int, [
        _p, _i64, _i64,             # q
        _p, _p, _i64, _i64, _i64,   # caches + strides
        _i32,                       # num_blocks
        _p, _i64, _i32,             # block_tables, bt_stride, max_blocks
        _p, _p, _p, _f32,           # query_start_loc, seq_lens, context_lens, scale
        _p, _i64, _i64,             # out
        _i32, _i32, _i32,           # num_seqs, num_tokens, max_query_len
        _i32,                       # single_query_seqs (-1 = unknown)
        _i32, _i32, _i32, _i32,     # H, Hkv, D, block_size
        _p,                         # stream
    ]),
    "bvllm_set_tuning": (ctypes.c_int, [_i32, _i32]),
    "bvllm_argmax_workspace_bytes": (ctypes.c_int64, [_i32, _i32]),
    "bvllm_greedy_argmax": (ctypes.c_int, [
        _p, _i64, _i32, _i32,       # logits, row_stride, rows, vocab
        _i32, _p, _p,               # logits_fp32, workspace, out
        _p,                         # stream
    ]),
    "bvllm_fused_add_rms_norm": (ctypes.c_int, [
        _p, _i64, _p, _i64,         # input, stride, residual, stride
        _p, _i32,                   # weight, weight_fp32
        _p, _i64,                   # out, stride
        _i32, _i32, _f32,           # rows, hidden, eps
        _p,                         # stream
    ]),
    "bvllm_silu_mul": (ctypes.c_int, [_p, _i64, _i32, _p, _p]),
}

ABI_VERSION = 6


# Knobs of bvllm_set_tuning (include/babyvllm_amd.h).
TUNE_DECODE_SPLIT_MODE = 0
TUNE_PREFILL_BLOCKS_PER_WG = 1
TUNE_DECODE_ORDER = 2
TUNE_DECODE_SINGLE_PASS_STREAM = 3
TUNE_DECODE_CACHED = 4
TUNE_APPEND_CHUNKS = 5
TUNE_PREFILL_SHORT_GRID = 6


class KernelLibraryError(RuntimeError):
    """The HIP library is missing, stale, or a launch returned an error."""


@functools.lru_cache(maxsize=None)
def lib() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise KernelLibraryError(
            f"{LIB_PATH} not found: build it with `python baby-vllm_amd/build_lib.py` "
            "(the paged-KV ops have no non-HIP fallback)")
    handle = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    got = handle.bvllm_abi_version()
    if got != ABI_VERSION:
        raise KernelLibraryError(f"{LIB_PATH} has ABI {got}, expected {ABI_VERSION}: rebuild it")
    return handle


def set_tuning(knob: int, value: int) -> int:
    """Sets a process-wide tuning knob (0 = default); returns its previous value."""
    prev = lib().bvllm_set_tuning(knob, value)
    if prev < 0:
        raise ValueError(f"unknown tuning knob {knob}")
    return prev


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().bvllm_error_string(rc)
        raise KernelLibraryError(f"{what} failed: {msg.decode() if msg else rc} (code {rc})")


def stream_handle(device) -> int:
    """hipStream_t of torch's current stream on ``device`` (captured streams included)."""
    import torch

    return torch.cuda.current_stream(device).cuda_stream


def require_rocm_tensor(name: str, t) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"{name} is on {t.device}: the babyvllm_amd kernels run only on a ROCm (HIP) device")
