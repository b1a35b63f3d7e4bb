"""ctypes binding of libmgg.so, the gfx950 C-ABI library (include/mgg.h).

The library is built in-tree by ``build_native.build()``.  It is loaded after
``import torch`` so that it binds to the HIP runtime torch already loaded
(same soname), and therefore shares torch's devices and streams.  A missing
library raises: there is no other implementation of these entry points.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime this library must share)

LIB_PATH = Path(__file__).resolve().parent / "libmgg.so"
ABI_VERSION = 8

MGG_OK = 0
MGG_ERR_INVALID = 1
MGG_ERR_UNSUPPORTED = 2
MGG_ERR_HIP = 3

MGG_DTYPE_BF16 = 0
MGG_DTYPE_FP16 = 1
MGG_DTYPE_FP8_E4M3 = 2
MGG_B_KMAJOR = 0x100  # | BF16/FP16: B stored [E, N, K], ldb_k = stride between N rows
MGG_INT32 = 0
MGG_INT64 = 1
# Largest expert count for which the kernels derive the work queue on the
# device (the per-expert tile prefix lives in LDS; kMaxLdsExpertsGemm).
MAX_DEVICE_QUEUE_EXPERTS = 2048
# Largest expert count of the device-side queue builder mgg_build_work_queue
# (kMaxLdsExpertsQueue).
MAX_DEVICE_BUILDER_EXPERTS = 8192

MGG_EPI_NONE = 0
MGG_EPI_GELU = 1
MGG_EPI_SWIGLU = 2

_c_i32 = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_ptr = ctypes.c_void_p

# name -> argument types (all return int except mgg_last_error)
_SIGNATURES = {
    "mgg_abi_version": [],
    "mgg_device_cu_count": [_c_i32, ctypes.POINTER(_c_i32)],
    "mgg_expert_offsets_from_counts": [_c_ptr, _c_i32, _c_i64, _c_ptr, _c_i32, _c_ptr],
    "mgg_expert_offsets_from_counts_host": [_c_ptr, _c_i32, _c_i64, _c_ptr, _c_i32],
    "mgg_build_work_queue": [
        _c_ptr, _c_i64, _c_i64, _c_i32, _c_i32, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_ptr,
    ],
    "mgg_build_work_queue_host": [
        _c_ptr, _c_i64, _c_i64, _c_i32, _c_i32, _c_ptr, _c_ptr, _c_ptr, _c_i64,
    ],
    "mgg_grouped_gemm": [
        _c_i32, _c_ptr, _c_ptr, _c_ptr,  # dtype, a, b, c
        _c_ptr, _c_i64, _c_i64, _c_i64,  # offsets, M, K, N
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,  # E, lda, ldb_e, ldb_k, ldc
        _c_ptr, _c_ptr, _c_ptr, _c_i64,  # queue, num_work
        _c_i32, _c_i32, _c_i32, _c_i32,  # block_m, block_n, num_workers, atomic
        _c_ptr, _c_i32, _c_i32, _c_ptr,  # work_counter, report_block_m/n, stream
    ],
    "mgg_grouped_gemm_gathered": [
        _c_i32, _c_i32, _c_ptr, _c_ptr, _c_i64,  # dtype, epilogue, a, a_rows, a_src_rows
        _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64,  # b, c, offsets, M, K, N
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,  # E, lda, ldb_e, ldb_k, ldc
        _c_i32, _c_i32, _c_ptr,  # num_workers, atomic, stream
    ],
    "mgg_grouped_gemm_ex": [
        _c_i32, _c_i32, _c_ptr, _c_ptr, _c_ptr,  # dtype, epilogue, a, b, c
        _c_ptr, _c_i64, _c_i64, _c_i64,  # offsets, M, K, N
        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,  # E, lda, ldb_e, ldb_k, ldc
        _c_ptr, _c_ptr, _c_ptr, _c_i64,  # queue, num_work
        _c_i32, _c_i32, _c_i32, _c_i32,  # block_m, block_n, num_workers, atomic
        _c_ptr, _c_i32, _c_i32, _c_ptr,  # work_counter, report_block_m/n, stream
    ],
    "mgg_grouped_gemm_fp8": [
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,  # a, b, c, offsets, a_scale, b_scale
        _c_i64, _c_i64, _c_i64, _c_i64,  # M, K, N, E
        _c_i64, _c_i64, _c_i64, _c_i64,  # lda, ldb_e, ldb_n, ldc
        _c_ptr, _c_ptr, _c_ptr, _c_i64,  # queue, num_work
        _c_i32, _c_i32, _c_i32, _c_i32,  # block_m, block_n, num_workers, atomic
        _c_ptr, _c_i32, _c_i32, _c_ptr,  # work_counter, report_block_m/n, stream
    ],
    "mgg_debug_set_dequeue_counter": [ctypes.c_uint64, _c_ptr],
    "mgg_debug_set_clock_probe": [_c_ptr],
    "mgg_debug_set_split_flags": [ctypes.c_uint64, _c_ptr],
    "mgg_debug_counter_slots": [_c_i32, ctypes.POINTER(_c_i32)],
    "mgg_reserve_split_workspace": [_c_ptr],
    "mgg_split_workspace_bytes": [_c_ptr, ctypes.POINTER(_c_i64)],
    "mgg_set_split_last_round": [_c_i32],
    "mgg_dispatch_layout": [
        _c_ptr, _c_i32, _c_i64, _c_i32, _c_i64,  # topk_idx, idx_type, T, top_k, E
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,  # counts, offsets, slot_pos, token_index, row_assign
        _c_ptr, _c_i64, _c_ptr,  # workspace, workspace_bytes, stream
    ],
    "mgg_dispatch_layout_noalloc": [
        _c_ptr, _c_i32, _c_i64, _c_i32, _c_i64,  # topk_idx, idx_type, T, top_k, E
        _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,  # counts, offsets, slot_pos, token_index, row_assign
        _c_ptr,  # stream
    ],
    "mgg_gather_rows": [
        _c_i32, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr,
    ],
    "mgg_combine_rows": [
        _c_i32, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_i64, _c_i32, _c_i64, _c_ptr, _c_i64, _c_ptr,
    ],
}
# entry points whose return value is not a status code
_RESTYPES = {"mgg_dispatch_layout_workspace_bytes": ([_c_i64, _c_i32, _c_i64], _c_i64)}
EXPORTED = tuple(_SIGNATURES) + tuple(_RESTYPES) + ("mgg_last_error",)

_lib = None


class NativeError(RuntimeError):
    """A libmgg entry point returned an error status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"libmgg error {code}: {message}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Loads libmgg.so once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
            "g.build()'` (or moe-overlap_amd/build_native.py)"
        )
    handle = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = argtypes
        fn.restype = _c_i32
    for name, (argtypes, restype) in _RESTYPES.items():
        fn = getattr(handle, name)
        fn.argtypes = argtypes
        fn.restype = restype
    handle.mgg_last_error.argtypes = []
    handle.mgg_last_error.restype = ctypes.c_char_p
    version = handle.mgg_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libmgg ABI version {version}, expected {ABI_VERSION}: rebuild it")
    _lib = handle
    return _lib


def check(code: int) -> None:
    """Raises NativeError with the library's message for a non-zero status."""
    if code != MGG_OK:
        raise NativeError(code, lib().mgg_last_error().decode(errors="replace"))


def device_cu_count(device_index: int) -> int:
    n = _c_i32(0)
    check(lib().mgg_device_cu_count(int(device_index), ctypes.byref(n)))
    return int(n.value)
