"""libmgg.so on the CPU: it loads, exports every entry point include/mgg.h
declares, its host-side builders match the oracle bit for bit, and argument
validation rejects bad calls before any device work."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

import mgg_native as nat
from oracle import grouped_gemm_oracle as orc

HEADER = Path(__file__).resolve().parents[1] / "include" / "mgg.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(mgg_\w+)\s*\(", text))


def test_library_exports_every_declared_entry_point():
    lib = nat.lib()
    declared = declared_functions()
    assert {"mgg_grouped_gemm", "mgg_build_work_queue", "mgg_expert_offsets_from_counts"} <= declared
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(nat.EXPORTED)


def test_abi_version_and_empty_error():
    lib = nat.lib()
    assert lib.mgg_abi_version() == nat.ABI_VERSION
    assert isinstance(lib.mgg_last_error(), bytes)


def host_offsets(counts, in_dtype, out_dtype):
    c = np.ascontiguousarray(np.asarray(counts, dtype=in_dtype))
    out = np.empty(c.size + 1, dtype=out_dtype)
    code_in = nat.MGG_INT32 if in_dtype == np.int32 else nat.MGG_INT64
    code_out = nat.MGG_INT32 if out_dtype == np.int32 else nat.MGG_INT64
    nat.check(nat.lib().mgg_expert_offsets_from_counts_host(
        c.ctypes.data_as(ctypes.c_void_p), code_in, c.size,
        out.ctypes.data_as(ctypes.c_void_p), code_out))
    return out


@settings(max_examples=100, deadline=None)
@given(st.lists(st.integers(-(2**40), 2**40), max_size=40),
       st.sampled_from([np.int32, np.int64]), st.sampled_from([np.int32, np.int64]))
def test_host_offsets_match_oracle(counts, in_dtype, out_dtype):
    counts = np.asarray(counts, dtype=np.int64)
    if in_dtype == np.int32:
        counts = counts.astype(np.int32)  # wrap into the int32 input
    got = host_offsets(counts, in_dtype, out_dtype)
    np.testing.assert_array_equal(got, orc.expert_offsets_from_recv_counts(counts, dtype=out_dtype))


def host_queue(offsets, n_size, bm, bn):
    off = np.ascontiguousarray(np.asarray(offsets, dtype=np.int64))
    total = orc.queue_length(off, n_size, bm, bn)
    out = [np.empty(total, np.int32) for _ in range(3)]
    nat.check(nat.lib().mgg_build_work_queue_host(
        off.ctypes.data_as(ctypes.c_void_p), off.size - 1, n_size, bm, bn,
        *[o.ctypes.data_as(ctypes.c_void_p) for o in out], total))
    return out


@settings(max_examples=100, deadline=None)
@given(st.lists(st.integers(-5, 600), max_size=20), st.integers(0, 5000),
       st.sampled_from([16, 64, 128, 256]), st.sampled_from([32, 64, 128, 256]))
def test_host_queue_matches_oracle(counts, n_size, bm, bn):
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    for got, want in zip(host_queue(offs, n_size, bm, bn), orc.build_work_queue(offs, n_size, bm, bn)):
        np.testing.assert_array_equal(got, want)


def test_host_queue_rejects_wrong_length():
    off = np.array([0, 5], np.int64)
    out = [np.empty(8, np.int32) for _ in range(3)]
    rc = nat.lib().mgg_build_work_queue_host(
        off.ctypes.data_as(ctypes.c_void_p), 1, 64, 4, 64,
        *[o.ctypes.data_as(ctypes.c_void_p) for o in out], 1)
    assert rc == nat.MGG_ERR_INVALID and b"num_work" in nat.lib().mgg_last_error()


FAKE = 1 << 20  # a 16-byte aligned non-null address; validation rejects before any access


def gemm_call(**over):
    args = dict(dtype=nat.MGG_DTYPE_BF16, a=FAKE, b=FAKE, c=FAKE, off=FAKE, m=64, k=64, n=64, e=1,
                lda=64, ldb_e=64 * 64, ldb_k=64, ldc=64, we=None, wm=None, wn=None, nw=-1,
                bm=128, bn=128, workers=4, atomic=0, counter=None, rbm=0, rbn=0, stream=None)
    args.update(over)
    return nat.lib().mgg_grouped_gemm(*args.values())


@pytest.mark.parametrize("over, code, text", [
    (dict(dtype=7), nat.MGG_ERR_UNSUPPORTED, b"dtype"),
    (dict(bm=96), nat.MGG_ERR_UNSUPPORTED, b"block_m"),
    (dict(bn=1024), nat.MGG_ERR_UNSUPPORTED, b"block_m"),
    (dict(bm=256, bn=512), nat.MGG_ERR_UNSUPPORTED, b"block_m"),
    # K need not be a multiple of 8 for N-major 16-bit B (A is read to the next
    # multiple, B's rows stop at K), but must be for K-major B.
    (dict(dtype=nat.MGG_DTYPE_BF16 | nat.MGG_B_KMAJOR, k=60, lda=64, ldb_k=64, ldb_e=64 * 64),
     nat.MGG_ERR_UNSUPPORTED, b"multiple of 8"),
    (dict(k=60, lda=56), nat.MGG_ERR_INVALID, b"leading"),
    # Any N and any B and C strides are read in place with N-major B (the
    # checks below reject these calls for other reasons before a launch).
    (dict(n=61, ldb_k=61, ldc=61, ldb_e=61 * 64, lda=68), nat.MGG_ERR_UNSUPPORTED, b"lda"),
    # Odd N has kernel instances for 256x256, 128x128 and (N-major 16-bit B,
    # no fused epilogue) 128x512 tiles only.
    (dict(n=61, ldb_k=61, ldc=61, ldb_e=61 * 64, bm=64, bn=64), nat.MGG_ERR_UNSUPPORTED, b"odd N"),
    (dict(n=61, ldb_k=61, ldc=61, ldb_e=61 * 64, bm=256, bn=128), nat.MGG_ERR_UNSUPPORTED,
     b"odd N"),
    (dict(dtype=nat.MGG_DTYPE_BF16 | nat.MGG_B_KMAJOR, n=61, ldb_k=64, ldc=61, ldb_e=64 * 61,
          bm=128, bn=512), nat.MGG_ERR_UNSUPPORTED, b"odd N"),
    (dict(lda=32), nat.MGG_ERR_INVALID, b"leading"),
    (dict(lda=68), nat.MGG_ERR_UNSUPPORTED, b"multiple of 8"),
    (dict(dtype=nat.MGG_DTYPE_BF16 | nat.MGG_B_KMAJOR, ldb_k=68, ldb_e=68 * 64),
     nat.MGG_ERR_UNSUPPORTED, b"multiple of 8"),
    (dict(ldc=66, n=60, ldb_k=60, ldb_e=60 * 64, a=FAKE + 8), nat.MGG_ERR_UNSUPPORTED, b"aligned"),
    (dict(a=None), nat.MGG_ERR_INVALID, b"null"),
    (dict(off=None), nat.MGG_ERR_INVALID, b"null"),
    (dict(a=FAKE + 8), nat.MGG_ERR_UNSUPPORTED, b"aligned"),
    (dict(m=-1), nat.MGG_ERR_INVALID, b">= 0"),
    (dict(k=1 << 24, lda=1 << 24), nat.MGG_ERR_UNSUPPORTED, b"32-bit"),
    (dict(e=4096), nat.MGG_ERR_UNSUPPORTED, b"2048 experts"),
    (dict(nw=5), nat.MGG_ERR_INVALID, b"null work queue"),
    (dict(workers=70000), nat.MGG_ERR_INVALID, b"num_workers"),
    # K-major B: the flag is for 16-bit dtypes only, and ldb_k is then the stride between N
    # rows, so it must cover K (64 covers N = 64 but not K = 128).
    (dict(dtype=nat.MGG_DTYPE_FP8_E4M3 | nat.MGG_B_KMAJOR), nat.MGG_ERR_UNSUPPORTED, b"dtype"),
    (dict(dtype=nat.MGG_DTYPE_BF16 | 0x200), nat.MGG_ERR_UNSUPPORTED, b"dtype"),
    (dict(dtype=nat.MGG_DTYPE_BF16 | nat.MGG_B_KMAJOR, k=128, lda=128, ldb_k=64, ldb_e=64 * 128),
     nat.MGG_ERR_INVALID, b"leading"),
])
def test_gemm_validation_rejects_before_launch(over, code, text):
    assert gemm_call(**over) == code
    assert text in nat.lib().mgg_last_error()


def gathered_call(**over):
    args = dict(dtype=nat.MGG_DTYPE_BF16, epi=nat.MGG_EPI_NONE, a=FAKE, rows=FAKE, src=64, b=FAKE,
                c=FAKE, off=FAKE, m=64, k=64, n=256, e=1, lda=64, ldb_e=64 * 256, ldb_k=256,
                ldc=256, workers=4, atomic=0, stream=None)
    args.update(over)
    return nat.lib().mgg_grouped_gemm_gathered(*args.values())


@pytest.mark.parametrize("over, code, text", [
    (dict(rows=None), nat.MGG_ERR_INVALID, b"a_rows"),
    (dict(dtype=nat.MGG_DTYPE_FP8_E4M3), nat.MGG_ERR_UNSUPPORTED, b"16-bit"),
    (dict(dtype=nat.MGG_DTYPE_BF16 | nat.MGG_B_KMAJOR, ldb_k=64), nat.MGG_ERR_UNSUPPORTED,
     b"gathered A needs"),
    (dict(src=-1), nat.MGG_ERR_INVALID, b"a_src_rows"),
    (dict(src=1 << 24), nat.MGG_ERR_UNSUPPORTED, b"32-bit"),
    (dict(lda=32), nat.MGG_ERR_INVALID, b"leading"),
    (dict(e=4096), nat.MGG_ERR_UNSUPPORTED, b"2048 experts"),
])
def test_gathered_validation_rejects_before_launch(over, code, text):
    """The gathered up GEMM covers the A-block tile only (16-bit, N-major B,
    256x256, device-derived queue) and 32-bit offsets into the source rows."""
    assert gathered_call(**over) == code
    assert text in nat.lib().mgg_last_error()


def test_gemm_empty_output_is_a_no_op():
    assert gemm_call(m=0) == nat.MGG_OK
    assert gemm_call(n=0) == nat.MGG_OK


def test_builders_validate():
    lib = nat.lib()
    assert lib.mgg_build_work_queue(FAKE, 9000, 64, 128, 128, FAKE, FAKE, FAKE, 1, None) \
        == nat.MGG_ERR_UNSUPPORTED
    assert lib.mgg_build_work_queue(FAKE, 4, 64, 0, 128, FAKE, FAKE, FAKE, 1, None) \
        == nat.MGG_ERR_INVALID
    assert lib.mgg_expert_offsets_from_counts(FAKE, 5, 4, FAKE, 0, None) == nat.MGG_ERR_INVALID
    assert lib.mgg_expert_offsets_from_counts(None, 0, 4, FAKE, 0, None) == nat.MGG_ERR_INVALID
