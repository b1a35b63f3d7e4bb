"""GPU parity for N not a multiple of 8.

The reference's Triton kernel masks the N edge in its loads and its store
(src/triton_grouped_gemm.py:83-84, :96-97) and reads B and C through any
strides (:72-78).  Here any even N is read and written in place: B's and
C's rows need not be 16-byte aligned (16-byte DMAs and stores run at any
4-byte alignment), the chunk of a B row that holds column N-1 is read as it
lies (its columns past N come from the next row, or as zeros past the
buffer descriptor, never stored), and the last chunk of a C row is stored by
words.  Odd N goes through a copy of B with one zero column.

Checked against the fp64 oracle (max |C - C_fp64| <= 2e-2 * sqrt(max(K,
512)/512)), for both dtypes, N-major and K-major B, both schedules, ragged
and empty experts; through the C ABI with a NaN-filled C whose row stride
exceeds N (no store may land past column N); the empty-queue zero fill; and
fp8 against the decoded-operand bound.
"""
import math
import sys

import numpy as np
import pytest
import torch

import grouped_gemm as gg
import mgg_native as nat
from oracle import grouped_gemm_oracle as orc

pytestmark = pytest.mark.gpu


def tol(k):
    return 2e-2 * math.sqrt(max(k, 512) / 512)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def inputs(counts, k, n, dtype, device, seed):
    gen = torch.Generator().manual_seed(seed)
    a = torch.randn(int(sum(counts)), k, generator=gen).to(dtype)
    b = (torch.randn(len(counts), k, n, generator=gen) / math.sqrt(k)).to(dtype)
    offs = torch.tensor(orc.expert_offsets_from_recv_counts(counts), dtype=torch.int32)
    return a.to(device), b.to(device), offs.to(device)


def oracle(a, b, offs):
    return orc.grouped_gemm(a.float().cpu().numpy(), b.float().cpu().numpy(), offs.cpu().numpy(),
                            acc_dtype=np.float64)


COUNTS = [300, 0, 257, 1, 600]


@pytest.mark.parametrize("n", [4092, 1404, 38, 6, 2050, 37, 1401])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["n_major", "k_major"])
def test_n_not_multiple_of_8(cuda_device, n, dtype, layout):
    k = 264
    a, b, offs = inputs(COUNTS, k, n, dtype, cuda_device, seed=n)
    if layout == "k_major":
        b = b.transpose(1, 2).contiguous().transpose(1, 2)
    want = oracle(a, b, offs)
    for atomic in (False, True):  # (the atomic launches split their short last round)
        log(f"N={n} {dtype} {layout} atomic={atomic}")
        c = gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=atomic)
        torch.cuda.synchronize()
        assert c.shape == (a.shape[0], n)
        err = float(np.abs(c.float().cpu().numpy() - want).max())
        assert err <= tol(k), (atomic, err)


@pytest.mark.parametrize("n,ldc", [(4092, 4100), (38, 40), (6, 10), (1404, 1406)])
def test_c_abi_stores_stop_at_n(cuda_device, n, ldc):
    """Through the C ABI with C's row stride past N: columns N .. ldc-1 keep
    their NaNs, rows outside every expert's range too, and B is read in place
    with its own odd-looking row stride (ldb_k = N + 2)."""
    counts, k = [130, 0, 3, 70], 128
    gen = torch.Generator().manual_seed(n)
    a = torch.randn(sum(counts) + 5, k, generator=gen).to(torch.bfloat16).to(cuda_device)
    b_full = (torch.randn(len(counts), k, n + 2, generator=gen) / math.sqrt(k)).to(torch.bfloat16)
    b_full = b_full.to(cuda_device)
    b = b_full[:, :, :n]  # row stride n + 2
    offs = torch.tensor(orc.expert_offsets_from_recv_counts(counts), dtype=torch.int32,
                        device=cuda_device)
    m = a.shape[0]
    for atomic in (0, 1):
        c = torch.full((m, ldc), float("nan"), dtype=torch.bfloat16, device=cuda_device)
        nat.check(nat.lib().mgg_grouped_gemm(
            nat.MGG_DTYPE_BF16, a.data_ptr(), b.data_ptr(), c.data_ptr(), offs.data_ptr(), m, k, n,
            len(counts), a.stride(0), b.stride(0), b.stride(1), ldc, None, None, None, -1, 256,
            256, 0, atomic, None, 0, 0, torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        rows = sum(counts)
        assert bool(torch.isnan(c[:rows, n:]).all()), "a store landed past column N"
        assert bool(torch.isnan(c[rows:]).all()), "a store landed outside the experts' rows"
        want = oracle(a[:rows], b, offs)
        err = float(np.abs(c[:rows, :n].float().cpu().numpy() - want).max())
        assert err <= tol(k), (atomic, err)


def test_empty_queue_zero_fills_odd_widths(cuda_device):
    """No expert holds a row: C (N = 38, C row stride 38) is zero-filled whole,
    its last 6 columns of every row by words."""
    for n in (38, 6):
        a = torch.randn(40, 64, device=cuda_device).to(torch.bfloat16)
        b = torch.randn(3, 64, n, device=cuda_device).to(torch.bfloat16)
        offs = torch.zeros(4, dtype=torch.int32, device=cuda_device)
        for atomic in (False, True):
            c = gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=atomic)
            torch.cuda.synchronize()
            assert c.shape == (40, n) and bool((c == 0).all()), (n, atomic)


@pytest.mark.parametrize("n", [1404, 38, 37])
def test_fp8_n_not_multiple_of_8(cuda_device, n):
    counts, k = [300, 5, 0, 600], 512
    gen = torch.Generator().manual_seed(n)
    x = torch.randn(sum(counts), k, generator=gen)
    wt = torch.randn(len(counts), n, k, generator=gen) / math.sqrt(k)
    a, sa = gg.quantize_fp8_rows(x)
    b, sb = gg.quantize_fp8_rows(wt)
    offs = torch.tensor(orc.expert_offsets_from_recv_counts(counts), dtype=torch.int32)
    ref = orc.grouped_gemm_fp8(a.view(torch.uint8).numpy(), b.view(torch.uint8).numpy(),
                               offs.numpy(), sa.numpy(), sb.numpy())
    mag = orc.grouped_gemm_fp8(a.view(torch.uint8).numpy(), b.view(torch.uint8).numpy(),
                               offs.numpy(), sa.numpy(), sb.numpy(), magnitude=True)
    a, sa, b, sb, offs = (t.to(cuda_device) for t in (a, sa, b, sb, offs))
    for atomic in (False, True):
        log(f"fp8 N={n} atomic={atomic}")
        c = gg.persistent_grouped_gemm(a, b.transpose(1, 2), offs, a_scale=sa, b_scale=sb,
                                       use_atomic_queue=atomic)
        torch.cuda.synchronize()
        got = c.float().cpu().numpy()
        assert got.shape == ref.shape
        assert np.all(np.abs(got - ref) <= 2 ** -8 * np.abs(ref) + 2 ** -16 * mag), atomic
