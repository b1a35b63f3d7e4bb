"""GPU parity for N not a multiple of 8, odd N included.

The reference's Triton kernel masks the N edge in its loads and its store
(src/triton_grouped_gemm.py:83-84, :96-97) and reads B and C through any
strides (:72-78).  Here any N is read and written in place: B's and C's rows
need not be 16-byte aligned (16-byte DMAs and stores run at any 2-byte
alignment), the chunk of a B row that holds column N-1 is read as it lies
(its columns past N come from the next row, or as zeros past the buffer
descriptor, never stored), and the last chunk of a C row is stored by pairs
and, for odd N, one 2-byte store.  With odd N the range check would zero the
dword that holds B's very last element (it straddles the end of B's view):
the kernel adds that element's term A[r][K-1] * B[e][K-1][N-1] itself.

Checked against the fp64 oracle (max |C - C_fp64| <= 2e-2 * sqrt(max(K,
512)/512)), for both dtypes, N-major and K-major B, both schedules, ragged
and empty experts; through the C ABI with a NaN-filled C whose row stride
exceeds N (no store may land past column N); the empty-queue zero fill; fp8
against the decoded-operand bound; and B's last element made large (4.0
against A's 1.0) so that a dropped term shows, with B exactly allocated,
shared by every expert (stride 0), in split tiles, and in the gathered
GELU up GEMM of the expert MLP.
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
    for atomic in (False, True):
        log(f"N={n} {dtype} {layout} atomic={atomic}")
        c = gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=atomic)
        torch.cuda.synchronize()
        assert c.shape == (a.shape[0], n)
        err = float(np.abs(c.float().cpu().numpy() - want).max())
        assert err <= tol(k), (atomic, err)


@pytest.mark.parametrize("n,ldc", [(4092, 4100), (38, 40), (6, 10), (1404, 1406), (37, 41),
                                   (1401, 1402), (7, 7), (3, 9)])
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
    """No expert holds a row: C (N = 38, 6, 37, 1; row stride N) is
    zero-filled whole, its last columns of every row by elements."""
    for n in (38, 6, 37, 1):
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


def last_element_inputs(counts, k, n, dtype, device, seed):
    """Inputs whose B[-1][K-1][N-1] is 4.0 and A[:, K-1] is 1.0, so the term
    the kernel adds itself moves C[:, N-1] of the last expert's rows by 4."""
    a, b, offs = inputs(counts, k, n, dtype, "cpu", seed)
    a[:, k - 1] = 1.0
    b[-1, k - 1, n - 1] = 4.0
    return a.to(device), b.to(device), offs.to(device)


@pytest.mark.parametrize("n", [1, 7, 37, 255, 257, 1401])
@pytest.mark.parametrize("k", [13, 264])
@pytest.mark.parametrize("tile", [(256, 256), (128, 512), (128, 128), (64, 64), (256, 128)])
def test_odd_n_last_element_of_b(cuda_device, n, k, tile):
    """(Tiles without an odd-N instance compute on the nearest that has one.)"""
    counts = [70, 0, 300, 1, 260]
    a, b, offs = last_element_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=n + k)
    want = oracle(a, b, offs)
    for atomic in (False, True):
        log(f"odd N last element N={n} K={k} tile={tile} atomic={atomic}")
        c = gg.persistent_grouped_gemm(a, b, offs, kernel_tile=tile, use_atomic_queue=atomic)
        torch.cuda.synchronize()
        err = float(np.abs(c.float().cpu().numpy() - want).max())
        assert err <= tol(k), (atomic, err)


@pytest.mark.parametrize("n", [37, 1401])
def test_odd_n_b_shared_by_experts(cuda_device, n):
    """B with expert stride 0 (one weight expanded over every expert): every
    expert's last element is B's last element."""
    counts, k = [70, 0, 300, 1, 260], 264
    gen = torch.Generator().manual_seed(n)
    a = torch.randn(sum(counts), k, generator=gen).to(torch.bfloat16)
    a[:, k - 1] = 1.0
    w = (torch.randn(k, n, generator=gen) / math.sqrt(k)).to(torch.bfloat16)
    w[k - 1, n - 1] = 4.0
    offs = torch.tensor(orc.expert_offsets_from_recv_counts(counts), dtype=torch.int32)
    want = oracle(a, w[None].expand(len(counts), k, n), offs)
    a, w, offs = a.to(cuda_device), w.to(cuda_device), offs.to(cuda_device)
    b = w[None].expand(len(counts), k, n)
    assert b.stride(0) == 0
    for atomic in (False, True):
        log(f"odd N shared B N={n} atomic={atomic}")
        c = gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=atomic)
        torch.cuda.synchronize()
        err = float(np.abs(c.float().cpu().numpy() - want).max())
        assert err <= tol(k), (atomic, err)


@pytest.mark.parametrize("counts,num_sms", [([300, 0, 257, 200], 4), ([300, 0, 257, 200], 2),
                                            ([300, 257], 3), ([1, 0, 0, 200], 8)])
def test_odd_n_split_tiles(cuda_device, counts, num_sms):
    """The atomic schedule's split last round with odd N (256x256 tiles, one
    n-tile): 5 tiles on 4 workers take the last one, the last expert's, in 4
    K parts; 5 on 2 in 2 parts; 4 on 3 in 3 parts; 2 on 8 both in 4 parts.
    The last part's descriptor stops at B's last element (K = 4104: each part
    at least 1024 deep)."""
    k, n = 4104, 201
    a, b, offs = last_element_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=num_sms)
    want = oracle(a, b, offs)
    log(f"odd N split counts={counts} num_sms={num_sms}")
    c = gg.persistent_grouped_gemm(a, b, offs, num_sms=num_sms, kernel_tile=(256, 256))
    torch.cuda.synchronize()
    err = float(np.abs(c.float().cpu().numpy() - want).max())
    assert err <= tol(k), err


@pytest.mark.parametrize("f", [75, 201])
def test_odd_ffn_gelu_mlp(cuda_device, f):
    """Expert MLP with GELU and an odd FFN width: the up GEMM reads its rows
    through the layout (gathered A) with odd N, the down GEMM has odd K."""
    import expert_mlp as mlp
    from oracle import expert_mlp_oracle as mo
    T, k, E, H = 300, 2, 5, 136
    gen = torch.Generator().manual_seed(f)
    idx = torch.randint(0, E, (T, k), generator=gen)
    w = torch.rand(T, k, generator=gen)
    x = torch.randn(T, H, generator=gen).to(torch.bfloat16)
    w1 = (torch.randn(E, H, f, generator=gen) / math.sqrt(H)).to(torch.bfloat16)
    w2 = (torch.randn(E, f, H, generator=gen) / math.sqrt(f)).to(torch.bfloat16)
    w1[-1, H - 1, f - 1] = 4.0
    assert mlp._gathered_ok(x.to(cuda_device), w1.to(cuda_device), 256)
    log(f"odd FFN GELU MLP F={f}")
    got = mlp.expert_mlp_forward(x.to(cuda_device), idx.to(cuda_device), w.to(cuda_device),
                                 w1.to(cuda_device), w2.to(cuda_device), "gelu",
                                 block=256).float().cpu().numpy()
    ref = mo.expert_mlp(x.float().numpy(), idx.numpy(), w.numpy(), w1.float().numpy(),
                        w2.float().numpy(), "gelu")
    err = np.abs(got - ref)
    assert err.max() <= 2 * tol(f), err.max()
