"""GPU tests of the gathered up GEMM (mgg_grouped_gemm_gathered): A's rows
read from a token matrix through an index array in the GEMM's own DMAs.

The reference gathers first (grouped_tokens = valid_tokens[perm],
src/train_moe_baseline.py:224) and multiplies the gathered matrix
(:239-241); the fused launch must give bitwise what mgg_grouped_gemm_ex
gives on that gathered matrix, tile for tile and schedule for schedule
(striped, atomic, with the atomic schedule's split last round), for every
epilogue, and agree with the oracle.  Indices outside the source matrix read
zeros.  Every call goes through the C ABI.
"""
import math
import sys

import numpy as np
import pytest
import torch

import expert_mlp as mlp
import mgg_native as nat
from oracle import grouped_gemm_oracle as orc

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def gathered(x, rows, w, offs, epi, out_cols, workers, atomic):
    m = rows.numel()
    c = torch.full((m, out_cols), float("nan"), dtype=x.dtype, device=x.device)
    nat.check(nat.lib().mgg_grouped_gemm_gathered(
        mlp._DTYPES[x.dtype], epi, x.data_ptr(), rows.data_ptr(), x.shape[0], w.data_ptr(),
        c.data_ptr(), offs.data_ptr(), m, x.shape[1], w.shape[2], w.shape[0], x.stride(0),
        w.stride(0), w.stride(1), c.stride(0), workers, atomic,
        torch.cuda.current_stream().cuda_stream))
    return c


def explicit(xg, w, offs, epi, out_cols, workers, atomic):
    m = xg.shape[0]
    c = torch.full((m, out_cols), float("nan"), dtype=xg.dtype, device=xg.device)
    nat.check(nat.lib().mgg_grouped_gemm_ex(
        mlp._DTYPES[xg.dtype], epi, xg.data_ptr(), w.data_ptr(), c.data_ptr(), offs.data_ptr(), m,
        xg.shape[1], w.shape[2], w.shape[0], xg.stride(0), w.stride(0), w.stride(1), c.stride(0),
        None, None, None, -1, 256, 256, workers, atomic, None, 0, 0,
        torch.cuda.current_stream().cuda_stream))
    return c


# (counts, T source rows, K, N, workers; 0 = the CU count): ragged experts
# with an empty one, a one-row expert and a partial K stage.  Atomic launches
# split their last round: case 0 its 16 tiles in 4 parts, case 1 (7 workers)
# the 2 tiles past two rounds in thirds, case 2 (K = 264) its 5 tiles in
# halves, case 3 its 64 tiles in 4 parts.
CASES = [([300, 0, 257, 1, 600], 700, 1032, 512, 0),
         ([300, 0, 257, 1, 600], 700, 1032, 512, 7),
         ([64, 520, 3], 97, 264, 256, 0),
         ([1024] * 4, 2048, 2048, 1024, 0)]


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("epi", [nat.MGG_EPI_NONE, nat.MGG_EPI_GELU, nat.MGG_EPI_SWIGLU])
@pytest.mark.parametrize("atomic", [0, 1])
def test_gathered_matches_explicit_gather(cuda_device, case, epi, atomic):
    counts, t, k, n, workers = CASES[case]
    log(f"gathered case={case} epi={epi} atomic={atomic}")
    gen = torch.Generator().manual_seed(case)
    m = sum(counts)
    x = torch.randn(t, k, generator=gen).to(torch.bfloat16).to(cuda_device)
    rows = torch.randint(0, t, (m,), generator=gen, dtype=torch.int32).to(cuda_device)
    w = (torch.randn(len(counts), k, n, generator=gen) / math.sqrt(k)).to(torch.bfloat16)
    w = w.to(cuda_device)
    offs = torch.tensor(orc.expert_offsets_from_recv_counts(counts), dtype=torch.int32,
                        device=cuda_device)
    out_cols = n // 2 if epi == nat.MGG_EPI_SWIGLU else n
    got = gathered(x, rows, w, offs, epi, out_cols, workers, atomic)
    want = explicit(x[rows.long()].contiguous(), w, offs, epi, out_cols, workers, atomic)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    if epi == nat.MGG_EPI_NONE and case < 3:
        ref = orc.grouped_gemm(x[rows.long()].float().cpu().numpy(), w.float().cpu().numpy(),
                               offs.cpu().numpy(), acc_dtype=np.float64)
        err = float(np.abs(got.float().cpu().numpy() - ref).max())
        assert err <= 2e-2 * math.sqrt(max(k, 512) / 512), err


def test_gathered_out_of_range_rows_read_zeros(cuda_device):
    """Indices below 0 or at/after the source row count give rows of zeros."""
    counts, t, k, n = [200, 90], 50, 520, 256
    gen = torch.Generator().manual_seed(7)
    m = sum(counts)
    x = torch.randn(t, k, generator=gen).to(torch.float16).to(cuda_device)
    rows = torch.randint(0, t, (m,), generator=gen, dtype=torch.int32)
    bad = torch.arange(0, m, 7)
    rows[bad] = torch.tensor([-1, t, t + 1000, -(2 ** 31)], dtype=torch.int32).repeat(len(bad))[:len(bad)]
    rows = rows.to(cuda_device)
    w = (torch.randn(2, k, n, generator=gen) / math.sqrt(k)).to(torch.float16).to(cuda_device)
    offs = torch.tensor(orc.expert_offsets_from_recv_counts(counts), dtype=torch.int32,
                        device=cuda_device)
    xg = torch.zeros(m, k, dtype=x.dtype, device=cuda_device)
    ok = (rows >= 0) & (rows < t)
    xg[ok] = x[rows[ok].long()]
    for atomic in (0, 1):
        got = gathered(x, rows, w, offs, nat.MGG_EPI_NONE, n, 0, atomic)
        want = explicit(xg, w, offs, nat.MGG_EPI_NONE, n, 0, atomic)
        torch.cuda.synchronize()
        assert torch.equal(got, want), atomic
        assert torch.count_nonzero(got[bad.to(cuda_device)]) == 0


def test_gathered_offsets_past_m_read_only_m_indices(cuda_device):
    """Expert offsets that run past M (offsets[E] > m_size) cover only the
    first M rows: the launch reads no index at or past M (the index array here
    is longer, so the launch stays inside it either way) and rows < M equal
    the explicit gather's, which clamps A's rows at M."""
    counts, t, k, n = [200, 90], 300, 264, 256
    m = 250  # offsets end at 290
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(t, k, generator=gen).to(torch.bfloat16).to(cuda_device)
    rows = torch.randint(0, t, (sum(counts) + 64,), generator=gen, dtype=torch.int32)
    rows = rows.to(cuda_device)
    w = (torch.randn(2, k, n, generator=gen) / math.sqrt(k)).to(torch.bfloat16).to(cuda_device)
    offs = torch.tensor(orc.expert_offsets_from_recv_counts(counts), dtype=torch.int32,
                        device=cuda_device)
    xg = x[rows[:m].long()].contiguous()
    for atomic in (0, 1):
        log(f"gathered offsets past M atomic={atomic}")
        got = torch.full((m, n), float("nan"), dtype=x.dtype, device=cuda_device)
        nat.check(nat.lib().mgg_grouped_gemm_gathered(
            nat.MGG_DTYPE_BF16, nat.MGG_EPI_NONE, x.data_ptr(), rows.data_ptr(), t, w.data_ptr(),
            got.data_ptr(), offs.data_ptr(), m, k, n, 2, x.stride(0), w.stride(0), w.stride(1),
            got.stride(0), 0, atomic, torch.cuda.current_stream().cuda_stream))
        want = explicit(xg, w, offs, nat.MGG_EPI_NONE, n, 0, atomic)
        torch.cuda.synchronize()
        assert torch.equal(got, want), atomic
