"""Seeded random shapes through the drop-in and the gathered up GEMM.

Each case draws an expert count, ragged row counts (empty and one-row experts
included), K (multiples of 8 and K tails), N, the kernel tile, the schedule
and the worker count (so the atomic schedule's split last round, at 2 or 4
parts, comes up with many tile and worker counts).  The drop-in's result is
checked against an fp32 per-expert matmul on the GPU within north_star's
tolerance (the reference's per-expert loop, src/triton_grouped_gemm.py:446-457,
in fp32); where the shape allows the gathered up GEMM, it must give bitwise
what mgg_grouped_gemm_ex gives on the gathered matrix.
"""
import math
import random
import sys

import pytest
import torch

import expert_mlp as mlp
import grouped_gemm as gg
import mgg_native as nat

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def draw_case(rng):
    e = rng.randint(1, 12)
    counts = [rng.choice([0, 1, rng.randint(1, 300), rng.randint(100, 520)]) for _ in range(e)]
    k = rng.choice([rng.randint(1, 1500), 8 * rng.randint(1, 190)])
    n = 8 * rng.randint(1, 66)
    tile = rng.choice([None, (256, 256), (128, 128), (256, 128), (64, 64)])
    atomic = rng.random() < 0.6
    sms = rng.choice([None, rng.randint(1, 300)])
    dtype = rng.choice([torch.bfloat16, torch.float16])
    return counts, k, n, tile, atomic, sms, dtype


@pytest.mark.parametrize("seed", range(24))
def test_random_case(cuda_device, seed):
    rng = random.Random(1000 + seed)
    counts, k, n, tile, atomic, sms, dtype = draw_case(rng)
    m = sum(counts)
    log(f"sweep seed={seed} counts={counts} K={k} N={n} tile={tile} atomic={atomic} sms={sms} {dtype}")
    gen = torch.Generator().manual_seed(seed)
    a = torch.randn(m, k, generator=gen).to(dtype).to(cuda_device)
    b = (torch.randn(len(counts), k, n, generator=gen) / math.sqrt(k)).to(dtype).to(cuda_device)
    offs = gg.expert_offsets_from_recv_counts(counts, device=cuda_device)
    kw = dict(use_atomic_queue=atomic, num_sms=sms)
    if tile is not None:
        kw["kernel_tile"] = tile
    c = gg.persistent_grouped_gemm(a, b, offs, **kw)
    o = offs.tolist()
    tol = 2e-2 * math.sqrt(max(k, 512) / 512)
    for e in range(len(counts)):
        if o[e + 1] > o[e]:
            want = a[o[e]:o[e + 1]].float() @ b[e].float()
            err = (c[o[e]:o[e + 1]].float() - want).abs().max().item()
            assert err <= tol, (e, err, tol)
    if m == 0:
        return
    # The gathered up GEMM on the same routing: K rounded up to 8 (its DMAs
    # read whole 16-byte chunks of x's rows) and N a multiple of 64 (SwiGLU).
    kg, ng = (k + 7) // 8 * 8, 64 * rng.randint(1, 8)
    t = rng.randint(1, 2 * m)
    x = torch.randn(t, kg, generator=gen).to(dtype).to(cuda_device)
    w = (torch.randn(len(counts), kg, ng, generator=gen) / math.sqrt(kg)).to(dtype).to(cuda_device)
    rows = torch.randint(0, t, (m,), generator=gen, dtype=torch.int32).to(cuda_device)
    epi = rng.choice([nat.MGG_EPI_NONE, nat.MGG_EPI_GELU, nat.MGG_EPI_SWIGLU])
    oc = ng // 2 if epi == nat.MGG_EPI_SWIGLU else ng
    log(f"  gathered K={kg} N={ng} epi={epi} T={t}")
    stream = torch.cuda.current_stream().cuda_stream
    got = torch.empty(m, oc, dtype=dtype, device=cuda_device)
    nat.check(nat.lib().mgg_grouped_gemm_gathered(
        mlp._DTYPES[dtype], epi, x.data_ptr(), rows.data_ptr(), t, w.data_ptr(), got.data_ptr(),
        offs.data_ptr(), m, kg, ng, len(counts), x.stride(0), w.stride(0), w.stride(1),
        got.stride(0), int(sms or 0), int(atomic), stream))
    xg = x[rows.long()].contiguous()
    want = torch.empty(m, oc, dtype=dtype, device=cuda_device)
    nat.check(nat.lib().mgg_grouped_gemm_ex(
        mlp._DTYPES[dtype], epi, xg.data_ptr(), w.data_ptr(), want.data_ptr(), offs.data_ptr(), m,
        kg, ng, len(counts), xg.stride(0), w.stride(0), w.stride(1), want.stride(0), None, None,
        None, -1, 256, 256, int(sms or 0), int(atomic), None, 0, 0, stream))
    torch.cuda.synchronize()
    assert torch.equal(got, want)
