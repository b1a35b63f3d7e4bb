"""GPU tests of the atomic schedule's split last round.

With the device-derived queue, an atomic launch whose last round holds at most
a quarter (a half) as many tiles as there are workers takes each of those
tiles as 4 (2) parts of K on as many workers.  The parts meet pairwise in a
binary tree: at each meeting the worker that arrives first writes its fp32
partial sums and the other adds them and goes on; the last meeting's winner
stores the tile.  Checked here: parity with the oracle (tolerance as in
test_gpu_gemm), a repeated launch giving the same bits (each meeting's sum does
not depend on which worker arrives first), the work_counter's W + G, flag
words left at any value by an unfinished launch, and the K-major and fp8
variants.  The reference never splits a tile (src/triton_grouped_gemm.py:157-233
takes whole items); results agree with it within the tolerance, not bitwise.
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


def make_inputs(counts, k, n, dtype, device, seed=0):
    gen = torch.Generator().manual_seed(seed)
    a = torch.randn(int(sum(counts)), k, generator=gen).to(dtype)
    b = (torch.randn(len(counts), k, n, generator=gen) / math.sqrt(k)).to(dtype)
    offs = torch.tensor(orc.expert_offsets_from_recv_counts(counts), dtype=torch.int32)
    return a.to(device), b.to(device), offs.to(device)


def assert_parity(c, a, b, offs, k):
    want = orc.grouped_gemm(a.float().cpu().numpy(), b.float().cpu().numpy(), offs.cpu().numpy(),
                            acc_dtype=np.float64)
    err = float(np.abs(c.float().cpu().numpy() - want).max())
    assert err <= tol(k), f"max abs err {err} > {tol(k)}"


def tiles(counts, n, bm, bn):
    return sum((c + bm - 1) // bm for c in counts if c > 0) * ((n + bn - 1) // bn)


def split_parts(w, g, k, gran=64, min_k=1024):
    """(tiles split, parts per tile) of the atomic schedule's last round: the
    most parts s in (4, 3, 2) with s * rem <= g and at least min_k of K per
    part (16 granules, the 64-deep A blocks of the 256x256 tile)."""
    rem = w % g if w > g else w
    n_gran = -(-k // gran)
    for s in (4, 3, 2):
        if 0 < rem and s * rem <= g and n_gran >= -(-min_k // gran) * s:
            return rem, s
    return 0, 1


# (counts, K, N, workers): 24 tiles of 256x256 on 256 workers (all split in
# 4), on 20 (4 tiles past the full round, in 4), 7 (3 tiles in 2), 30 (24 >
# 15: whole); K = 2056: 3 tiles in halves of 1216 and 840 (a partial
# stage); K = 4104: 3 tiles in quarters of 1408, 1024, 1024 and 648; 28
# tiles on 12 workers: two static rounds, then the 4 tiles past them in
# thirds (3 * 4 <= 12 < 4 * 4), of K = 3144 (1280, 960, 904) and K = 3100
# (1280, 896, 924); 40 whole 256-row m-tiles on 12 workers: three static
# rounds (stripes, no ticket), then the 4 tiles past them in thirds.  (An
# even cut would give each part at least 1024 of K; part q is cut 384 of K
# shorter per bit set in q.)
CASES = [([300, 0, 257, 1, 600], 4104, 520, 256),
         ([300, 0, 257, 1, 600], 4104, 520, 20),
         ([300, 0, 257, 1, 600], 4104, 520, 7),
         ([300, 0, 257, 1, 600], 4104, 520, 30),
         ([64] * 3, 2056, 256, 256),
         ([64] * 3, 4104, 256, 256),
         ([256] * 27 + [5], 3144, 256, 12),
         ([256] * 27 + [5], 3100, 256, 12),
         ([256] * 40, 3144, 256, 12)]
EXPECT_PARTS = [4, 4, 2, 1, 2, 4, 3, 3, 3]


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_split_last_round(cuda_device, case, dtype):
    counts, k, n, g = CASES[case]
    a, b, offs = make_inputs(counts, k, n, dtype, cuda_device, seed=case)
    w = tiles(counts, n, 256, 256)
    n_split, parts = split_parts(w, g, k)
    assert parts == EXPECT_PARTS[case]
    log(f"split case={case} W={w} G={g} split tiles={n_split} parts={parts} dtype={dtype}")
    counter = torch.zeros(1, dtype=torch.int32, device=cuda_device)
    c = gg.persistent_grouped_gemm(a, b, offs, num_sms=g, block_m=256, block_n=256,
                                   work_counter=counter)
    torch.cuda.synchronize()
    assert counter.item() == w + g  # the reference's count for the requested tile
    assert_parity(c, a, b, offs, k)
    for rep in range(3):
        again = gg.persistent_grouped_gemm(a, b, offs, num_sms=g)
        torch.cuda.synchronize()
        assert torch.equal(again, c), rep
    whole = gg.persistent_grouped_gemm(a, b, offs, num_sms=g, use_atomic_queue=False)
    torch.cuda.synchronize()
    if n_split == 0:
        assert torch.equal(whole, c)
    elif case == 0:  # 24 split tiles of random sums: some output rounds differently
        assert not torch.equal(whole, c)


@pytest.mark.parametrize("poison", [0xFFFFFFFFFFFFFFFF, 0x0000000100000001, 0x7FFFFFFF00000001,
                                    0x0000000000000005])
def test_split_flags_left_dirty(cuda_device, poison):
    """Flag words left at any value (as a launch that did not finish could
    leave them) neither lose a half's partial sums nor add them twice."""
    counts, k, n = [300, 0, 257, 1, 600], 4104, 520
    a, b, offs = make_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=3)
    stream = torch.cuda.current_stream().cuda_stream
    clean = gg.persistent_grouped_gemm(a, b, offs)  # also creates this stream's split workspace
    torch.cuda.synchronize()
    assert_parity(clean, a, b, offs, k)
    for rep in range(2):
        nat.check(nat.lib().mgg_debug_set_split_flags(poison, stream))
        got = gg.persistent_grouped_gemm(a, b, offs)
        torch.cuda.synchronize()
        log(f"poison={poison:#x} rep={rep}")
        assert torch.equal(got, clean), rep


def test_split_kmajor_b_matches_nmajor(cuda_device):
    """K-major B (a [E, K, N] view of [E, N, K] memory) splits at the same K
    and gives the same bits as N-major B."""
    counts, k, n = [300, 0, 257, 1, 600], 4104, 520
    a, b, offs = make_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=4)
    b_km = b.transpose(1, 2).contiguous().transpose(1, 2)
    for tile in ((256, 256), (128, 128)):
        c_n = gg.persistent_grouped_gemm(a, b, offs, kernel_tile=tile)
        c_k = gg.persistent_grouped_gemm(a, b_km, offs, kernel_tile=tile)
        torch.cuda.synchronize()
        assert_parity(c_k, a, b, offs, k)
        assert torch.equal(c_k, c_n), tile


def test_split_fp8(cuda_device):
    """fp8 (12 tiles of 256x256, K = 8192: quarters, each at least 2048 deep):
    the parts' sums are unscaled; the worker that completes the last meeting
    applies the row and column scales once, after adding them."""
    counts, k, n = [300, 5, 0, 600], 8192, 384
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(sum(counts), k, generator=gen)
    wt = torch.randn(len(counts), n, k, generator=gen) / math.sqrt(k)
    a, sa = gg.quantize_fp8_rows(x)
    b, sb = gg.quantize_fp8_rows(wt)
    offs = torch.tensor(orc.expert_offsets_from_recv_counts(counts), dtype=torch.int32)
    a, sa, b, sb, offs = (t.to(cuda_device) for t in (a, sa, b, sb, offs))
    ref = orc.grouped_gemm_fp8(a.cpu().view(torch.uint8).numpy(), b.cpu().view(torch.uint8).numpy(),
                               offs.cpu().numpy(), sa.cpu().numpy(), sb.cpu().numpy())
    mag = orc.grouped_gemm_fp8(a.cpu().view(torch.uint8).numpy(), b.cpu().view(torch.uint8).numpy(),
                               offs.cpu().numpy(), sa.cpu().numpy(), sb.cpu().numpy(), magnitude=True)
    outs = []
    for rep in range(2):
        c = gg.persistent_grouped_gemm(a, b.transpose(1, 2), offs, a_scale=sa, b_scale=sb,
                                       kernel_tile=(256, 256))
        torch.cuda.synchronize()
        got = c.float().cpu().numpy()
        assert np.all(np.abs(got - ref) <= 2 ** -8 * np.abs(ref) + 2 ** -16 * mag)
        outs.append(c)
    assert torch.equal(outs[0], outs[1])


def test_split_switched_off_takes_whole_tiles(cuda_device):
    """set_split_last_round(False): the atomic call takes every tile whole and
    gives the striped call's bits; switched back on it splits again."""
    counts, k, n, g = CASES[0]
    a, b, offs = make_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=0)
    striped = gg.persistent_grouped_gemm(a, b, offs, num_sms=g, use_atomic_queue=False)
    split = gg.persistent_grouped_gemm(a, b, offs, num_sms=g)
    try:
        gg.set_split_last_round(False)
        whole = gg.persistent_grouped_gemm(a, b, offs, num_sms=g)
    finally:
        gg.set_split_last_round(True)
    again = gg.persistent_grouped_gemm(a, b, offs, num_sms=g)
    torch.cuda.synchronize()
    assert torch.equal(whole, striped)
    assert not torch.equal(split, striped)  # 24 tiles of random sums split in 4
    assert torch.equal(again, split)


def test_captured_split_call_agrees_with_eager(cuda_device):
    """A call that splits eagerly takes whole tiles under graph capture: every
    replay gives the striped call's bits and agrees with the eager split call
    within the tolerance (both checked against the oracle)."""
    counts, k, n, g = CASES[0]
    a, b, offs = make_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=1)
    eager = gg.persistent_grouped_gemm(a, b, offs, num_sms=g)
    striped = gg.persistent_grouped_gemm(a, b, offs, num_sms=g, use_atomic_queue=False)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = gg.persistent_grouped_gemm(a, b, offs, num_sms=g)
    for rep in range(3):
        graph.replay()
        other = gg.persistent_grouped_gemm(a, b, offs, num_sms=g)  # eager split work between
        torch.cuda.synchronize()
        log(f"captured split rep={rep}")
        assert torch.equal(captured, striped), rep
        assert torch.equal(other, eager), rep
        err = (captured.float() - eager.float()).abs().max().item()
        assert err <= tol(k), err
    assert_parity(eager, a, b, offs, k)
    assert_parity(captured, a, b, offs, k)


def test_reserve_split_workspace_refused_under_capture(cuda_device):
    """Reserving the workspace would allocate and clear flags inside the
    capture: refused with an error, the capture itself unharmed."""
    counts, k, n, g = CASES[0]
    a, b, offs = make_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=3)
    striped = gg.persistent_grouped_gemm(a, b, offs, num_sms=g, use_atomic_queue=False)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        with pytest.raises(nat.NativeError, match="graph capture"):
            gg.reserve_split_workspace(cuda_device)
        captured = gg.persistent_grouped_gemm(a, b, offs, num_sms=g)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(captured, striped)


def test_split_workspace_is_one_slot_per_cu(cuda_device):
    """The split workspace of a stream holds one 256 x 256 fp32 slot and one
    flag word per CU, whatever the worker count: 64 MiB on a 256-CU device
    after a num_sms=1000 call (24 tiles in 4 parts), and reserving it again
    changes nothing."""
    counts, k, n = [300, 0, 257, 1, 600], 4104, 520
    a, b, offs = make_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=2)
    gg.reserve_split_workspace(cuda_device)
    c = gg.persistent_grouped_gemm(a, b, offs, num_sms=1000)
    torch.cuda.synchronize()
    assert_parity(c, a, b, offs, k)
    cus = gg._cu_count(cuda_device.index or 0)
    want = cus * (256 * 256 * 4 + 8)
    assert gg.split_workspace_bytes(cuda_device) == want
    assert want <= 64 * 2 ** 20 + 8 * 256 or cus > 256
    gg.reserve_split_workspace(cuda_device)
    assert gg.split_workspace_bytes(cuda_device) == want
