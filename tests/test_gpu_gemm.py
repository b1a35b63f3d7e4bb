"""GPU parity of the HIP grouped GEMM (through libmgg's C ABI) against the CPU
oracle, plus the kernel's scheduling and counter semantics.

Tolerance (benchmark's stated): max |C - C_fp32| <= 2e-2 * sqrt(K / 512) for
bf16/fp16 outputs against an fp32/fp64 reference on the same (already
rounded) inputs, over every row inside an expert range.  K is floored at 512
in the formula: with N(0, 1/K) weights the outputs are O(1) at every K, and
rounding them to bf16 alone costs up to half an ulp, 2^-6 = 0.0156 for
|y| in [4, 8), which is above 2e-2 * sqrt(K/512) for K < 512.  Every
benchmark config has K >= 512, where the formula applies unchanged.
"""
import ctypes
import math
import sys

import numpy as np
import pytest
import torch

import grouped_gemm as gg
import mgg_native as nat
import workloads
from oracle import grouped_gemm_oracle as orc

pytestmark = pytest.mark.gpu


def tol(k):
    return 2e-2 * math.sqrt(max(k, 512) / 512)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_inputs(counts, k, n, dtype, device, seed=0, extra_rows=0):
    gen = torch.Generator().manual_seed(seed)
    m = int(sum(counts)) + extra_rows
    a = torch.randn(m, k, generator=gen).to(dtype)
    b = (torch.randn(len(counts), k, n, generator=gen) / math.sqrt(max(k, 1))).to(dtype)
    offs = torch.tensor(orc.expert_offsets_from_recv_counts(counts), dtype=torch.int32)
    return a.to(device), b.to(device), offs.to(device)


def oracle_out(a, b, offs, rows=None):
    a32 = a.float().cpu().numpy()
    b32 = b.float().cpu().numpy()
    return orc.grouped_gemm(a32, b32, offs.cpu().numpy(), acc_dtype=np.float64)


def covered_rows(offs):
    o = offs.cpu().numpy().astype(np.int64)
    mask = np.zeros(int(max(o.max(initial=0), 0)), bool)
    for e in range(len(o) - 1):
        if o[e + 1] > o[e]:
            mask[o[e]:o[e + 1]] = True
    return mask


def assert_parity(c, a, b, offs, k):
    want = oracle_out(a, b, offs)
    mask = covered_rows(offs)
    got = c.float().cpu().numpy()[: mask.size][mask]
    ref = want[: mask.size][mask]
    err = float(np.abs(got - ref).max()) if got.size else 0.0
    assert np.isfinite(got).all()
    assert err <= tol(k), f"max abs err {err} > {tol(k)}"
    return err


SMALL_CASES = [
    # counts, K, N
    ([3, 0, 5], 64, 64),
    ([1, 200, 0, 77, 300], 128, 192),
    ([0, 0, 513, 0], 256, 136),          # one ragged expert, N edge inside a tile
    ([130, 1, 257], 72, 64),             # K tail (72 = 64 + 8)
    ([64] * 4, 2048, 256),
    ([600], 520, 520),
]


@pytest.mark.parametrize("case", range(len(SMALL_CASES)))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_small_ragged_parity_all_modes(cuda_device, case, dtype):
    counts, k, n = SMALL_CASES[case]
    a, b, offs = make_inputs(counts, k, n, dtype, cuda_device, seed=case, extra_rows=3)
    outs = {}
    for blocks in [(256, 256), (128, 128), (64, 64), (256, 128), (128, 256), (64, 256), (128, 512)]:
        for atomic in (False, True):
            for queue in ("device", "prebuilt"):
                log(f"case={case} dtype={dtype} blocks={blocks} atomic={atomic} queue={queue}")
                c = gg.persistent_grouped_gemm(a, b, offs, kernel_tile=blocks,
                                               use_atomic_queue=atomic, queue=queue)
                torch.cuda.synchronize()
                assert_parity(c, a, b, offs, k)
                outs[(blocks, atomic, queue)] = c
    # A launch that takes every tile whole computes each tile the same way
    # whatever the schedule or queue: those outputs are bitwise equal.  An
    # atomic launch with the device-derived queue takes its last round's tiles
    # in two halves of K when they are at most half the workers (two fp32
    # partial sums added once: another rounding); it is checked against the
    # oracle above, and repeats itself bitwise.
    mask = torch.from_numpy(covered_rows(offs)).to(cuda_device)
    for blocks in [(256, 256), (128, 128), (128, 512)]:
        ref = outs[(blocks, False, "device")][: mask.numel()][mask]
        for atomic, queue in ((False, "prebuilt"), (True, "prebuilt")):
            got = outs[(blocks, atomic, queue)][: mask.numel()][mask]
            assert torch.equal(got, ref), (blocks, atomic, queue)
        again = gg.persistent_grouped_gemm(a, b, offs, kernel_tile=blocks, use_atomic_queue=True)
        assert torch.equal(again[: mask.numel()][mask],
                           outs[(blocks, True, "device")][: mask.numel()][mask]), blocks


# K values around the 256x256 tile's staging: A moves in 64-deep blocks and B
# in 32-deep stages, so K = 8 and 40 end inside a B stage, 32 and 96 give an
# odd stage count (half an A block at the end), 64 and 128 whole blocks, 72 and
# 136 one stage past a block, 2056 a long loop with a tail.
ABLOCK_KS = [8, 32, 40, 64, 72, 96, 128, 136, 2056]


@pytest.mark.parametrize("k", ABLOCK_KS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_k_staging_edges_256x256(cuda_device, k, dtype):
    counts = [300, 0, 257, 1, 512]
    n = 264
    a, b, offs = make_inputs(counts, k, n, dtype, cuda_device, seed=k, extra_rows=5)
    outs = []
    for atomic, queue in ((False, "device"), (True, "device"), (True, "prebuilt"), (True, "device")):
        log(f"k={k} dtype={dtype} atomic={atomic} queue={queue}")
        c = gg.persistent_grouped_gemm(a, b, offs, kernel_tile=(256, 256), use_atomic_queue=atomic,
                                       queue=queue)
        torch.cuda.synchronize()
        assert_parity(c, a, b, offs, k)
        outs.append(c)
    # Whole tiles: bitwise equal across schedules; the atomic device-queue
    # launch (whose last round may be split in K) repeats itself bitwise.
    mask = torch.from_numpy(covered_rows(offs)).to(cuda_device)
    assert torch.equal(outs[0][: mask.numel()][mask], outs[2][: mask.numel()][mask])
    assert torch.equal(outs[1][: mask.numel()][mask], outs[3][: mask.numel()][mask])


def random_case(seed):
    """A seeded random problem: 1-9 experts with counts in [0, 600] (some
    empty, some a single row), K in [8, 1200] and N in [8, 700] (multiples of
    8, so tails inside a K stage and a column tile are common)."""
    rng = np.random.default_rng(seed)
    e = int(rng.integers(1, 10))
    counts = rng.integers(0, 601, e)
    counts[rng.random(e) < 0.25] = 0
    counts[rng.random(e) < 0.15] = 1
    k = 8 * int(rng.integers(1, 151))
    n = 8 * int(rng.integers(1, 88))
    blocks = [(256, 256), (128, 128), (256, 128), (128, 256), (64, 64), (64, 128), (128, 64),
              (256, 64), (64, 256), (128, 512)][int(rng.integers(0, 10))]
    return counts.tolist(), k, n, blocks


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_match_oracle(cuda_device, seed):
    counts, k, n, blocks = random_case(seed)
    log(f"random seed={seed} counts={counts} K={k} N={n} blocks={blocks}")
    dtype = torch.bfloat16 if seed % 2 == 0 else torch.float16
    a, b, offs = make_inputs(counts, k, n, dtype, cuda_device, seed=100 + seed, extra_rows=seed % 3)
    outs = []
    for atomic in (False, True):
        for queue in ("device", "prebuilt"):
            c = gg.persistent_grouped_gemm(a, b, offs, kernel_tile=blocks,
                                           use_atomic_queue=atomic, queue=queue,
                                           num_sms=int(7 + 37 * seed) % 300 + 1)
            torch.cuda.synchronize()
            outs.append(c)
    assert_parity(outs[0], a, b, offs, k)
    assert_parity(outs[2], a, b, offs, k)  # atomic, device queue: last round maybe split in K
    mask = torch.from_numpy(covered_rows(offs)).to(cuda_device)
    for c in (outs[1], outs[3]):  # whole tiles: bitwise equal to the striped device-queue result
        assert torch.equal(c[: mask.numel()][mask], outs[0][: mask.numel()][mask])


def test_cpu_plumbing_config_in_bf16(cuda_device):
    case = workloads.make_case("cpu_plumbing", device="cpu", dtype=torch.bfloat16)
    offs = gg.expert_offsets_from_recv_counts(case.counts, device=cuda_device)
    a, b = case.a.to(cuda_device), case.b.to(cuda_device)
    for atomic in (False, True):
        c = gg.persistent_grouped_gemm(a, b, offs, kernel_tile=(128, 128), use_atomic_queue=atomic)
        assert_parity(c, a, b, offs, case.k)


def sampled_parity(c, case, offs, stride=16):
    """Full-size check: every `stride`-th row against the oracle (fp64)."""
    rows = np.arange(0, case.m, stride)
    a32 = case.a.float().cpu().numpy()
    b32 = case.b.float().cpu().numpy()
    o = offs.cpu().numpy().astype(np.int64)
    expert = np.searchsorted(o, rows, side="right") - 1
    got = c.float().cpu().numpy()[rows]
    err = 0.0
    for e in np.unique(expert):
        sel = expert == e
        ref = a32[rows[sel]].astype(np.float64) @ b32[e].astype(np.float64)
        err = max(err, float(np.abs(got[sel] - ref).max()))
    assert err <= tol(case.k), f"max abs err {err} > {tol(case.k)}"
    return err


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", ["uniform", "skewed"])
def test_full_size_configs(cuda_device, name, dtype):
    case = workloads.make_case(name, device="cpu", dtype=dtype)
    log(f"full-size {name} {dtype}: M={case.m}")
    offs = gg.expert_offsets_from_recv_counts(case.counts, device=cuda_device)
    case_gpu_a, case_gpu_b = case.a.to(cuda_device), case.b.to(cuda_device)
    ref32 = None
    outs = []
    for blocks in [(256, 256), (128, 128)]:
        for atomic in (False, True):
            log(f"  blocks={blocks} atomic={atomic}")
            c = gg.persistent_grouped_gemm(case_gpu_a, case_gpu_b, offs, kernel_tile=blocks,
                                           use_atomic_queue=atomic)
            torch.cuda.synchronize()
            sampled_parity(c, case, offs)
            outs.append(c)
    # Whole output against a float32 per-expert torch loop on the device.
    ref32 = gg.reference_grouped_gemm(case_gpu_a.float(), case_gpu_b.float(), offs)
    for c in outs:
        err = (c.float() - ref32).abs().max().item()
        assert err <= tol(case.k), err
    # Striped launches take whole tiles: the same sums whatever the tile shape.
    assert torch.equal(outs[0], outs[2])
    if name == "uniform":  # 512 tiles, two full rounds: nothing is split
        assert torch.equal(outs[0], outs[1]) and torch.equal(outs[2], outs[3])


def test_empty_queue_zero_fills_and_keeps_counter(cuda_device):
    a, b, offs = make_inputs([0, 0, 0], 64, 64, torch.bfloat16, cuda_device, extra_rows=5)
    counter = torch.full((1,), 77, dtype=torch.int32, device=cuda_device)
    for queue in ("device", "prebuilt"):
        c = gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=True, work_counter=counter,
                                       queue=queue)
        torch.cuda.synchronize()
        assert c.shape == (5, 64) and bool((c == 0).all())
        assert counter.item() == 77  # untouched, as when the reference returns early
    # No experts at all.
    c = gg.persistent_grouped_gemm(a, b[:0], offs[:1])
    assert bool((c == 0).all())


@pytest.mark.parametrize("num_sms", [1, 7, 64, 256, 1000])
def test_work_counter_final_value(cuda_device, num_sms):
    counts = [300, 0, 129, 511]
    a, b, offs = make_inputs(counts, 128, 256, torch.bfloat16, cuda_device)
    counter = torch.zeros(1, dtype=torch.int32, device=cuda_device)
    w = orc.queue_length(offs.cpu().numpy(), 256, 128, 128)
    for rep in range(3):  # the library counter must be back at zero between calls
        c = gg.persistent_grouped_gemm(a, b, offs, num_sms=num_sms, block_m=128, block_n=128,
                                       use_atomic_queue=True, work_counter=counter)
        torch.cuda.synchronize()
        assert counter.item() == w + num_sms, (rep, counter.item())
        assert_parity(c, a, b, offs, 128)


def test_striped_with_few_workers(cuda_device):
    a, b, offs = make_inputs([100, 250, 3], 96, 320, torch.float16, cuda_device)
    for g in (1, 3, 9):
        c = gg.persistent_grouped_gemm(a, b, offs, num_sms=g, use_atomic_queue=False)
        assert_parity(c, a, b, offs, 96)


@pytest.mark.parametrize("num_experts", [2048, 2500])
def test_many_experts(cuda_device, num_experts):
    """2048 experts is the largest count whose queue the kernel derives in
    LDS; beyond it the drop-in builds the queue on the host (the reference's
    path) without being asked."""
    rng = np.random.default_rng(num_experts)
    counts = rng.integers(0, 40, num_experts).tolist()
    counts[7] = 300  # one expert spans two 256-row tiles
    a, b, offs = make_inputs(counts, 64, 64, torch.bfloat16, cuda_device, seed=3)
    for blocks in [(64, 64), (256, 256)]:
        for atomic in (False, True):
            log(f"E={num_experts} blocks={blocks} atomic={atomic}")
            c = gg.persistent_grouped_gemm(a, b, offs, kernel_tile=blocks,
                                           use_atomic_queue=atomic)
            torch.cuda.synchronize()
            assert_parity(c, a, b, offs, 64)


def test_odd_shapes_are_padded(cuda_device):
    a, b, offs = make_inputs([17, 0, 40], 50, 37, torch.bfloat16, cuda_device)
    c = gg.persistent_grouped_gemm(a, b, offs)
    assert c.shape == (57, 37) and c.is_contiguous()
    assert_parity(c, a, b, offs, 50)


K_TAILS = [1, 3, 7, 13, 50, 257, 1001, 2044]


@pytest.mark.parametrize("k", K_TAILS)
@pytest.mark.parametrize("tile", [(256, 256), (128, 128), (64, 64)])
def test_k_tail_reads_b_in_place(cuda_device, k, tile):
    """K not a multiple of 8: A is zero-padded, B (N-major, allocated exactly
    [E, K, N], the last expert non-empty) is read as it lies with its rows
    stopped at K.  Bitwise equal to the fully zero-padded problem, for both
    schedules (the atomic one splitting its last round where K allows)."""
    log(f"k tail k={k} tile={tile}")
    a, b, offs = make_inputs([70, 0, 300, 1, 260], k, 264, torch.bfloat16, cuda_device, seed=k)
    kp = (k + 7) // 8 * 8
    a_pad = torch.nn.functional.pad(a, (0, kp - k))
    b_pad = torch.nn.functional.pad(b, (0, 0, 0, kp - k))
    for atomic in (False, True):
        c = gg.persistent_grouped_gemm(a, b, offs, kernel_tile=tile, use_atomic_queue=atomic)
        c_pad = gg.persistent_grouped_gemm(a_pad, b_pad, offs, kernel_tile=tile,
                                           use_atomic_queue=atomic)
        torch.cuda.synchronize()
        assert torch.equal(c, c_pad), atomic
    # Against the fp64 oracle: one bf16 rounding of the output (relative
    # 2^-8; with K = 1 the outputs are products of two N(0, 1) values, so an
    # absolute bound alone would not fit) plus the fp32 accumulation's share.
    rows = covered_rows(offs)
    want = oracle_out(a, b, offs)[rows]
    got = c.float().cpu().numpy()[rows]
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-3 * math.sqrt(k))


def test_strided_operands(cuda_device):
    a_wide, b, offs = make_inputs([33, 70], 128, 64, torch.bfloat16, cuda_device)
    big = torch.randn(103, 256, device=cuda_device).to(torch.bfloat16)
    big[:, 64:192] = a_wide
    a_view = big[:, 64:192]  # row stride 256, 16-byte aligned
    assert a_view.stride() == (256, 1)
    bt = b.transpose(1, 2).contiguous().transpose(1, 2)  # N not contiguous -> copied
    c = gg.persistent_grouped_gemm(a_view, bt, offs)
    assert_parity(c, a_wide, b, offs, 128)


def test_rows_outside_experts_are_not_written(cuda_device):
    """Calls the C ABI directly with a sentinel-filled C."""
    a, b, offs = make_inputs([5, 0, 9], 64, 128, torch.bfloat16, cuda_device, extra_rows=0)
    m = 20
    a_full = torch.zeros(m, 64, dtype=torch.bfloat16, device=cuda_device)
    a_full[2:16] = a
    offs_shift = (offs + 2).to(torch.int32)  # rows [2, 16) covered, others not
    c = torch.full((m, 128), 123.0, dtype=torch.bfloat16, device=cuda_device)
    for atomic in (0, 1):
        nat.check(nat.lib().mgg_grouped_gemm(
            nat.MGG_DTYPE_BF16, a_full.data_ptr(), b.data_ptr(), c.data_ptr(), offs_shift.data_ptr(),
            m, 64, 128, 3, 64, 64 * 128, 128, 128, None, None, None, -1, 64, 64, 5, atomic, None,
            0, 0, torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert bool((c[:2] == 123).all()) and bool((c[16:] == 123).all())
        want = oracle_out(a, b, offs)
        assert float(np.abs(c[2:16].float().cpu().numpy() - want).max()) <= tol(64)


def test_caller_queue_with_invalid_items(cuda_device):
    """A caller-built queue may hold items that cover no rows: a tile_m past the
    expert's rows or a tile_n past N (the reference's masks make those no-ops,
    tgg:83-84), an empty expert, or an expert index outside [0, E).  The kernel
    skips them; the result equals the clean queue's, bitwise, in both
    schedules, and the atomic count is still (queue length) + G."""
    counts = [300, 0, 129]
    k, n, bm, bn = 128, 256, 128, 128
    a, b, offs = make_inputs(counts, k, n, torch.bfloat16, cuda_device)
    we, wm, wn = orc.build_work_queue(offs.cpu().numpy(), n, bm, bn)
    bad = [(0, 3, 0), (2, 1, 2), (1, 0, 0), (-1, 0, 0), (3, 0, 1), (0, 0, 5)]
    rng = np.random.default_rng(4)
    items = [tuple(t) for t in zip(we.tolist(), wm.tolist(), wn.tolist())] + bad
    order = rng.permutation(len(items))
    q = np.array([items[i] for i in order], dtype=np.int32)
    qe, qm, qn = (torch.from_numpy(np.ascontiguousarray(q[:, j])).to(cuda_device) for j in range(3))
    m = a.shape[0]
    ref = None
    for atomic in (0, 1):
        c = torch.zeros(m, n, dtype=torch.bfloat16, device=cuda_device)
        counter = torch.full((1,), 5, dtype=torch.int32, device=cuda_device)
        nat.check(nat.lib().mgg_grouped_gemm(
            nat.MGG_DTYPE_BF16, a.data_ptr(), b.data_ptr(), c.data_ptr(), offs.data_ptr(),
            m, k, n, len(counts), k, k * n, n, n, qe.data_ptr(), qm.data_ptr(), qn.data_ptr(),
            len(q), bm, bn, 7, atomic, counter.data_ptr() if atomic else None,
            0, 0, torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert_parity(c, a, b, offs, k)
        if atomic:
            assert counter.item() == len(q) + 7
        if ref is None:
            ref = c
        else:
            assert torch.equal(c, ref)


def test_device_queue_builder_bit_exact(cuda_device):
    data = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "queues.npz",
                   allow_pickle=False)
    tags = sorted({k.rsplit("__", 1)[0] for k in data.files if not k.endswith("__offsets")})
    for tag in tags:
        name, n_part, tile = tag.split("__")
        bm, bn = map(int, tile.split("x"))
        offs = torch.from_numpy(data[f"{name}__offsets"]).to(cuda_device)
        gg._WORK_QUEUE_CACHE.clear()
        q = gg._build_work_queue(offs, int(n_part[1:]), bm, bn)
        for arr, suffix in zip(q, ("expert", "tile_m", "tile_n")):
            np.testing.assert_array_equal(arr.cpu().numpy(), data[f"{tag}__{suffix}"], err_msg=tag)


def test_device_offsets_bit_exact(cuda_device):
    rng = np.random.default_rng(5)
    for size in (0, 1, 16, 1000, 5000):
        for src_dtype in (torch.int32, torch.int64):
            counts = rng.integers(0, 3000, size)
            t = torch.from_numpy(counts).to(src_dtype).to(cuda_device)
            for out_dtype in (torch.int32, torch.int64):
                got = gg.expert_offsets_from_recv_counts(t, dtype=out_dtype)
                want = orc.expert_offsets_from_recv_counts(counts, dtype=np.int32 if out_dtype == torch.int32 else np.int64)
                np.testing.assert_array_equal(got.cpu().numpy(), want)
    wrap = torch.tensor([2**31 - 1, 1, 2**32 + 3], dtype=torch.int64, device=cuda_device)
    assert gg.expert_offsets_from_recv_counts(wrap).tolist() == [0, 2**31 - 1, -(2**31), -(2**31) + 3]


KMAJOR_CASES = [
    # counts, K, N, extra K columns of the [E, N, K] storage (N-row stride K + pad)
    ([3, 0, 5], 64, 64, 0),
    ([130, 1, 257], 72, 64, 8),
    ([0, 0, 513, 0], 256, 136, 0),
    ([600], 520, 520, 24),
    ([300, 0, 257, 1, 512], 2056, 264, 0),
]
ALL_BLOCKS = [(256, 256), (128, 128), (256, 128), (128, 256), (64, 64), (64, 128), (128, 64),
              (256, 64), (64, 256), (128, 512)]


def kmajor_copy(b, pad):
    """The values of b [E, K, N] stored [E, N, K + pad] (K contiguous), as an [E, K, N] view."""
    e, k, n = b.shape
    store = torch.zeros(e, n, k + pad, dtype=b.dtype, device=b.device)
    store[:, :, :k] = b.transpose(1, 2)
    return store[:, :, :k].transpose(1, 2)


@pytest.mark.parametrize("case", range(len(KMAJOR_CASES)))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_kmajor_b_is_read_in_place_bitwise(cuda_device, case, dtype):
    """B as a [E, K, N] view of [E, N, K] memory (a linear layer's weight
    transposed, which the reference's Triton kernel reads through its strides)
    takes the K-major kernels, with no copy, and gives bitwise the result of
    the same values stored [E, K, N] on every tile and schedule."""
    counts, k, n, pad = KMAJOR_CASES[case]
    a, b, offs = make_inputs(counts, k, n, dtype, cuda_device, seed=100 + case, extra_rows=2)
    b_km = kmajor_copy(b, pad)
    assert b_km.stride(1) == 1 and b_km.stride(2) == k + pad and gg._kmajor_layout(b_km)
    mask = torch.from_numpy(covered_rows(offs)).to(cuda_device)
    for blocks in ALL_BLOCKS:
        for atomic in (False, True):
            log(f"kmajor case={case} dtype={dtype} blocks={blocks} atomic={atomic}")
            c_n = gg.persistent_grouped_gemm(a, b, offs, kernel_tile=blocks,
                                             use_atomic_queue=atomic)
            c_k = gg.persistent_grouped_gemm(a, b_km, offs, kernel_tile=blocks,
                                             use_atomic_queue=atomic)
            torch.cuda.synchronize()
            assert torch.equal(c_k[: mask.numel()][mask], c_n[: mask.numel()][mask]), (blocks, atomic)
        assert_parity(c_k, a, b, offs, k)


@pytest.mark.parametrize("epilogue", ["gelu", "swiglu"])
@pytest.mark.parametrize("block", [256, 128])
def test_kmajor_b_fused_epilogues_bitwise(cuda_device, epilogue, block):
    import expert_mlp as mlp
    counts, k, n = [300, 0, 257, 1, 200], 136, 256
    a, b, offs = make_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=7, extra_rows=1)
    b_km = kmajor_copy(b, 16)
    out = n // 2 if epilogue == "swiglu" else n
    epi = mlp._EPILOGUES[epilogue]
    c_n = mlp._grouped_gemm_ex(a, b, offs, epi, out, None, block, True)
    c_k = mlp._grouped_gemm_ex(a, b_km, offs, epi, out, None, block, True)
    torch.cuda.synchronize()
    mask = torch.from_numpy(covered_rows(offs)).to(cuda_device)
    assert torch.equal(c_k[: mask.numel()][mask], c_n[: mask.numel()][mask])


# The 128x512 tile (the default when experts hold at most 128 rows on
# average): N edges inside and past a 512-wide tile, K tails inside a 32-deep
# stage, ragged and empty experts, experts above 128 rows (two m-tiles).
WIDE_CASES = [([128] * 6 + [0, 37], 264, 1000),
              ([5, 300, 0, 128, 129], 136, 520),
              ([64] * 12, 2048, 2048),
              ([1, 2, 3], 40, 512)]


@pytest.mark.parametrize("case", range(len(WIDE_CASES)))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_wide_tile_matches_square_tile(cuda_device, case, dtype):
    """128x512 against the oracle, and bitwise against the 256x256 tile on
    striped launches (each output's K sum runs in the same order)."""
    counts, k, n = WIDE_CASES[case]
    a, b, offs = make_inputs(counts, k, n, dtype, cuda_device, seed=300 + case, extra_rows=1)
    mask = torch.from_numpy(covered_rows(offs)).to(cuda_device)
    square = gg.persistent_grouped_gemm(a, b, offs, kernel_tile=(256, 256), use_atomic_queue=False)
    for atomic in (False, True):
        log(f"wide case={case} dtype={dtype} atomic={atomic}")
        c = gg.persistent_grouped_gemm(a, b, offs, kernel_tile=(128, 512), use_atomic_queue=atomic)
        torch.cuda.synchronize()
        assert_parity(c, a, b, offs, k)
        if not atomic:
            assert torch.equal(c[: mask.numel()][mask], square[: mask.numel()][mask])

