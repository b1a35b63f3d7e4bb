"""GPU tests of the drop-in's queue semantics beyond plain parity: the tile a
caller requests (block_m/block_n) against the tile the kernel computes with,
the atomic schedule's counter word (dirty words, concurrent streams, graph
capture), K == 0 and the prebuilt-queue fallbacks above 2048 experts.

Reference behaviour pinned here (src/triton_grouped_gemm.py):
* :240-297  the queue is counted for the requested block_m x block_n;
* :379-386  the counter starts every launch at zero (the caller's
            work_counter is zeroed) and ends at W + G (:201-233: each worker
            over-fetches once);
* :369-371  an empty queue zero-fills and leaves the counter untouched.
Tolerance as in test_gpu_gemm: max |C - C_fp64| <= 2e-2 * sqrt(max(K, 512) / 512).
"""
import ctypes
import gc
import math
import sys
import time

import numpy as np
import pytest
import torch

import expert_mlp as mlp
import grouped_gemm as gg
import mgg_native as nat
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


def covered(offs):
    o = offs.cpu().numpy().astype(np.int64)
    mask = np.zeros(int(max(o.max(initial=0), 0)), bool)
    for e in range(len(o) - 1):
        if o[e + 1] > o[e]:
            mask[o[e]:o[e + 1]] = True
    return mask


def assert_parity(c, a, b, offs, k):
    want = orc.grouped_gemm(a.float().cpu().numpy(), b.float().cpu().numpy(),
                            offs.cpu().numpy(), acc_dtype=np.float64)
    mask = covered(offs)
    got = c.float().cpu().numpy()[: mask.size][mask]
    err = float(np.abs(got - want[: mask.size][mask]).max()) if got.size else 0.0
    assert np.isfinite(got).all() and err <= tol(k), err


def queue_len(offs, n, bm, bn):
    return orc.queue_length(offs.cpu().numpy().astype(np.int64), n, bm, bn)


# Requested tiles the reference's Triton kernel compiles (powers of two >= 16),
# including its default 128 x 128 and tiles no kernel here is compiled for.
REQUESTED = [(16, 64), (32, 32), (512, 128), (128, 128), (64, 1024), (256, 256)]


@pytest.mark.parametrize("tile", REQUESTED)
@pytest.mark.parametrize("queue", ["device", "prebuilt"])
def test_requested_tile_sets_counter_not_result(cuda_device, tile, queue):
    """Any requested tile computes on the library's tile: identical bits to
    the default, parity with the oracle, and work_counter = W(requested) + G."""
    counts, k, n = [300, 0, 129, 1, 517], 136, 264
    a, b, offs = make_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=11, extra_rows=2)
    base = gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=False)
    mask = torch.from_numpy(covered(offs)).to(cuda_device)
    for g_workers in (7, 256):
        counter = torch.full((1,), -3, dtype=torch.int32, device=cuda_device)
        log(f"requested tile={tile} queue={queue} G={g_workers}")
        c = gg.persistent_grouped_gemm(a, b, offs, num_sms=g_workers, block_m=tile[0],
                                       block_n=tile[1], use_atomic_queue=True,
                                       work_counter=counter, queue=queue)
        torch.cuda.synchronize()
        assert counter.item() == queue_len(offs, n, *tile) + g_workers
        assert torch.equal(c[: mask.numel()][mask], base[: mask.numel()][mask])
    assert_parity(base, a, b, offs, k)


def test_requested_tile_validation(cuda_device):
    a, b, offs = make_inputs([4], 64, 64, torch.bfloat16, cuda_device)
    for bad in (0, 8, 48, 96, 100):
        with pytest.raises(ValueError, match="power of two"):
            gg.persistent_grouped_gemm(a, b, offs, block_m=bad)
    with pytest.raises(ValueError, match="kernel_tile"):
        gg.persistent_grouped_gemm(a, b, offs, kernel_tile=(32, 32))


@pytest.mark.parametrize("poison", [12345, (7 << 32) | 3, 0xFFFFFFFFFFFFFFFF, (0xDEADBEEF << 32) | 0x7FFFFFFF])
def test_dirty_counter_word_is_reclaimed(cuda_device, poison):
    """A counter word left at any value (as a launch that did not finish could
    leave it) does not drop or repeat tiles: the next atomic launch computes
    every tile and reports W + G, and so does the launch after it."""
    counts, k, n = [513, 0, 200, 1, 64, 700], 128, 320
    a, b, offs = make_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=5)
    w = queue_len(offs, n, 256, 256)
    stream = torch.cuda.current_stream().cuda_stream
    for g_workers in (3, 256):
        for rep in range(2):
            nat.check(nat.lib().mgg_debug_set_dequeue_counter(poison, stream))
            counter = torch.zeros(1, dtype=torch.int32, device=cuda_device)
            c = torch.full((a.shape[0], n), float("nan"), dtype=torch.bfloat16, device=cuda_device)
            log(f"poison={poison:#x} G={g_workers} rep={rep}")
            out = gg.persistent_grouped_gemm(a, b, offs, num_sms=g_workers, block_m=256,
                                             block_n=256, work_counter=counter)
            c.copy_(out)
            torch.cuda.synchronize()
            assert counter.item() == w + g_workers
            assert_parity(c, a, b, offs, k)
            # A clean launch right after (the dirty one left the word tagged for it).
            counter.zero_()
            c2 = gg.persistent_grouped_gemm(a, b, offs, num_sms=g_workers, block_m=256,
                                            block_n=256, work_counter=counter)
            torch.cuda.synchronize()
            assert counter.item() == w + g_workers
            assert torch.equal(c2, out)


@pytest.mark.parametrize("counts,tiles", [([512, 256, 0, 768], 12), ([300, 0, 257, 1, 600], 16)])
@pytest.mark.parametrize("g_workers", [2, 3, 4, 5])
@pytest.mark.parametrize("poison", [None, (9 << 32) | 5])
def test_atomic_static_rounds(cuda_device, counts, tiles, g_workers, poison):
    """With the device-derived queue and at least two rounds of tiles the
    atomic schedule runs every whole round in the striped placement and
    draws tickets only for the tail past them.  12 tiles (whole 256-row
    m-tiles) on 2, 3 and 4 workers (6, 4 and 3 static rounds: one ticket per
    worker past the queue) and on 5 (two static rounds, then 2 tiles by
    ticket); 16 tiles with partial m-tiles on 2, 4 (8 and 4 rounds), 3 and 5
    (5 and 3 rounds, then one tile by ticket): every tile once (oracle
    parity), the counter ends at W + G, also after a dirty counter word, and
    the results are bitwise the striped schedule's (K = 128 is too short to
    split a tile: each part needs 1024 of K)."""
    k, n = 128, 512
    a, b, offs = make_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=11)
    w = queue_len(offs, n, 256, 256)
    assert w == tiles
    stream = torch.cuda.current_stream().cuda_stream
    striped = gg.persistent_grouped_gemm(a, b, offs, num_sms=g_workers, block_m=256, block_n=256,
                                         kernel_tile=(256, 256), use_atomic_queue=False)
    for rep in range(2):
        if poison is not None:
            nat.check(nat.lib().mgg_debug_set_dequeue_counter(poison, stream))
        counter = torch.zeros(1, dtype=torch.int32, device=cuda_device)
        log(f"static rounds W={tiles} G={g_workers} poison={poison} rep={rep}")
        c = gg.persistent_grouped_gemm(a, b, offs, num_sms=g_workers, block_m=256, block_n=256,
                                       kernel_tile=(256, 256), work_counter=counter)
        torch.cuda.synchronize()
        assert counter.item() == w + g_workers
        assert_parity(c, a, b, offs, k)
        assert torch.equal(c, striped)


def test_atomic_launches_on_two_streams_at_once(cuda_device):
    """Atomic launches on two created streams run concurrently on separate
    counter words and split-tile workspaces (12 tiles on 128 and 192
    workers, each split in halves of K = 2056); every result matches the
    serial one bitwise."""
    cases = [make_inputs([300, 5, 0, 600], 2056, 512, torch.bfloat16, cuda_device, seed=s)
             for s in (1, 2)]
    refs = [gg.persistent_grouped_gemm(a, b, o, num_sms=128 + 64 * i, use_atomic_queue=True)
            for i, (a, b, o) in enumerate(cases)]
    streams = [torch.cuda.Stream(device=cuda_device) for _ in cases]
    torch.cuda.synchronize()
    outs = [[], []]
    for it in range(8):
        for i, ((a, b, o), st) in enumerate(zip(cases, streams)):
            with torch.cuda.stream(st):
                outs[i].append(gg.persistent_grouped_gemm(a, b, o, num_sms=128 + 64 * i,
                                                          use_atomic_queue=True))
    torch.cuda.synchronize()
    for i in range(2):
        for got in outs[i]:
            assert torch.equal(got, refs[i])
    assert_parity(refs[0], *cases[0], 2056)


def test_graph_capture_and_replay(cuda_device):
    """The atomic call captured into a HIP graph (torch.cuda.graph) replays
    correctly again and again, with eager atomic launches on the capture
    stream's neighbour and host synchronisations between the replays."""
    a, b, offs = make_inputs([300, 0, 257, 40], 192, 256, torch.bfloat16, cuda_device, seed=9)
    counter = torch.zeros(1, dtype=torch.int32, device=cuda_device)
    eager = gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=False)
    w = queue_len(offs, 256, 128, 128)
    side = torch.cuda.Stream(device=cuda_device)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=True, work_counter=counter)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=True,
                                              work_counter=counter)
    g_workers = gg._cu_count(cuda_device.index or 0)
    for rep in range(4):
        counter.zero_()
        torch.cuda.synchronize()
        log(f"graph replay {rep}")
        graph.replay()
        # Eager atomic work between replays, on the default stream.
        other = gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=True)
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), rep
        assert torch.equal(other, eager), rep
        assert counter.item() == w + g_workers, rep


def test_k_zero_gives_zeros_and_counts(cuda_device):
    """K == 0: every covered row is zero and the counter ends at W + G (the
    reference's kernel runs its tiles with an empty K loop)."""
    counts, n = [5, 0, 300], 96
    a = torch.empty(305, 0, dtype=torch.bfloat16, device=cuda_device)
    b = torch.empty(3, 0, n, dtype=torch.bfloat16, device=cuda_device)
    offs = torch.tensor(orc.expert_offsets_from_recv_counts(counts), dtype=torch.int32,
                        device=cuda_device)
    for atomic in (False, True):
        counter = torch.zeros(1, dtype=torch.int32, device=cuda_device)
        c = gg.persistent_grouped_gemm(a, b, offs, num_sms=9, use_atomic_queue=atomic,
                                       work_counter=counter)
        torch.cuda.synchronize()
        assert c.shape == (305, n) and bool((c == 0).all())
        assert counter.item() == (queue_len(offs, n, 128, 128) + 9 if atomic else 0)


def test_fp8_and_fused_entry_points_above_2048_experts(cuda_device):
    """Above the device-derived queue's 2048 experts the fp8 and fused-epilogue
    entry points run on a prebuilt queue (no expert limit, as the reference)."""
    num_experts = 2300
    rng = np.random.default_rng(2300)
    counts = rng.integers(0, 12, num_experts).tolist()
    counts[5] = 300
    k, n = 64, 128
    a, b, offs = make_inputs(counts, k, n, torch.bfloat16, cuda_device, seed=4)
    c = mlp._grouped_gemm_ex(a, b, offs, nat.MGG_EPI_GELU, n, None, 128, True)
    torch.cuda.synchronize()
    ref = torch.nn.functional.gelu(gg.reference_grouped_gemm(a.float(), b.float(), offs))
    mask = torch.from_numpy(covered(offs)).to(cuda_device)
    err = (c.float()[mask] - ref[mask]).abs().max().item()
    assert err <= 2 * tol(k), err
    # fp8: e4m3 operands with unit scales, against the decoded product.
    a8 = (a.float().clamp(-8, 8)).to(torch.float8_e4m3fn)
    b8 = (b.float() * 8).to(torch.float8_e4m3fn)
    sa = torch.ones(a.shape[0], device=cuda_device)
    sb = torch.full((num_experts, n), 1.0 / 8, device=cuda_device)
    counter = torch.zeros(1, dtype=torch.int32, device=cuda_device)
    c8 = gg.persistent_grouped_gemm(a8, b8.transpose(1, 2).contiguous().transpose(1, 2), offs,
                                    num_sms=64, work_counter=counter, a_scale=sa, b_scale=sb)
    torch.cuda.synchronize()
    ref8 = gg.reference_grouped_gemm(a8.float(), b8.float() / 8, offs)
    rel = ((c8.float()[mask] - ref8[mask]).norm() / ref8[mask].norm()).item()
    assert rel <= 1e-2, rel
    assert counter.item() == queue_len(offs, n, 128, 128) + 64


def _held_slots(device):
    n = ctypes.c_int(0)
    nat.check(nat.lib().mgg_debug_counter_slots(device.index or 0, ctypes.byref(n)))
    return n.value


def test_captured_launches_share_and_release_counter_words(cuda_device):
    """Atomic launches captured on one stream in one capture share one counter
    word (40 captures of two launches hold 40 words), every replay is right,
    and destroying the graphs frees their words, so captures never use up the
    device's 4096."""
    a, b, offs = make_inputs([300, 0, 257, 40], 192, 256, torch.bfloat16, cuda_device, seed=9)
    eager = gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=False)
    torch.cuda.synchronize()
    base = _held_slots(cuda_device)
    graphs, outs = [], []
    for _ in range(40):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            o1 = gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=True)
            o2 = gg.persistent_grouped_gemm(a, b, offs, use_atomic_queue=True)
        graphs.append(graph)
        outs.append((o1, o2))
    held = _held_slots(cuda_device)
    log(f"counter words held: {base} before, {held} with 40 graphs")
    assert held == base + 40
    for rep in range(2):
        for graph in graphs:
            graph.replay()
        torch.cuda.synchronize()
        for o1, o2 in outs:
            assert torch.equal(o1, eager) and torch.equal(o2, eager), rep
    del graphs, graph, outs, o1, o2
    gc.collect()
    torch.cuda.synchronize()
    deadline = time.time() + 5
    while _held_slots(cuda_device) != base and time.time() < deadline:
        time.sleep(0.05)
    assert _held_slots(cuda_device) == base
