"""The drop-in module's host-side behaviour (no GPU): the reference's
ValueError conditions, CPU-tensor paths of the two integer builders (which run
in libmgg's host code) against the oracle, and the FIFO queue cache."""
import numpy as np
import pytest
import torch

import grouped_gemm as gg
import triton_grouped_gemm as tgg
from oracle import grouped_gemm_oracle as orc


def test_alias_module_exports_reference_names():
    for name in ("persistent_grouped_gemm", "expert_offsets_from_recv_counts",
                 "reference_grouped_gemm", "_build_work_queue"):
        assert getattr(tgg, name) is getattr(gg, name)


def test_gemm_requires_gpu_tensors():
    a = torch.zeros(4, 8, dtype=torch.bfloat16)
    b = torch.zeros(1, 8, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="requires CUDA tensors"):
        gg.persistent_grouped_gemm(a, b, torch.tensor([0, 4], dtype=torch.int32))


@pytest.mark.parametrize("counts", [[], [0], [5], [3, 0, 5], [128] * 8, list(range(40))])
@pytest.mark.parametrize("as_tensor", [False, True])
def test_offsets_cpu_match_oracle(counts, as_tensor):
    src = torch.tensor(counts, dtype=torch.int64) if as_tensor else counts
    got = gg.expert_offsets_from_recv_counts(src)
    assert got.dtype == torch.int32 and got.device.type == "cpu"
    np.testing.assert_array_equal(got.numpy(), orc.expert_offsets_from_recv_counts(counts))


def test_offsets_cpu_dtypes_and_shapes():
    t = torch.tensor([[1, 2], [3, 4]], dtype=torch.int16)
    assert gg.expert_offsets_from_recv_counts(t).tolist() == [0, 1, 3, 6, 10]
    f = torch.tensor([1.9, 2.2])  # float counts truncate, as .to(int32) does
    assert gg.expert_offsets_from_recv_counts(f).tolist() == [0, 1, 3]
    big = torch.tensor([2**31 - 1, 1], dtype=torch.int64)
    assert gg.expert_offsets_from_recv_counts(big).tolist() == [0, 2**31 - 1, -(2**31)]
    out64 = gg.expert_offsets_from_recv_counts(big, dtype=torch.int64)
    assert out64.dtype == torch.int64 and out64.tolist() == [0, 2**31 - 1, 2**31]
    assert gg.expert_offsets_from_recv_counts([1, 2], dtype=torch.float32).tolist() == [0.0, 1.0, 3.0]


@pytest.mark.parametrize("counts,n,bm,bn", [
    ([3, 0, 5], 5, 2, 2), ([128] * 8, 1024, 128, 128), ([0, 0, 586, 3269, 7, 4331], 4096, 256, 256),
    ([], 64, 64, 64), ([0, 0], 64, 64, 64), ([9], 0, 4, 4),
])
def test_queue_cpu_match_oracle(counts, n, bm, bn):
    offs = torch.tensor(np.concatenate([[0], np.cumsum(counts)]).astype(np.int64))
    got = gg._build_work_queue(offs, n, bm, bn)
    for g, w in zip(got, orc.build_work_queue(offs.numpy(), n, bm, bn)):
        assert g.dtype == torch.int32
        np.testing.assert_array_equal(g.numpy(), w)


def test_queue_cache_hits_and_fifo_eviction():
    gg._WORK_QUEUE_CACHE.clear()
    off = torch.tensor([0, 7, 7, 20], dtype=torch.int32)
    q1 = gg._build_work_queue(off, 64, 4, 32)
    q2 = gg._build_work_queue(off.to(torch.int64), 64, 4, 32)  # same key bytes (int64 view)
    assert all(x is y for x, y in zip(q1, q2))
    first_key = next(iter(gg._WORK_QUEUE_CACHE))
    for i in range(gg._WORK_QUEUE_CACHE_MAX):
        gg._build_work_queue(torch.tensor([0, i + 1]), 64, 4, 32)
    assert len(gg._WORK_QUEUE_CACHE) == gg._WORK_QUEUE_CACHE_MAX
    assert first_key not in gg._WORK_QUEUE_CACHE


def test_flops_helper():
    assert gg.grouped_gemm_flops(torch.tensor([0, 512, 1024]), 2048, 4096) == 2 * 1024 * 2048 * 4096
    assert gg.grouped_gemm_flops([0, 5, 3], 8, 8) == 2 * 5 * 64  # negative counts add nothing


@pytest.mark.parametrize("avg,want", [(1, (128, 128)), (100, (128, 128)), (128, (128, 128)),
                                      (129, (256, 128)), (192, (256, 128)), (256, (256, 128)),
                                      (257, (256, 256)), (384, (256, 256)), (4096, (256, 256))])
def test_default_fp8_tile(avg, want):
    """128x128 up to 128 rows per expert, 256x128 for 129-256, else 256x256;
    the fp8 benchmark config (64 experts, 24576 rows: 384 per expert) takes 256x256."""
    assert gg._default_fp8_kernel_tile(avg * 64, 64) == want
    assert gg._default_fp8_kernel_tile(0, 0) == (128, 128)


@pytest.mark.parametrize("edge", [16, 32, 64, 128, 256, 512, 1024, 1 << 20])
def test_requested_tile_accepts_triton_tiles(edge):
    """Every power of two >= 16 (what tl.arange and tl.dot accept,
    src/triton_grouped_gemm.py:54-56, :67-69) is a valid requested tile."""
    assert gg._requested_tile(edge, 16) == (edge, 16)
    assert gg._requested_tile(np.int64(edge), edge) == (edge, edge)


@pytest.mark.parametrize("bad", [0, -128, 1, 8, 24, 48, 96, 100, 2 ** 21, 128.0, "128", None])
def test_requested_tile_rejects_others(bad):
    with pytest.raises(ValueError):
        gg._requested_tile(bad, 128)
    with pytest.raises(ValueError):
        gg._requested_tile(128, bad)


def test_large_expert_queue_builds_on_host():
    """Above the device builder's 8192 experts the queue is built by the host
    builder (CPU offsets here take that path always); checked against the oracle."""
    rng = np.random.default_rng(3)
    counts = rng.integers(0, 300, 9000)
    offs = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)]).astype(np.int64))
    got = gg._build_work_queue(offs, 300, 128, 256)
    for g, w in zip(got, orc.build_work_queue(offs.numpy(), 300, 128, 256)):
        np.testing.assert_array_equal(g.numpy(), w)


def test_default_tile_follows_expert_size():
    """The drop-in computes with 128x512 when experts hold at most 128 rows on
    average, N is at least 512, and the wide tiles fill enough rounds of the
    workers (1.6 x its rounds under the square tile's), else with 256x256."""
    assert gg._default_kernel_tile(256 * 128, 256, 2048) == (128, 512)   # 4 rounds against 8
    assert gg._default_kernel_tile(128 * 32, 128, 4096) == (128, 512)    # 4 against 8
    assert gg._default_kernel_tile(16 * 128, 16, 4096) == (256, 256)     # 1 against 1
    assert gg._default_kernel_tile(64 * 128, 64, 1024) == (256, 256)     # 1 against 1
    assert gg._default_kernel_tile(16 * 512, 16, 4096) == (256, 256)     # 512 rows
    assert gg._default_kernel_tile(256 * 128, 256, 256) == (256, 256)    # N < 512
    assert gg._default_kernel_tile(0, 0, 4096) == (256, 256)
    assert gg._default_kernel_tile(256 * 128, 256, 2048, workers=1024) == (128, 512)  # 1 against 2
    assert gg._default_kernel_tile(256 * 128, 256, 2048, workers=2048) == (256, 256)  # 1 against 1


def test_odd_n_tiles():
    """Odd N computes on the tiles its kernel instances are compiled for."""
    for t in ((256, 256), (128, 128)):
        assert gg._odd_n_tile(t, True) == t and gg._odd_n_tile(t, False) == t
    assert gg._odd_n_tile((128, 512), True) == (128, 512)
    assert gg._odd_n_tile((128, 512), False) == (256, 256)
    assert gg._odd_n_tile((256, 128), True) == (256, 256)
    assert gg._odd_n_tile((64, 256), True) == (256, 256)
    assert gg._odd_n_tile((192, 128), False) == (128, 128)
    for t in ((64, 64), (128, 64), (64, 128)):
        assert gg._odd_n_tile(t, True) == (128, 128)
