"""Pins the CPU oracle (oracle/grouped_gemm_oracle.py) against checks that do
not restate its formulas: brute-force enumeration, hand-computed cases,
invariants, exact integer arithmetic and the committed fixtures."""
import json
from pathlib import Path

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from oracle import grouped_gemm_oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- offsets
def test_offsets_hand_cases():
    assert orc.expert_offsets_from_recv_counts([]).tolist() == [0]
    assert orc.expert_offsets_from_recv_counts([0, 0, 0]).tolist() == [0, 0, 0, 0]
    assert orc.expert_offsets_from_recv_counts([3, 0, 5]).tolist() == [0, 3, 3, 8]
    assert orc.expert_offsets_from_recv_counts([128] * 8).tolist() == list(range(0, 1025, 128))
    out = orc.expert_offsets_from_recv_counts(np.array([[1, 2], [3, 4]], dtype=np.int64))
    assert out.tolist() == [0, 1, 3, 6, 10] and out.dtype == np.int32


def test_offsets_int32_wrap_and_narrowing():
    big = 2**31 - 1
    # int32 result wraps modulo 2**32, int64 keeps the exact sum
    assert orc.expert_offsets_from_recv_counts([big, 1]).tolist() == [0, big, -(2**31)]
    assert orc.expert_offsets_from_recv_counts([big, 1], dtype=np.int64).tolist() == [0, big, 2**31]
    # each count is narrowed to int32 before the sum (2**32 + 5 -> 5)
    assert orc.expert_offsets_from_recv_counts(np.array([2**32 + 5], np.int64)).tolist() == [0, 5]


@given(st.lists(st.integers(0, 10_000), max_size=70))
def test_offsets_match_running_sum(counts):
    out = orc.expert_offsets_from_recv_counts(counts)
    run = 0
    assert out[0] == 0
    for i, c in enumerate(counts):
        run += c
        assert out[i + 1] == run


# ---------------------------------------------------------------- queue
def brute_queue(offsets, n_size, bm, bn):
    items = []
    tiles_n = -(-n_size // bn)
    for e in range(len(offsets) - 1):
        cnt = max(offsets[e + 1] - offsets[e], 0)
        tm = 0
        while tm * bm < cnt:
            for tn in range(tiles_n):
                items.append((e, tm, tn))
            tm += 1
    return items


def test_queue_hand_case():
    # counts [3, 0, 5], N=5, 2x2 tiles: expert 0 -> 2 m-tiles, expert 2 -> 3 m-tiles, 3 n-tiles
    we, wm, wn = orc.build_work_queue([0, 3, 3, 8], 5, 2, 2)
    assert we.tolist() == [0] * 6 + [2] * 9
    assert wm.tolist() == [0, 0, 0, 1, 1, 1, 0, 0, 0, 1, 1, 1, 2, 2, 2]
    assert wn.tolist() == [0, 1, 2] * 5
    assert we.dtype == wm.dtype == wn.dtype == np.int32


def test_queue_empty_and_negative_counts():
    for offs in ([0], [0, 0, 0], [5, 3, 3]):  # no experts, all empty, a negative count
        q = orc.build_work_queue(offs, 64, 16, 16)
        assert all(x.size == 0 and x.dtype == np.int32 for x in q)
    assert orc.build_work_queue([0, 4], 0, 2, 2)[0].size == 0  # N = 0


@settings(max_examples=150, deadline=None)
@given(
    st.lists(st.integers(-3, 40), max_size=9),
    st.integers(0, 70),
    st.sampled_from([1, 2, 3, 8, 16, 64]),
    st.sampled_from([1, 4, 8, 32, 128]),
)
def test_queue_matches_brute_force(counts, n_size, bm, bn):
    offs = [0]
    for c in counts:
        offs.append(offs[-1] + c)
    we, wm, wn = orc.build_work_queue(offs, n_size, bm, bn)
    assert list(zip(we.tolist(), wm.tolist(), wn.tolist())) == brute_queue(offs, n_size, bm, bn)
    assert orc.queue_length(offs, n_size, bm, bn) == we.size


@settings(max_examples=60, deadline=None)
@given(st.lists(st.integers(0, 40), min_size=1, max_size=6), st.integers(1, 50),
       st.sampled_from([4, 8, 16]), st.sampled_from([4, 8, 32]))
def test_queue_covers_each_expert_element_exactly_once(counts, n_size, bm, bn):
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    m = int(offs[-1]) + 3  # rows past the last expert stay uncovered
    cover = orc.queue_coverage(offs, m, n_size, bm, bn, orc.build_work_queue(offs, n_size, bm, bn))
    assert (cover[: offs[-1]] == 1).all()
    assert (cover[offs[-1]:] == 0).all()


def test_queue_lengths_of_baseline_configs():
    # Queue lengths quoted for the benchmark configs (computed independently there).
    counts = json.loads((GOLDEN / "routing_counts.json").read_text())
    offs = {k: orc.expert_offsets_from_recv_counts(v) for k, v in counts.items()}
    assert orc.queue_length(offs["cpu_plumbing"], 1024, 128, 128) == 64
    assert orc.queue_length(offs["uniform"], 4096, 128, 128) == 2048
    assert orc.queue_length(offs["uniform"], 4096, 256, 256) == 512
    assert orc.queue_length(offs["skewed"], 4096, 128, 128) == 4160
    assert orc.queue_length(offs["skewed"], 4096, 256, 256) == 1056
    assert orc.queue_length(offs["expert_mlp"], 8192, 128, 128) == 8768
    assert orc.queue_length(offs["fp8_fine"], 1408, 128, 128) == 2486


def test_skewed_counts_pinned():
    counts = json.loads((GOLDEN / "routing_counts.json").read_text())
    assert counts["skewed"] == [0, 0, 586, 3269, 7, 4331, 0, 0, 0, 0, 0, 0, 0, 8191, 0, 0]
    assert sum(counts["skewed"]) == 16384
    assert sum(counts["fp8_fine"]) == 24576 and min(counts["fp8_fine"]) == 344


def test_queue_fixtures():
    data = np.load(GOLDEN / "queues.npz", allow_pickle=False)
    tags = sorted({k.rsplit("__", 1)[0] for k in data.files if not k.endswith("__offsets")})
    assert len(tags) >= 25
    for tag in tags:
        name, n_part, tile = tag.split("__")
        bm, bn = map(int, tile.split("x"))
        offs = data[f"{name}__offsets"]
        q = orc.build_work_queue(offs, int(n_part[1:]), bm, bn)
        for arr, suffix in zip(q, ("expert", "tile_m", "tile_n")):
            np.testing.assert_array_equal(arr, data[f"{tag}__{suffix}"], err_msg=tag)


# ---------------------------------------------------------------- GEMM
def brute_gemm(a, b, offs):
    m, k = a.shape
    n = b.shape[2]
    out = np.full((m, n), np.nan)
    for e in range(b.shape[0]):
        for i in range(offs[e], offs[e + 1]):
            for j in range(n):
                out[i, j] = sum(float(a[i, kk]) * float(b[e, kk, j]) for kk in range(k))
    return out


def test_gemm_matches_scalar_loop():
    rng = np.random.default_rng(0)
    offs = [0, 3, 3, 7, 8]
    a = rng.standard_normal((9, 5)).astype(np.float32)
    b = rng.standard_normal((4, 5, 6)).astype(np.float32)
    got = orc.grouped_gemm(a, b, offs, acc_dtype=np.float64)
    want = brute_gemm(a, b, offs)
    np.testing.assert_allclose(got[:8], want[:8], rtol=1e-12, atol=1e-12)
    assert np.isnan(got[8]).all()  # row outside every expert range untouched


def test_gemm_integer_golden_exact():
    for case in json.loads((GOLDEN / "tiny_gemm.json").read_text()):
        a = np.array(case["a"], np.float32)
        b = np.array(case["b"], np.float32).reshape(len(case["offsets"]) - 1, a.shape[1], -1)
        got = orc.grouped_gemm(a, b, case["offsets"])
        for i, row in enumerate(case["c"]):
            if row[0] is None:
                assert np.isnan(got[i]).all()
            else:
                assert got[i].tolist() == row


def test_gemm_one_hot_rows_select_rows_of_the_right_expert():
    # Row i of expert e is one-hot at k = i % K, so C row i must equal B[e][i % K].
    rng = np.random.default_rng(1)
    offs = [0, 4, 4, 10]
    k, n = 6, 7
    a = np.zeros((10, k), np.float32)
    for i in range(10):
        a[i, i % k] = 1.0
    b = rng.standard_normal((3, k, n)).astype(np.float32)
    got = orc.grouped_gemm(a, b, offs)
    for e in range(3):
        for i in range(offs[e], offs[e + 1]):
            np.testing.assert_array_equal(got[i], b[e, i % k])


def test_gemm_expert_scaled_identity():
    # B[e] = (e+1) * I: C rows of expert e are (e+1) * A rows.
    rng = np.random.default_rng(2)
    offs = [0, 2, 5, 5, 9]
    a = rng.standard_normal((9, 8)).astype(np.float32)
    b = np.stack([(e + 1) * np.eye(8, dtype=np.float32) for e in range(4)])
    got = orc.grouped_gemm(a, b, offs)
    for e in range(4):
        np.testing.assert_array_equal(got[offs[e]:offs[e + 1]], (e + 1) * a[offs[e]:offs[e + 1]])


def test_gemm_single_expert_is_plain_matmul():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((17, 9))
    b = rng.standard_normal((1, 9, 4))
    np.testing.assert_allclose(orc.grouped_gemm(a, b, [0, 17], acc_dtype=np.float64), a @ b[0],
                               rtol=1e-13)


def test_bf16_round_trip_and_rounding():
    x = np.array([1.0, -2.5, 3.14159, 1e-3, 65504.0, np.inf, -np.inf], np.float32)
    bits = orc.f32_to_bf16_bits(x)
    back = orc.bf16_bits_to_f32(bits)
    assert back[0] == 1.0 and back[1] == -2.5 and np.isinf(back[5]) and np.isinf(back[6])
    assert abs(back[2] - 3.140625) < 1e-7  # 3.14159 -> nearest bf16 3.140625
    # ties go to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7
    assert orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(np.float32(1 + 2**-8)))[()] == 1.0
    assert np.isnan(orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(np.float32(np.nan))))


def test_bf16_matches_torch_rounding():
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(4).standard_normal(10_000).astype(np.float32) * 100
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(orc.f32_to_bf16_bits(x), want)


def test_fp8_decode_matches_torch_on_every_code():
    import torch

    codes = np.arange(256, dtype=np.uint8)
    ours = orc.fp8_e4m3_to_f32(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert nan.sum() == 2  # 0x7F and 0xFF
    np.testing.assert_array_equal(ours[~nan], ref[~nan])


def test_fp8_decode_closed_forms():
    assert orc.fp8_e4m3_to_f32([0x38])[0] == 1.0
    assert orc.fp8_e4m3_to_f32([0x7E])[0] == 448.0  # largest finite
    assert orc.fp8_e4m3_to_f32([0x01])[0] == 2.0 ** -9  # smallest subnormal
    assert orc.fp8_e4m3_to_f32([0xC0])[0] == -2.0
    assert orc.fp8_e4m3_to_f32([0x80])[0] == 0.0 and np.signbit(orc.fp8_e4m3_to_f32([0x80])[0])


def test_fp8_grouped_gemm_reduces_to_dequantized_grouped_gemm():
    rng = np.random.default_rng(11)
    counts = [3, 0, 5, 2]
    offs = orc.expert_offsets_from_recv_counts(counts)
    M, K, N, E = int(offs[-1]) + 1, 32, 6, len(counts)
    a = rng.integers(0, 256, size=(M, K), dtype=np.uint8)
    b = rng.integers(0, 256, size=(E, N, K), dtype=np.uint8)
    a[(a & 0x7F) == 0x7F] = 0x38  # no NaN codes
    b[(b & 0x7F) == 0x7F] = 0x38
    sa = rng.random(M) + 0.5
    sb = rng.random((E, N)) + 0.5
    got = orc.grouped_gemm_fp8(a, b, offs, sa, sb)
    deq_b = np.transpose(orc.fp8_e4m3_to_f32(b).astype(np.float64), (0, 2, 1)) * sb[:, None, :]
    deq_a = orc.fp8_e4m3_to_f32(a).astype(np.float64) * sa[:, None]
    ref = orc.grouped_gemm(deq_a, deq_b, offs, acc_dtype=np.float64)
    rows = int(offs[-1])
    np.testing.assert_allclose(got[:rows], ref[:rows], rtol=1e-12, atol=1e-9)
