"""CPU oracle for the expert-grouped GEMM path -- TEST INFRASTRUCTURE ONLY.

A restatement, in numpy, of the reference's algorithm for this path
(Hongyu15/moe-overlap, ``src/triton_grouped_gemm.py``), used as the checker in
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py``.  Nothing in the product (``moe-overlap_amd/``) imports it.

Functions and what pins each one (tests/test_oracle_*.py):

* ``expert_offsets_from_recv_counts`` -- reference :300-323.  Pinned by the
  closed form [0, cumsum], hand-computed cases, the wrap of int32 sums and
  the committed fixtures.
* ``build_work_queue`` -- reference :240-297 (vectorised like the reference:
  repeat + local position).  Pinned by a brute-force triple loop on random
  inputs, by the coverage invariant (every expert row x column is covered by
  exactly one tile), by the queue lengths of the benchmark configurations, and
  by hand-enumerated cases.
* ``grouped_gemm`` -- reference :446-457 (per-expert loop), computed in fp32 or
  fp64.  Pinned by a brute-force scalar triple loop on tiny inputs, one-hot
  rows (which select rows of B[e] and expose transposed operands or wrong
  experts), expert-scaled identities, E=1 reducing to a plain matmul, and
  integer-valued inputs with exact expected outputs.
* ``queue_coverage`` -- the coverage invariant itself (a counting check).
* ``fp8_e4m3_to_f32`` / ``grouped_gemm_fp8`` -- the fp8 extension (the
  reference rejects fp8 at :357-358): OCP e4m3 decoded from its definition
  (sign, 4-bit exponent with bias 7, 3-bit mantissa, subnormals, 0x7F/0xFF
  NaN, no infinities), then the per-expert product scaled per row of A and
  per (expert, column).  Pinned by torch's own float8_e4m3fn conversion on
  all 256 codes, by closed-form codes (1.0, 448, the smallest subnormal), and
  by reduction to ``grouped_gemm`` on the decoded values.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "expert_offsets_from_recv_counts",
    "build_work_queue",
    "queue_length",
    "grouped_gemm",
    "queue_coverage",
    "bf16_bits_to_f32",
    "f32_to_bf16_bits",
    "fp8_e4m3_to_f32",
    "grouped_gemm_fp8",
]


def expert_offsets_from_recv_counts(counts, dtype=np.int32) -> np.ndarray:
    """[0, c0, c0+c1, ...] of length E+1 (reference :315-323).

    Each count is narrowed to int32 (``.to(torch.int32)``), the prefix sum is
    taken in int64 (torch's integer cumsum) and the result cast to ``dtype``
    (an int32 result wraps modulo 2**32).
    """
    c = np.asarray(counts)
    if c.dtype.kind == "f":
        c = np.trunc(c)
    c32 = c.astype(np.int64).astype(np.int32).reshape(-1)
    cum = np.cumsum(c32.astype(np.int64), dtype=np.int64)
    out = np.concatenate([np.zeros(1, np.int64), cum])
    return out.astype(dtype)


def queue_length(offsets, n_size: int, block_m: int, block_n: int) -> int:
    off = np.asarray(offsets, dtype=np.int64)
    if off.size <= 1:
        return 0
    counts = np.clip(off[1:] - off[:-1], 0, None)
    tiles_m = (counts + block_m - 1) // block_m
    tiles_n = (int(n_size) + block_n - 1) // block_n
    return int(tiles_m.sum()) * tiles_n


def build_work_queue(offsets, n_size: int, block_m: int, block_n: int):
    """(expert, tile_m, tile_n) int32 arrays (reference :253-292).

    Per expert: count = max(off[e+1]-off[e], 0), ceil(count/block_m) m-tiles
    times ceil(n_size/block_n) n-tiles, listed expert-major, then tile_m, then
    tile_n (fastest).
    """
    off = np.asarray(offsets, dtype=np.int64)
    num_experts = max(off.size - 1, 0)
    counts = np.clip(off[1:] - off[:-1], 0, None) if num_experts else np.zeros(0, np.int64)
    tiles_m = (counts + block_m - 1) // block_m
    tiles_n = (int(n_size) + block_n - 1) // block_n
    per_expert = tiles_m * tiles_n
    total = int(per_expert.sum())
    if total == 0:
        z = np.zeros(0, np.int32)
        return z, z.copy(), z.copy()
    expert = np.repeat(np.arange(num_experts, dtype=np.int64), per_expert)
    first = np.cumsum(per_expert) - per_expert
    local = np.arange(total, dtype=np.int64) - first[expert]
    return (
        expert.astype(np.int32),
        (local // tiles_n).astype(np.int32),
        (local % tiles_n).astype(np.int32),
    )


def queue_coverage(offsets, m_size: int, n_size: int, block_m: int, block_n: int, queue):
    """How many tiles of `queue` write each element of C [m_size, n_size].

    A tile (e, tm, tn) writes rows off[e] + tm*block_m + [0, block_m) that lie
    below off[e+1], and columns tn*block_n + [0, block_n) below n_size (the
    store mask of reference :96-98).
    """
    off = np.asarray(offsets, dtype=np.int64)
    cover = np.zeros((m_size, n_size), np.int32)
    for e, tm, tn in zip(*queue):
        r0 = off[e] + int(tm) * block_m
        r1 = min(r0 + block_m, off[e + 1])
        c0 = int(tn) * block_n
        c1 = min(c0 + block_n, n_size)
        if r1 > r0 and c1 > c0:
            cover[r0:r1, c0:c1] += 1
    return cover


def grouped_gemm(a, b, offsets, acc_dtype=np.float32, out=None) -> np.ndarray:
    """out[s:t] = a[s:t] @ b[e] for each expert with t > s (reference :449-456).

    ``a`` [M, K] and ``b`` [E, K, N] are real arrays (bf16 inputs arrive
    already widened to float32, exactly).  The product is computed in
    ``acc_dtype``.  Rows outside every expert range keep the value of ``out``
    (NaN when ``out`` is None), the counterpart of the reference's
    uninitialised ``torch.empty`` rows.
    """
    a = np.asarray(a)
    b = np.asarray(b)
    off = np.asarray(offsets, dtype=np.int64)
    if out is None:
        out = np.full((a.shape[0], b.shape[2]), np.nan, dtype=acc_dtype)
    for e in range(b.shape[0]):
        s, t = int(off[e]), int(off[e + 1])
        if t <= s:
            continue
        out[s:t] = a[s:t].astype(acc_dtype) @ b[e].astype(acc_dtype)
    return out


def bf16_bits_to_f32(bits) -> np.ndarray:
    """Widen raw bf16 bit patterns (uint16) to float32 (exact)."""
    u = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return u.view(np.float32)


def f32_to_bf16_bits(x) -> np.ndarray:
    """Round float32 to bf16 bit patterns, nearest-even (NaN stays NaN)."""
    x = np.asarray(x, dtype=np.float32)
    u = x.reshape(-1).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = rounded.astype(np.uint16)
    out[np.isnan(x.reshape(-1))] = 0x7FC0
    return out.reshape(x.shape)


def fp8_e4m3_to_f32(bits) -> np.ndarray:
    """OCP e4m3 (float8_e4m3fn) bytes -> float32: (-1)^s * 2^(e-7) * (1 + m/8),
    subnormals 2^-6 * m/8 for e == 0, NaN for exponent and mantissa all ones."""
    b = np.asarray(bits, dtype=np.uint8).astype(np.int64)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 0x7
    val = np.where(e == 0, np.ldexp(m / 8.0, -6), np.ldexp(1.0 + m / 8.0, e - 7))
    val = np.where((e == 0xF) & (m == 0x7), np.nan, val)
    return (sign * val).astype(np.float32)


def grouped_gemm_fp8(a_bits, b_bits_nk, offsets, a_scale, b_scale, acc_dtype=np.float64,
                     magnitude: bool = False) -> np.ndarray:
    """C[r, n] = a_scale[r] * b_scale[e, n] * sum_k A[r, k] * B[e, n, k] over
    each expert's row range (rows outside every range are zero here).
    a_bits [M, K] and b_bits_nk [E, N, K] are e4m3 bytes.  With magnitude=True
    the same with |A| and |B| (the scale of the sum's rounding errors)."""
    a = fp8_e4m3_to_f32(a_bits).astype(acc_dtype)
    b = fp8_e4m3_to_f32(b_bits_nk).astype(acc_dtype)
    if magnitude:
        a, b = np.abs(a), np.abs(b)
    offs = np.asarray(offsets, dtype=np.int64)
    sa = np.asarray(a_scale, dtype=acc_dtype).reshape(-1)
    sb = np.asarray(b_scale, dtype=acc_dtype).reshape(b.shape[0], b.shape[1])
    out = np.zeros((a.shape[0], b.shape[1]), dtype=acc_dtype)
    for e in range(b.shape[0]):
        s, t = int(offs[e]), int(offs[e + 1])
        if t > s:
            out[s:t] = (a[s:t] @ b[e].T) * sa[s:t, None] * sb[e][None, :]
    return out
