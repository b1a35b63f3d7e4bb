"""Expert-grouped GEMM for MoE on MI355X (gfx950): the host side of the drop-in.

Module-level API of the reference's ``src/triton_grouped_gemm.py``, same names,
arguments, results and ``ValueError`` conditions, computed by hand-written HIP
kernels in libmgg.so (``include/mgg.h``) instead of Triton:

* ``persistent_grouped_gemm``          (reference :326-443)
* ``expert_offsets_from_recv_counts``  (reference :300-323)
* ``_build_work_queue``                (reference :240-297, with its FIFO cache)
* ``reference_grouped_gemm``           (reference :446-457, the per-expert loop)

Differences, all in arguments that do not change results:

* ``num_sms`` defaults to the device's CU count (256 on MI355X) instead of 24;
  an explicit value is honoured (it doubles as a CU-reservation knob).
* ``block_m``/``block_n`` (default 128 x 128, as there) are the tile the
  caller asks for: any power of two >= 16, the tiles the reference's Triton
  kernel compiles.  They set the queue whose length the atomic schedule's
  ``work_counter`` reports (W + G, W counted for the requested tile) and the
  keys of ``_build_work_queue``; the kernel itself computes with the fastest
  compiled tile, 256 x 256 for bf16/fp16 (eight waves, two per SIMD, 32-deep
  B stages and 64-deep A blocks), or the tile named by the keyword-only
  ``kernel_tile``.  Every output element is the same fp32 sum in the same K
  order whatever the tile, so results do not depend on either choice.
* ``block_k``, ``num_warps``, ``num_stages`` are accepted and ignored: the
  kernel's K staging, wave count and LDS ring are fixed by its design.
* ``queue="device"`` (default) derives the same (expert, tile_m, tile_n)
  tiles inside the kernel from the offsets (an expert's m-tiles grouped by
  four, each group taken n-tile by n-tile, for L2 reuse), so a call never
  waits on the device; ``queue="prebuilt"`` goes through
  ``_build_work_queue`` (a host round trip for the cache key, as in the
  reference) and runs its row order.  Each tile's sums are the same either
  way (the split last round below aside).  Above
  2048 experts (the device-derived queue keeps its tile prefix in LDS) the
  prebuilt path is taken without being asked.
* ``work_counter`` (atomic mode) receives the final count W + G, the value
  the reference leaves there, while the dequeue itself runs on a
  library-owned per-stream counter word, so no separate zeroing launch is
  needed.
* The atomic schedule with the device-derived queue takes a last round of
  at most a quarter (a half) as many tiles as workers as 4 (2) parts of K per
  tile, their fp32 sums added pairwise in a fixed tree: the output can differ
  in the last bits from the striped schedule's (both within the tolerance of
  the fp32 product; each repeats itself bitwise).  Graph-captured launches
  and prebuilt queues take whole tiles, and ``set_split_last_round(False)``
  turns the split off (every schedule then gives bitwise the same output).
  The parts meet in a per-stream workspace of 64 MiB (one 256 x 256 fp32
  slot per CU) that the stream's first atomic call allocates, unless
  ``reserve_split_workspace`` made it beforehand.
* Operands whose inner stride is not 1 are copied on the device first, and
  so is A when its row stride is not a multiple of 8 elements.  K not a multiple of 8: A is copied with
  zero columns to the next multiple of 8 and B is read in place (the kernel
  stops B's rows at K; a K-major B view is copied).  Any N is read and
  written in place (B's and C's rows need not be 16-byte aligned).  K == 0
  gives zeros, as there.
"""
from __future__ import annotations

import ctypes
import operator
from typing import List, Optional, Tuple, Union

import numpy as np
import torch

import mgg_native as _nat

__all__ = [
    "persistent_grouped_gemm",
    "expert_offsets_from_recv_counts",
    "reference_grouped_gemm",
    "_build_work_queue",
    "grouped_gemm_flops",
    "quantize_fp8_rows",
    "set_split_last_round",
    "reserve_split_workspace",
    "split_workspace_bytes",
]

# Tiles compiled into libmgg for bf16/fp16 (fused epilogues: 256x256, 128x128).
_KERNEL_TILES = ((256, 256), (128, 128), (256, 128), (128, 256), (128, 64), (64, 128),
                 (64, 64), (256, 64), (64, 256), (128, 512))
_DTYPE_CODES = {torch.bfloat16: _nat.MGG_DTYPE_BF16, torch.float16: _nat.MGG_DTYPE_FP16}

_WORK_QUEUE_CACHE: dict = {}
_WORK_QUEUE_CACHE_MAX = 32


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_CU_COUNTS: dict = {}


def _cu_count(dev_index: int) -> int:
    n = _CU_COUNTS.get(dev_index)
    if n is None:
        n = _CU_COUNTS[dev_index] = _nat.device_cu_count(dev_index)
    return n


def set_split_last_round(enabled: bool) -> None:
    """Turns the atomic schedule's split last round on (the default) or off,
    process-wide.  Off, every tile is summed whole, so an atomic call gives
    bitwise the striped (and graph-captured) call's output."""
    _nat.check(_nat.lib().mgg_set_split_last_round(1 if enabled else 0))


def reserve_split_workspace(device: Optional[torch.device] = None) -> None:
    """Makes the split-round workspace of the current stream of `device` now
    (64 MiB on MI355X, never freed), so that no later atomic call on that
    stream allocates device memory."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    dev_index = dev.index if dev.index is not None else torch.cuda.current_device()
    with torch.cuda.device(dev_index):
        _nat.check(_nat.lib().mgg_reserve_split_workspace(_stream_handle(dev)))


def split_workspace_bytes(device: Optional[torch.device] = None) -> int:
    """Bytes of split-round workspace held for the current stream of `device`."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    dev_index = dev.index if dev.index is not None else torch.cuda.current_device()
    n = ctypes.c_int64(0)
    with torch.cuda.device(dev_index):
        _nat.check(_nat.lib().mgg_split_workspace_bytes(_stream_handle(dev), ctypes.byref(n)))
    return int(n.value)


# --------------------------------------------------------------------------
# expert offsets
# --------------------------------------------------------------------------
def expert_offsets_from_recv_counts(
    num_recv_tokens_per_expert: Union[torch.Tensor, List[int]],
    device: Optional[torch.device] = None,
    dtype: torch.dtype = torch.int32,
) -> torch.Tensor:
    """``[0, c_0, c_0 + c_1, ...]`` of length E+1 from per-expert counts.

    Reference: src/triton_grouped_gemm.py:300-323.  A list becomes an int32
    tensor; a tensor is narrowed to int32 and flattened; ``device`` moves it;
    the prefix sum is taken in int64 and cast to ``dtype`` (so int32 sums wrap).
    The scan runs in libmgg (device kernel for GPU tensors, host loop for CPU
    tensors).
    """
    if isinstance(num_recv_tokens_per_expert, list):
        t = torch.tensor(num_recv_tokens_per_expert, dtype=torch.int32)
    else:
        t = num_recv_tokens_per_expert.flatten()
        if t.dtype not in (torch.int32, torch.int64):
            t = t.to(torch.int32)
    if device is not None:
        t = t.to(device)
    t = t.contiguous()
    num = t.numel()
    out_dtype = dtype if dtype in (torch.int32, torch.int64) else torch.int64
    out = torch.empty(num + 1, dtype=out_dtype, device=t.device)
    in_code = _nat.MGG_INT32 if t.dtype == torch.int32 else _nat.MGG_INT64
    out_code = _nat.MGG_INT32 if out_dtype == torch.int32 else _nat.MGG_INT64
    lib = _nat.lib()
    if t.device.type == "cuda":
        with torch.cuda.device(t.device):
            _nat.check(
                lib.mgg_expert_offsets_from_counts(
                    _ptr(t), in_code, num, _ptr(out), out_code, _stream_handle(t.device)
                )
            )
    elif t.device.type == "cpu":
        _nat.check(lib.mgg_expert_offsets_from_counts_host(_ptr(t), in_code, num, _ptr(out), out_code))
    else:
        raise ValueError(f"unsupported device {t.device}")
    return out if out_dtype == dtype else out.to(dtype)


# --------------------------------------------------------------------------
# work queue
# --------------------------------------------------------------------------
def _queue_length(offsets_host: np.ndarray, n_size: int, block_m: int, block_n: int) -> int:
    counts = np.clip(offsets_host[1:] - offsets_host[:-1], 0, None)
    tiles_m = (counts + block_m - 1) // block_m
    tiles_n = (int(n_size) + block_n - 1) // block_n
    return int(tiles_m.sum()) * tiles_n


def _build_work_queue(
    expert_offsets: torch.Tensor,
    n_size: int,
    block_m: int,
    block_n: int,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(expert_id, tile_m, tile_n) int32 vectors, expert-major then tile_m then tile_n.

    Reference: src/triton_grouped_gemm.py:240-297.  Cached by (offsets bytes,
    n_size, block_m, block_n) with FIFO eviction at 32 entries; the offsets
    are copied to the host for the key (a device sync, as in the reference).
    Built by libmgg on the offsets' device (on the host, then copied, above
    the device builder's 8192 experts).
    """
    assert expert_offsets.dim() == 1
    if block_m <= 0 or block_n <= 0:
        raise ValueError("block_m and block_n must be positive.")
    device = expert_offsets.device
    host = expert_offsets.detach().to("cpu", torch.int64).contiguous().numpy()
    key = (host.tobytes(), int(n_size), int(block_m), int(block_n))
    cached = _WORK_QUEUE_CACHE.get(key)
    if cached is not None and cached[0].device == device:
        return cached

    num_experts = host.shape[0] - 1
    total = _queue_length(host, n_size, block_m, block_n) if num_experts > 0 else 0
    we = torch.empty(total, dtype=torch.int32, device=device)
    wm = torch.empty(total, dtype=torch.int32, device=device)
    wn = torch.empty(total, dtype=torch.int32, device=device)
    lib = _nat.lib()
    if total > 0:
        if device.type == "cuda" and num_experts > _nat.MAX_DEVICE_BUILDER_EXPERTS:
            host_q = [torch.empty(total, dtype=torch.int32) for _ in range(3)]
            _nat.check(
                lib.mgg_build_work_queue_host(
                    host.ctypes.data_as(ctypes.c_void_p), num_experts, int(n_size),
                    int(block_m), int(block_n), *(_ptr(q) for q in host_q), total,
                )
            )
            for dst, src in zip((we, wm, wn), host_q):
                dst.copy_(src)
        elif device.type == "cuda":
            off32 = expert_offsets.to(torch.int32).contiguous()
            with torch.cuda.device(device):
                _nat.check(
                    lib.mgg_build_work_queue(
                        _ptr(off32), num_experts, int(n_size), int(block_m), int(block_n),
                        _ptr(we), _ptr(wm), _ptr(wn), total, _stream_handle(device),
                    )
                )
        else:
            _nat.check(
                lib.mgg_build_work_queue_host(
                    host.ctypes.data_as(ctypes.c_void_p), num_experts, int(n_size),
                    int(block_m), int(block_n), _ptr(we), _ptr(wm), _ptr(wn), total,
                )
            )
    result = (we, wm, wn)
    if len(_WORK_QUEUE_CACHE) >= _WORK_QUEUE_CACHE_MAX:
        _WORK_QUEUE_CACHE.pop(next(iter(_WORK_QUEUE_CACHE)))
    _WORK_QUEUE_CACHE[key] = result
    return result


# --------------------------------------------------------------------------
# grouped GEMM
# --------------------------------------------------------------------------
def _default_kernel_tile(m_total: int, num_experts: int, n_size: int = 4096,
                         workers: int = 256) -> Tuple[int, int]:
    """128x512 or 256x256, from the average rows per expert (no host sync on
    the offsets).  Rows of a tile past its expert's end are zero-fill DMAs that
    read nothing, so a tile's cost follows the memory requests of its valid
    rows; both tiles hold the same 256 KiB of fp32 accumulators (two waves per
    SIMD).  With at most 128 rows an expert is one m-tile either way and the
    wide tile reads its A rows half as often, but each of its tiles takes about
    1.6 times as long and there are half as many: it is taken when N >= 512 and
    1.6 x its rounds of `workers` tiles stay under the square tile's rounds.
    Measured on MI355X (HIP-event medians, atomic, µs): E=256 x 128 rows,
    K=7168, N=2048 (the reference benchmark's default problem) 1271 against
    1584 (256x256); E=128 x 32 rows, K=N=4096, 682 against 776; but E=16 x 128
    rows, K=2048, N=4096 (128 wide tiles for 256 workers) 74.9 against 57.4;
    E=64 x 128, N=1024, 80.6 against 60.9; E=16 x 192 and x 256 rows 74.7 and
    80.1 against 63.0 and 68.8.  Among the tiles of at most 256 rows and
    columns, 256x256 is the fastest at every expert size (E=16, K=2048,
    N=4096, atomic / striped: 64 rows per expert 57.2 / 52.3 against 128x256
    63.4 / 54.5 and 128x128 55.4 / 50.9; 128 rows 60.9 / 60.5 against 95.5 /
    94.6 (128x256); 192 rows 63.2 / 62.4 against 101.2 / 98.5; 256-384 rows
    101-119 against 140-192)."""
    if num_experts <= 0 or n_size < 512 or m_total > 128 * num_experts:
        return 256, 256
    rows = max(-(-m_total // num_experts), 1)
    w = max(int(workers), 1)
    rounds_wide = -(-(num_experts * -(-rows // 128) * -(-n_size // 512)) // w)
    rounds_square = -(-(num_experts * -(-rows // 256) * -(-n_size // 256)) // w)
    return (128, 512) if 1.6 * rounds_wide < rounds_square else (256, 256)


def _requested_tile(block_m, block_n) -> Tuple[int, int]:
    """The caller's block_m x block_n: powers of two >= 16, the tile edges the
    reference's Triton kernel compiles (tl.arange needs a power of two, tl.dot
    at least 16; src/triton_grouped_gemm.py:54-56, :67-69)."""
    out = []
    for name, v in (("block_m", block_m), ("block_n", block_n)):
        try:
            v = operator.index(v)
        except TypeError:
            raise ValueError(f"{name} must be an int.") from None
        if v < 16 or v & (v - 1) or v > 1 << 20:
            raise ValueError(f"{name} must be a power of two >= 16 (got {v}).")
        out.append(v)
    return out[0], out[1]


def _fast_layout(t: torch.Tensor, mult: int = 8) -> bool:
    """Unit inner stride, 16-byte aligned base, outer strides multiples of
    `mult` elements (8 for A; 1 for N-major B, whose rows the kernel reads at
    any 2-byte alignment)."""
    if t.stride(-1) != 1 or t.data_ptr() % 16 != 0:
        return False
    return all(t.stride(d) % mult == 0 for d in range(t.dim() - 1) if t.size(d) > 1)


def _kmajor_layout(b: torch.Tensor) -> bool:
    """b [E, K, N] is a view of [E, N, K] memory (K contiguous: a linear
    layer's [out, in] weight transposed) that the kernel reads in place: N-row
    and expert strides multiples of 8 elements, 16-byte aligned base."""
    _, k, n = b.shape
    if k < 2 or n < 2 or b.stride(1) != 1 or b.stride(2) < k:
        return False
    if b.data_ptr() % 16 != 0 or b.stride(2) % 8 != 0:
        return False
    return b.size(0) < 2 or b.stride(0) % 8 == 0


def _odd_n_tile(tile: Tuple[int, int], wide_ok: bool) -> Tuple[int, int]:
    """Odd N runs on kernel instances of its own, compiled for 256x256 and
    128x128 tiles (and 128x512 when `wide_ok`: N-major 16-bit B): another
    kernel tile computes on the nearest of these (the requested tile still
    sets the queue the work_counter counts)."""
    if tile in ((256, 256), (128, 128)) or (wide_ok and tile == (128, 512)):
        return tile
    return (256, 256) if max(tile) >= 256 else (128, 128)


def _gemm_operand(t: torch.Tensor, mult: int = 8) -> torch.Tensor:
    """`t` itself when the kernel can read it in place, else a device copy."""
    if _fast_layout(t, mult):
        return t
    t = t.contiguous()
    if not _fast_layout(t, mult):
        t = t.clone(memory_format=torch.contiguous_format)
    return t


def persistent_grouped_gemm(
    a_cat: torch.Tensor,
    b_expert: torch.Tensor,
    expert_offsets: torch.Tensor,
    num_sms: Optional[int] = None,
    block_m: int = 128,
    block_n: int = 128,
    block_k: int = 32,
    use_atomic_queue: bool = True,
    work_counter: Optional[torch.Tensor] = None,
    num_warps: int = 8,
    num_stages: int = 3,
    *,
    queue: str = "device",
    kernel_tile: Optional[Tuple[int, int]] = None,
    a_scale: Optional[torch.Tensor] = None,
    b_scale: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """C[s_e:t_e] = A[s_e:t_e] @ B[e] for every expert, persistent workers.

    Reference: src/triton_grouped_gemm.py:326-443.  a_cat [M, K], b_expert
    [E, K, N], expert_offsets [E+1]; bf16 or fp16; fp32 accumulation; output
    [M, N] in the input dtype (rows outside every expert range are left
    uninitialised; an empty queue zero-fills).  Launches asynchronously on the
    current stream of a_cat's device.  b_expert may be a [E, K, N] view of
    [E, N, K] memory (K contiguous, e.g. w.transpose(1, 2) of a linear
    layer's weight, which the reference's Triton kernel reads through its
    strides): it is read in place, with results bitwise equal to those of the
    same values stored [E, K, N]; other layouts are copied first.

    block_m x block_n is the requested tile (queue granularity and the
    work_counter's W + G); kernel_tile, when given, names the compiled tile
    the kernel computes with (default: the fastest, see _default_kernel_tile).

    Extension beyond the reference (which rejects fp8, :357-358): with
    float8_e4m3fn a_cat and b_expert plus a_scale [M] (per token) and b_scale
    [E, N] (per expert output channel), both fp32, the result is
    a_scale[r] * b_scale[e, n] * (A @ B[e])[r, n] in bf16.  B is read K-major:
    pass b_expert as a [E, K, N] view of [E, N, K] memory (stride(1) == 1,
    e.g. w.transpose(1, 2) of a linear layer's [E, N, K] weight) to avoid a copy.
    """
    if a_cat.device.type != "cuda" or b_expert.device.type != "cuda":
        raise ValueError("persistent_grouped_gemm requires CUDA tensors.")
    if a_cat.dim() != 2 or b_expert.dim() != 3:
        raise ValueError("Shapes must be a_cat [M, K], b_expert [E, K, N].")
    if a_cat.size(1) != b_expert.size(1):
        raise ValueError("K dimension mismatch between a_cat and b_expert.")
    if expert_offsets.numel() != b_expert.size(0) + 1:
        raise ValueError("expert_offsets must have shape [num_experts + 1].")
    if expert_offsets.device != a_cat.device:
        raise ValueError("expert_offsets must be on the same device as input tensors.")
    if queue not in ("device", "prebuilt"):
        raise ValueError("queue must be 'device' or 'prebuilt'.")
    rep_m, rep_n = _requested_tile(block_m, block_n)
    if a_cat.dtype == torch.float8_e4m3fn:
        return _persistent_grouped_gemm_fp8(a_cat, b_expert, expert_offsets, a_scale, b_scale,
                                            num_sms, rep_m, rep_n, kernel_tile, use_atomic_queue,
                                            work_counter, queue)
    if a_cat.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("a_cat dtype must be bf16/fp16.")
    if b_expert.dtype != a_cat.dtype:
        raise ValueError("b_expert dtype should match a_cat dtype.")
    if queue == "device" and b_expert.size(0) > _nat.MAX_DEVICE_QUEUE_EXPERTS:
        queue = "prebuilt"  # the device-derived queue keeps its tile prefix in LDS

    m_total, k_size = a_cat.shape
    num_experts, _, n_size = b_expert.shape
    device = a_cat.device
    dev_index = device.index if device.index is not None else torch.cuda.current_device()
    if num_sms is None:
        num_sms = _cu_count(dev_index)
    if int(num_sms) <= 0:
        raise ValueError("num_sms must be positive.")
    if kernel_tile is None:
        kernel_tile = _default_kernel_tile(m_total, num_experts, n_size, int(num_sms))
    kbm, kbn = (int(v) for v in kernel_tile)
    if (kbm, kbn) not in _KERNEL_TILES:
        raise ValueError(f"kernel_tile must be one of {_KERNEL_TILES}.")
    counter_dev = _counter_arg(work_counter, use_atomic_queue, device)

    # K not a multiple of 8: A is zero-padded on the device to the next
    # multiple of 8 and B is read as it lies (the kernel stops B's rows at K,
    # so the padding columns meet zeros).  Any N: B and C are used as they
    # lie (the kernel reads and writes rows at any 2-byte alignment).
    k_pad = (k_size + 7) // 8 * 8
    a_op, b_op = a_cat, b_expert
    # B stored [E, N, K] is read as it lies (no transposing copy).
    b_kmajor = k_pad == k_size and _kmajor_layout(b_expert)
    if n_size & 1:
        kbm, kbn = _odd_n_tile((kbm, kbn), not b_kmajor)
    if k_pad != k_size:
        a_op = torch.nn.functional.pad(a_op, (0, k_pad - k_size))
    if k_pad > 0:
        a_op = _gemm_operand(a_op)
        if not b_kmajor:
            b_op = _gemm_operand(b_op, 1)
    # Leading dimensions; a size-1 dimension's stride is never used, nor are
    # A's and B's when K == 0.  ldb_k is the stride between B's rows: K rows,
    # or N rows for K-major B.
    lda = a_op.stride(0) if m_total > 1 else k_pad
    if b_kmajor:
        ldb_k = b_op.stride(2)
        ldb_e = b_op.stride(0) if num_experts > 1 else n_size * ldb_k
    else:
        ldb_k = b_op.stride(1) if k_size > 1 else n_size
        ldb_e = b_op.stride(0) if num_experts > 1 else k_size * ldb_k
    dtype_code = _DTYPE_CODES[a_cat.dtype] | (_nat.MGG_B_KMAJOR if b_kmajor else 0)
    c_op = torch.empty((m_total, n_size), device=device, dtype=a_cat.dtype)

    we, wm, wn, num_work = _queue_args(queue, expert_offsets, n_size, kbm, kbn)
    off32 = _offsets_i32(expert_offsets)
    args = (
        dtype_code, _ptr(a_op), _ptr(b_op), _ptr(c_op),
        _ptr(off32), m_total, k_size, n_size,
        num_experts, lda, ldb_e, ldb_k, c_op.stride(0),
        _ptr(we), _ptr(wm), _ptr(wn), num_work,
        kbm, kbn, int(num_sms), 1 if use_atomic_queue else 0,
        _ptr(counter_dev), rep_m, rep_n, torch.cuda.current_stream(device).cuda_stream,
    )
    _launch(_nat.lib().mgg_grouped_gemm, args, dev_index)
    return c_op


def _counter_arg(work_counter, use_atomic_queue, device):
    """The device int32 [1] that receives W + G in atomic mode, or None.  As in
    the reference (:377-384), a counter on another device is copied there and
    the copy receives the count."""
    if not use_atomic_queue or work_counter is None:
        return None
    if work_counter.numel() != 1 or work_counter.dtype != torch.int32:
        raise ValueError("work_counter must be int32 tensor of shape [1].")
    counter_dev = work_counter.to(device)
    return counter_dev if counter_dev.is_contiguous() else counter_dev.contiguous()


def _offsets_i32(expert_offsets: torch.Tensor) -> torch.Tensor:
    off32 = expert_offsets if expert_offsets.dtype == torch.int32 else expert_offsets.to(torch.int32)
    return off32.contiguous()


def _queue_args(queue, expert_offsets, n_size, kbm, kbn):
    """(work_expert, work_tile_m, work_tile_n, num_work) for the kernel tile:
    the prebuilt queue of _build_work_queue, or no arrays and -1 (derived on
    the device)."""
    if queue == "prebuilt":
        we, wm, wn = _build_work_queue(expert_offsets, n_size=n_size, block_m=kbm, block_n=kbn)
        return we, wm, wn, we.numel()
    return None, None, None, -1


def _launch(fn, args, dev_index: int) -> None:
    """Calls a libmgg launch entry point with dev_index as the current HIP
    device (the library launches on the calling thread's current device)."""
    if torch.cuda.current_device() == dev_index:
        _nat.check(fn(*args))
    else:
        with torch.cuda.device(dev_index):
            _nat.check(fn(*args))


_FP8_KERNEL_TILES = ((256, 256), (256, 128), (192, 128), (128, 128))


def _default_fp8_kernel_tile(m_total: int, num_experts: int) -> Tuple[int, int]:
    """fp8 tile by the average rows per expert (top-k routing spreads the
    counts around it): 128x128 up to 128 rows, 256x128 for 129-256 (one tile
    holds most experts), 256x256 above.  Measured on MI355X at E=64, K=2048,
    N=1408, HIP-event medians (striped / atomic, µs): 96 rows 128x128
    43.2 / 45.6 against 256x256 58.6 / 57.4; 192 rows 256x128 55.4 / 60.4,
    256x256 59.5 / 59.0; 281 rows 256x256 81.9 / 86.9 against 192x128
    84.6 / 91.7; 384 rows 85.9 / 94.5 against 103.1 / 112.9; 515 rows
    111.5 / 122.8 against 256x128 130.3 / 136.5; 768 rows 190.7 / 190.2
    against 185.7 / 202.8.  The 256x256 tile moves 40% fewer bytes per FLOP
    than 192x128, and the K loop is bound by the L2 requests a CU keeps in
    flight."""
    avg = -(-m_total // max(num_experts, 1))
    if avg <= 128:
        return 128, 128
    if avg <= 256:
        return 256, 128
    return 256, 256


def _persistent_grouped_gemm_fp8(a_cat, b_expert, expert_offsets, a_scale, b_scale, num_sms,
                                 rep_m, rep_n, kernel_tile, use_atomic_queue, work_counter,
                                 queue):
    if b_expert.dtype != torch.float8_e4m3fn:
        raise ValueError("b_expert dtype should match a_cat dtype.")
    if a_scale is None or b_scale is None:
        raise ValueError("fp8 operands need a_scale [M] and b_scale [E, N] (float32).")
    m_total, k_size = a_cat.shape
    num_experts, _, n_size = b_expert.shape
    if a_scale.numel() != m_total or b_scale.numel() != num_experts * n_size:
        raise ValueError("a_scale must have M entries and b_scale E*N entries.")
    if a_scale.device != a_cat.device or b_scale.device != a_cat.device:
        raise ValueError("scales must be on the same device as input tensors.")
    device = a_cat.device
    dev_index = device.index if device.index is not None else torch.cuda.current_device()
    if kernel_tile is None:
        kernel_tile = _default_fp8_kernel_tile(m_total, num_experts)
    kbm, kbn = (int(v) for v in kernel_tile)
    if (kbm, kbn) not in _FP8_KERNEL_TILES:
        raise ValueError(f"fp8 kernel_tile must be one of {_FP8_KERNEL_TILES}.")
    if n_size & 1:
        kbm, kbn = _odd_n_tile((kbm, kbn), False)
    if queue == "device" and num_experts > _nat.MAX_DEVICE_QUEUE_EXPERTS:
        queue = "prebuilt"
    if num_sms is None:
        num_sms = _cu_count(dev_index)
    if int(num_sms) <= 0:
        raise ValueError("num_sms must be positive.")
    counter_dev = _counter_arg(work_counter, use_atomic_queue, device)
    # K to a multiple of 16 (zero padding adds nothing); any N.
    k_pad = (k_size + 15) // 16 * 16
    a_op = a_cat
    if k_pad != k_size:
        a_op = torch.nn.functional.pad(a_op.view(torch.uint8), (0, k_pad - k_size)).view(a_cat.dtype)
    if k_pad > 0 and (a_op.stride(1) != 1 or a_op.stride(0) % 16 or a_op.data_ptr() % 16):
        a_op = a_op.contiguous()
    b_nk = b_expert.transpose(1, 2)  # [E, N, K]
    if k_pad != k_size:
        b_nk = torch.nn.functional.pad(b_nk.contiguous().view(torch.uint8),
                                       (0, k_pad - k_size)).view(b_expert.dtype)
    if k_pad > 0 and (b_nk.stride(2) != 1 or b_nk.stride(1) % 16 or b_nk.stride(0) % 16
                      or b_nk.data_ptr() % 16):
        b_nk = b_nk.contiguous()
    sa = a_scale.reshape(-1).to(torch.float32).contiguous()
    sb = b_scale.reshape(num_experts, n_size).to(torch.float32).contiguous()
    off32 = _offsets_i32(expert_offsets)
    c_op = torch.empty((m_total, n_size), device=device, dtype=torch.bfloat16)
    lda = a_op.stride(0) if m_total > 1 else k_pad
    ldb_n = b_nk.stride(1) if n_size > 1 else k_pad
    ldb_e = b_nk.stride(0) if num_experts > 1 else n_size * ldb_n
    we, wm, wn, num_work = _queue_args(queue, expert_offsets, n_size, kbm, kbn)
    args = (_ptr(a_op), _ptr(b_nk), _ptr(c_op), _ptr(off32), _ptr(sa), _ptr(sb),
            m_total, k_pad, n_size, num_experts, lda, ldb_e, ldb_n, c_op.stride(0),
            _ptr(we), _ptr(wm), _ptr(wn), num_work,
            kbm, kbn, int(num_sms), 1 if use_atomic_queue else 0,
            _ptr(counter_dev), rep_m, rep_n, torch.cuda.current_stream(device).cuda_stream)
    _launch(_nat.lib().mgg_grouped_gemm_fp8, args, dev_index)
    return c_op


def quantize_fp8_rows(x: torch.Tensor, dim: int = -1):
    """(x_fp8, scale) with scale = amax / 448 along `dim` (per row of x by
    default), x_fp8 = float8_e4m3fn(x / scale): the per-token / per-channel
    recipe of the fp8 config.  Input preparation (torch ops), not a kernel."""
    amax = x.float().abs().amax(dim=dim, keepdim=True).clamp_min(1e-12)
    scale = amax / 448.0
    q = (x.float() / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, scale.squeeze(dim)


def reference_grouped_gemm(
    a_cat: torch.Tensor, b_expert: torch.Tensor, expert_offsets: torch.Tensor
) -> torch.Tensor:
    """Per-expert torch matmul loop (src/triton_grouped_gemm.py:446-457).

    The comparison loop of the reference API: one ``a[s:t] @ b[e]`` per
    non-empty expert on the tensors' own device (hipBLASLt on a GPU), rows
    outside every expert range uninitialised.  Not used by the kernels.
    """
    out = torch.empty((a_cat.size(0), b_expert.size(2)), device=a_cat.device, dtype=a_cat.dtype)
    offs = expert_offsets.detach().to("cpu", torch.int64).tolist()
    for e in range(b_expert.size(0)):
        s, t = offs[e], offs[e + 1]
        if t <= s:
            continue
        out[s:t] = a_cat[s:t] @ b_expert[e]
    return out


def grouped_gemm_flops(expert_offsets, k_size: int, n_size: int) -> int:
    """Algorithmic FLOPs 2 * sum_e max(c_e, 0) * K * N (masked work not counted)."""
    offs = torch.as_tensor(expert_offsets).detach().to("cpu", torch.int64)
    counts = (offs[1:] - offs[:-1]).clamp_min(0)
    return 2 * int(counts.sum()) * int(k_size) * int(n_size)
