"""Routed expert MLP on the MI355X grouped GEMM (one GPU's share).

The reference runs its experts as (src/train_moe_baseline.py:212-248, :335-341):

    valid = expert_ids >= 0; sort by expert; grouped_tokens = tokens[perm]
    offsets = cumsum(bincount(...)); hidden = gelu(grouped_gemm(tokens, w1))
    grouped_out = grouped_gemm(hidden, w2); out[valid] = grouped_out[inv_perm]
    out += y * gate                     (once per top-k slot)

Here all T*k assignments go through in one pass, with no host
synchronisation: the dispatch layout (two kernels), the up-projection GEMM
reading its rows through the layout (the row gather fused; a separate gather
launch for shapes the fused path does not take) with the activation fused
into its epilogue, the down-projection GEMM and the gate-weighted combine:
five launches on the current stream.  Buffers are
sized for T*k rows; the kernels read the number of valid rows (offsets[E])
on the device.  Every op runs in libmgg.so (include/mgg.h); there is no
fallback implementation.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

import mgg_native as nat
from grouped_gemm import _queue_args, persistent_grouped_gemm

__all__ = [
    "DispatchLayout",
    "dispatch_layout",
    "permute_tokens",
    "combine_tokens",
    "interleave_gate_up",
    "expert_mlp_forward",
    "expert_mlp_flops",
]

_DTYPES = {torch.bfloat16: nat.MGG_DTYPE_BF16, torch.float16: nat.MGG_DTYPE_FP16}
_EPILOGUES = {"none": nat.MGG_EPI_NONE, "gelu": nat.MGG_EPI_GELU, "swiglu": nat.MGG_EPI_SWIGLU}


def _p(t: Optional[torch.Tensor]) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _require_cuda(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError("expert MLP ops require CUDA tensors.")


def _stream_ptr(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


@dataclass
class DispatchLayout:
    """Where each (token, slot) assignment lives in the expert-major row order.

    counts [E], offsets [E+1], slot_position [T*k] (-1 for masked slots),
    token_index / row_assignment [T*k] (valid below offsets[E]); all int32 on
    the device.  top_k and num_tokens describe the routing it came from."""

    counts: torch.Tensor
    offsets: torch.Tensor
    slot_position: torch.Tensor
    token_index: torch.Tensor
    row_assignment: torch.Tensor
    num_tokens: int
    top_k: int

    @property
    def max_rows(self) -> int:
        return self.num_tokens * self.top_k


def dispatch_layout(topk_idx: torch.Tensor, num_experts: int) -> DispatchLayout:
    """Counts, offsets and stable row positions of a [T, k] routing (entries
    outside [0, E) are masked), on the device without a host round trip."""
    _require_cuda(topk_idx)
    if topk_idx.dim() != 2:
        raise ValueError("topk_idx must be [num_tokens, top_k]")
    if topk_idx.dtype not in (torch.int32, torch.int64):
        raise ValueError("topk_idx must be int32 or int64")
    idx = topk_idx.contiguous()
    T, k = idx.shape
    dev = idx.device
    i32 = dict(dtype=torch.int32, device=dev)
    counts = torch.empty(num_experts, **i32)
    offsets = torch.empty(num_experts + 1, **i32)
    slot = torch.empty(T * k, **i32)
    tok = torch.empty(T * k, **i32)
    row = torch.empty(T * k, **i32)
    lib = nat.lib()
    ws_bytes = int(lib.mgg_dispatch_layout_workspace_bytes(T, k, num_experts))
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        nat.check(lib.mgg_dispatch_layout(
            _p(idx), nat.MGG_INT64 if idx.dtype == torch.int64 else nat.MGG_INT32, T, k,
            num_experts, _p(counts), _p(offsets), _p(slot), _p(tok), _p(row), _p(ws), ws_bytes,
            _stream_ptr(dev)))
    return DispatchLayout(counts, offsets, slot, tok, row, T, k)


def permute_tokens(x: torch.Tensor, layout: DispatchLayout) -> torch.Tensor:
    """[T*k, H] rows in expert-major order (rows at and past offsets[E] are
    left unwritten): grouped_tokens = tokens[perm] of train:224."""
    _require_cuda(x)
    if x.dim() != 2 or x.dtype not in _DTYPES or x.stride(1) != 1:
        raise ValueError("x must be a 2-D bf16/fp16 tensor with unit inner stride")
    out = torch.empty(layout.max_rows, x.shape[1], dtype=x.dtype, device=x.device)
    num_rows = layout.offsets[-1:]  # device int32: the number of valid rows
    with torch.cuda.device(x.device):
        nat.check(nat.lib().mgg_gather_rows(
            _DTYPES[x.dtype], _p(x), x.stride(0), _p(layout.token_index), _p(num_rows),
            layout.max_rows, x.shape[1], _p(out), out.stride(0), _stream_ptr(x.device)))
    return out


def combine_tokens(y: torch.Tensor, layout: DispatchLayout, topk_weight: torch.Tensor) -> torch.Tensor:
    """out[t] = sum_j w[t, j] * y[slot_position[t, j]] over the valid slots
    (fp32 accumulation), the reference's inv_perm scatter plus gated sum."""
    _require_cuda(y, topk_weight)
    if y.dim() != 2 or y.dtype not in _DTYPES or y.stride(1) != 1:
        raise ValueError("y must be a 2-D bf16/fp16 tensor with unit inner stride")
    if tuple(topk_weight.shape) != (layout.num_tokens, layout.top_k):
        raise ValueError("topk_weight must be [num_tokens, top_k]")
    w = topk_weight.to(torch.float32).contiguous()
    out = torch.empty(layout.num_tokens, y.shape[1], dtype=y.dtype, device=y.device)
    with torch.cuda.device(y.device):
        nat.check(nat.lib().mgg_combine_rows(
            _DTYPES[y.dtype], _p(y), y.stride(0), _p(layout.slot_position), _p(w),
            layout.num_tokens, layout.top_k, y.shape[1], _p(out), out.stride(0),
            _stream_ptr(y.device)))
    return out


def interleave_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """[E, H, F] gate and up projections -> the [E, H, 2F] layout the fused
    SwiGLU epilogue reads: columns 64q..64q+31 are gate outputs 32q..32q+31,
    columns 64q+32..64q+63 the up outputs of the same indices.  A weight-load
    time transform (one copy), not part of the forward pass."""
    if w_gate.shape != w_up.shape or w_gate.dim() != 3 or w_gate.shape[2] % 32 != 0:
        raise ValueError("w_gate and w_up must both be [E, H, F] with F % 32 == 0")
    E, H, F = w_gate.shape
    out = torch.empty(E, H, F // 32, 64, dtype=w_gate.dtype, device=w_gate.device)
    out[..., :32] = w_gate.reshape(E, H, F // 32, 32)
    out[..., 32:] = w_up.reshape(E, H, F // 32, 32)
    return out.reshape(E, H, 2 * F)


def expert_mlp_flops(layout_rows: int, hidden: int, w1_cols: int, w2_rows: int) -> int:
    """2*M*H*N1 + 2*M*F*H for M routed rows (algorithmic, masked rows excluded)."""
    return 2 * layout_rows * hidden * w1_cols + 2 * layout_rows * w2_rows * hidden


def expert_mlp_forward(
    x: torch.Tensor,
    topk_idx: torch.Tensor,
    topk_weight: torch.Tensor,
    w1: torch.Tensor,
    w2: torch.Tensor,
    activation: str = "gelu",
    num_sms: Optional[int] = None,
    block: int = 256,
    use_atomic_queue: bool = True,
) -> torch.Tensor:
    """Routed expert MLP for tokens x [T, H] routed by topk_idx/topk_weight [T, k].

    activation "gelu":   w1 [E, H, F] (the reference's stacked W1^T), F.gelu.
    activation "swiglu": w1 [E, H, 2F] from interleave_gate_up(gate, up),
                         silu(x @ gate) * (x @ up).
    w2 [E, F, H].  Returns [T, H] in x's dtype: sum over the top-k slots of
    gate * expert(x), the value the reference accumulates per slot."""
    _require_cuda(x, topk_idx, topk_weight, w1, w2)
    if activation not in ("gelu", "swiglu"):
        raise ValueError("activation must be 'gelu' or 'swiglu'")
    if x.dtype not in _DTYPES or w1.dtype != x.dtype or w2.dtype != x.dtype:
        raise ValueError("x, w1 and w2 must share a bf16/fp16 dtype")
    if x.dim() != 2 or w1.dim() != 3 or w2.dim() != 3 or w1.shape[1] != x.shape[1]:
        raise ValueError("expected x [T, H], w1 [E, H, N1], w2 [E, F, H]")
    E = w1.shape[0]
    F = w1.shape[2] // 2 if activation == "swiglu" else w1.shape[2]
    if w2.shape[0] != E or w2.shape[1] != F or w2.shape[2] != x.shape[1]:
        raise ValueError("w2 must be [E, F, H] matching w1 and x")
    layout = dispatch_layout(topk_idx, E)
    if _gathered_ok(x, w1, block):
        # The gather of train:224 runs inside the up GEMM: its A rows are read
        # from x through layout.token_index (bitwise the same result).
        h = _grouped_gemm_gathered(x, layout, w1, _EPILOGUES[activation], F, num_sms,
                                   use_atomic_queue)
    else:
        xp = permute_tokens(x, layout)
        h = _grouped_gemm_ex(xp, w1, layout.offsets, _EPILOGUES[activation], F, num_sms, block,
                             use_atomic_queue)
    y = _grouped_gemm_ex(h, w2, layout.offsets, nat.MGG_EPI_NONE, x.shape[1], num_sms, block,
                         use_atomic_queue)
    return combine_tokens(y, layout, topk_weight)


def _gathered_ok(x, w1, block):
    """Whether the up GEMM can read its A rows from x in place: the 256x256
    tile with N-major weights (any N and strides), the device-derived queue,
    16-byte aligned rows of x and 32-bit offsets into x."""
    return (block == 256 and w1.shape[0] <= nat.MAX_DEVICE_QUEUE_EXPERTS
            and x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0
            and w1.stride(2) == 1 and w1.data_ptr() % 16 == 0 and x.shape[1] % 8 == 0
            and (x.shape[0] * x.stride(0) + x.shape[1]) * 2 < (1 << 31) - 4096)


def _grouped_gemm_gathered(x, layout, w1, epilogue, out_cols, num_sms, use_atomic_queue):
    """C [T*k, out_cols] = epilogue(x[token_index] @ w1[e]) over the expert row
    ranges of the layout, in one launch (rows past offsets[E] unwritten)."""
    T, H = x.shape
    E, _, N = w1.shape
    M = layout.max_rows
    c = torch.empty(M, out_cols, dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        nat.check(nat.lib().mgg_grouped_gemm_gathered(
            _DTYPES[x.dtype], epilogue, _p(x), _p(layout.token_index), T, _p(w1), _p(c),
            _p(layout.offsets), M, H, N, E, x.stride(0), w1.stride(0), w1.stride(1), c.stride(0),
            int(num_sms) if num_sms else 0, 1 if use_atomic_queue else 0, _stream_ptr(x.device)))
    return c


def _grouped_gemm_ex(a, b, offsets, epilogue, out_cols, num_sms, block, use_atomic_queue):
    """C [M, out_cols] = epilogue(A @ B[e]) over the expert row ranges, on the
    block x block kernel tile (queue derived on the device; above 2048
    experts prebuilt, as the drop-in does)."""
    if epilogue == nat.MGG_EPI_NONE:
        return persistent_grouped_gemm(a, b, offsets, num_sms=num_sms, block_m=block,
                                       block_n=block, use_atomic_queue=use_atomic_queue,
                                       kernel_tile=(block, block))
    M, K = a.shape
    E, _, N = b.shape
    kmajor = b.stride(1) == 1 and b.stride(2) != 1  # [E, K, N] view of [E, N, K] weights
    if a.stride(1) != 1 or (b.stride(2) != 1 and not kmajor):
        raise ValueError("operands need unit inner strides (B: along N, or along K)")
    dtype = _DTYPES[a.dtype] | (nat.MGG_B_KMAJOR if kmajor else 0)
    ldb_rows = b.stride(2) if kmajor else b.stride(1)
    c = torch.empty(M, out_cols, dtype=a.dtype, device=a.device)
    queue = ("prebuilt" if E > nat.MAX_DEVICE_QUEUE_EXPERTS else "device")
    we, wm, wn, num_work = _queue_args(queue, offsets, N, block, block)
    with torch.cuda.device(a.device):
        nat.check(nat.lib().mgg_grouped_gemm_ex(
            dtype, epilogue, _p(a), _p(b), _p(c), _p(offsets), M, K, N, E,
            a.stride(0), b.stride(0), ldb_rows, c.stride(0), _p(we), _p(wm), _p(wn), num_work,
            block, block, int(num_sms) if num_sms else 0, 1 if use_atomic_queue else 0, None,
            0, 0, _stream_ptr(a.device)))
    return c
