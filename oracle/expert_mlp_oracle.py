"""CPU oracle for the routed expert MLP around the grouped GEMM -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of how the reference moves tokens to expert rows and back
(Hongyu15/moe-overlap, ``src/train_moe_baseline.py``), used as the checker in
``tests/`` and ``bench.py``'s ``cpu_baseline`` leg.  Nothing in the product
(``moe-overlap_amd/``) imports it.

Functions and what pins each one (tests/test_oracle_mlp.py):

* ``dispatch_layout`` -- train:219-237 (valid mask, sort by expert, bincount,
  cumsum offsets, inv_perm), over all top-k slots at once.  Pinned by a
  counting-sort loop written independently, by the permutation invariants
  (positions are a bijection onto [0, M), expert-major, stable in assignment
  order within an expert) and by the per-expert counts of the benchmark
  expert-MLP and fp8 routings in tests/golden/routing_counts.json.
* ``gather_rows`` / ``combine_rows`` -- train:224 (grouped_tokens =
  valid_tokens[perm]) and train:245-246 with :340-341 (out[valid] =
  grouped_out[inv_perm]; out += y * gate over the slots).  Pinned by
  per-token loops.
* ``expert_mlp`` -- the expert computation of train:239-243 (GELU on a
  single W1, the reference's ExpertMLP :86-93) and the SwiGLU variant of the
  benchmark's expert-MLP configuration, in float64 via the permuted grouped form.
  Pinned against a per-token loop, and (GELU) against torch's own
  ``F.gelu(x @ w1) @ w2`` per expert on the CPU.
* ``interleave_gate_up`` -- the gate|up column layout mgg_grouped_gemm_ex
  expects (groups of 32 gate then 32 up columns).  Pinned by index checks.
"""
from __future__ import annotations

import math

import numpy as np

__all__ = [
    "dispatch_layout",
    "gather_rows",
    "combine_rows",
    "gelu",
    "silu",
    "interleave_gate_up",
    "expert_mlp",
]


def dispatch_layout(topk_idx, num_experts: int):
    """(counts, offsets, slot_position, token_index, row_assignment) of a routing.

    ``topk_idx`` is [T, k]; entries outside [0, E) are masked.  Assignment
    a = t*k + j goes to row offsets[e] + (number of earlier assignments to e).
    ``token_index`` / ``row_assignment`` have T*k entries, valid below
    offsets[E] (the rest is -1 here)."""
    idx = np.asarray(topk_idx).astype(np.int64)
    T, k = idx.shape if idx.ndim == 2 else (idx.shape[0], 1)
    flat = idx.reshape(-1)
    E = int(num_experts)
    valid = (flat >= 0) & (flat < E)
    a_valid = np.flatnonzero(valid)
    order = np.argsort(flat[a_valid], kind="stable")  # torch.sort by expert, stable
    rows = a_valid[order]  # assignment of each row
    counts = np.bincount(flat[a_valid], minlength=E).astype(np.int32)[:E] if E else np.zeros(0, np.int32)
    offsets = np.zeros(E + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts, dtype=np.int64).astype(np.int32)
    slot_position = np.full(flat.size, -1, dtype=np.int32)
    slot_position[rows] = np.arange(rows.size, dtype=np.int32)  # inv_perm
    token_index = np.full(flat.size, -1, dtype=np.int32)
    row_assignment = np.full(flat.size, -1, dtype=np.int32)
    token_index[: rows.size] = (rows // k).astype(np.int32)
    row_assignment[: rows.size] = rows.astype(np.int32)
    return counts, offsets, slot_position, token_index, row_assignment


def gather_rows(x, token_index, rows: int) -> np.ndarray:
    x = np.asarray(x)
    return x[np.asarray(token_index)[:rows]]


def combine_rows(y, slot_position, weights, top_k: int, acc_dtype=np.float32) -> np.ndarray:
    """out[t] = sum over valid slots j of w[t, j] * y[pos[t, j]], accumulated in slot order."""
    y = np.asarray(y)
    pos = np.asarray(slot_position).reshape(-1, top_k)
    w = np.asarray(weights, dtype=acc_dtype).reshape(-1, top_k)
    out = np.zeros((pos.shape[0], y.shape[1]), dtype=acc_dtype)
    for j in range(top_k):
        ok = pos[:, j] >= 0
        out[ok] += w[ok, j, None] * y[pos[ok, j]].astype(acc_dtype)
    return out


_erf = np.vectorize(math.erf, otypes=[np.float64])


def gelu(x):
    """Exact (erf) GELU, torch.nn.functional.gelu's default."""
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + _erf(x / math.sqrt(2.0)))


def silu(x):
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def interleave_gate_up(w_gate, w_up) -> np.ndarray:
    """[E, H, F] gate and up projections -> [E, H, 2F] with, for every q,
    columns 64q..64q+31 = gate[..., 32q..32q+31] and 64q+32..64q+63 = up[..., 32q..]."""
    g = np.asarray(w_gate)
    u = np.asarray(w_up)
    E, H, F = g.shape
    assert F % 32 == 0 and u.shape == g.shape
    out = np.empty((E, H, 2 * F), dtype=g.dtype)
    gv = g.reshape(E, H, F // 32, 32)
    uv = u.reshape(E, H, F // 32, 32)
    ov = out.reshape(E, H, F // 32, 64)
    ov[..., :32] = gv
    ov[..., 32:] = uv
    return out


def expert_mlp(x, topk_idx, topk_weight, w1, w2, activation: str = "gelu") -> np.ndarray:
    """Routed expert MLP in float64: permute, per-expert up projection with the
    activation, down projection, gate-weighted combine.

    activation "gelu":   w1 [E, H, F], h = gelu(x @ w1[e]).
    activation "swiglu": w1 [E, H, 2F] interleaved (interleave_gate_up),
                         h = silu(x @ gate) * (x @ up).
    w2 [E, F, H]."""
    x = np.asarray(x, dtype=np.float64)
    idx = np.asarray(topk_idx)
    k = idx.shape[1]
    E = w1.shape[0]
    w1 = np.asarray(w1, dtype=np.float64)
    w2 = np.asarray(w2, dtype=np.float64)
    counts, offsets, pos, token_index, _ = dispatch_layout(idx, E)
    M = int(offsets[-1])
    xp = x[token_index[:M]]
    y = np.zeros((M, w2.shape[2]), dtype=np.float64)
    for e in range(E):
        s, t = int(offsets[e]), int(offsets[e + 1])
        if t <= s:
            continue
        h = xp[s:t] @ w1[e]
        if activation == "gelu":
            h = gelu(h)
        elif activation == "swiglu":
            F2 = h.shape[1]
            hv = h.reshape(t - s, F2 // 64, 64)
            h = (silu(hv[..., :32]) * hv[..., 32:]).reshape(t - s, F2 // 2)
        else:
            raise ValueError(activation)
        y[s:t] = h @ w2[e]
    return combine_rows(y, pos, topk_weight, k, acc_dtype=np.float64)
