"""Pins the expert-MLP oracle (oracle/expert_mlp_oracle.py) with checks that do
not restate it: an independently written counting sort, the permutation
invariants, the committed routing counts, per-token loops, and torch's own
GELU / matmul on the CPU."""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
from hypothesis import given, settings, strategies as st

import workloads
from oracle import expert_mlp_oracle as mo

GOLDEN = Path(__file__).resolve().parent / "golden"


def counting_sort_layout(idx, E):
    """Per-expert buckets filled in assignment order (no argsort)."""
    flat = [int(v) for v in np.asarray(idx).reshape(-1)]
    buckets = [[] for _ in range(E)]
    for a, e in enumerate(flat):
        if 0 <= e < E:
            buckets[e].append(a)
    counts = [len(b) for b in buckets]
    offsets = [0]
    for c in counts:
        offsets.append(offsets[-1] + c)
    pos = [-1] * len(flat)
    rows = []
    for e in range(E):
        for r, a in enumerate(buckets[e]):
            pos[a] = offsets[e] + r
            rows.append(a)
    return counts, offsets, pos, rows


@settings(max_examples=60, deadline=None)
@given(st.integers(1, 6), st.integers(0, 40), st.integers(1, 4), st.data())
def test_layout_matches_counting_sort(E, T, k, data):
    idx = np.array(data.draw(st.lists(st.integers(-2, E + 1), min_size=T * k, max_size=T * k)),
                   dtype=np.int64).reshape(T, k)
    counts, offsets, pos, tok, row = mo.dispatch_layout(idx, E)
    c2, o2, p2, r2 = counting_sort_layout(idx, E)
    assert counts.tolist() == c2
    assert offsets.tolist() == o2
    assert pos.tolist() == p2
    M = o2[-1]
    assert row[:M].tolist() == r2
    assert tok[:M].tolist() == [a // k for a in r2]


def test_layout_invariants_on_a_large_routing():
    idx, _ = workloads.topk_routing(2048, 64, 6)
    idx = idx.numpy().copy()
    idx[::7, 1] = -1  # some masked slots
    counts, offsets, pos, tok, row = mo.dispatch_layout(idx, 64)
    flat = idx.reshape(-1)
    valid = np.flatnonzero(flat >= 0)
    M = offsets[-1]
    assert M == valid.size
    assert sorted(pos[valid].tolist()) == list(range(M))  # bijection onto [0, M)
    assert np.all(pos[flat < 0] == -1)
    e_of_row = flat[row[:M]]
    assert np.all(np.diff(e_of_row) >= 0)  # expert-major
    for e in range(64):
        rows = row[offsets[e]:offsets[e + 1]]
        assert np.all(np.diff(rows) > 0)  # stable within an expert
        assert np.all(flat[rows] == e)


@pytest.mark.parametrize("name,tokens,experts,top_k", [("expert_mlp", 8192, 16, 2),
                                                        ("fp8_fine", 4096, 64, 6)])
def test_layout_counts_match_committed_routing(name, tokens, experts, top_k):
    golden = json.loads((GOLDEN / "routing_counts.json").read_text())[name]
    idx, w = workloads.topk_routing(tokens, experts, top_k, softmax=name == "expert_mlp")
    counts, offsets, *_ = mo.dispatch_layout(idx.numpy(), experts)
    assert counts.tolist() == golden
    assert offsets[-1] == tokens * top_k


def test_combine_matches_per_token_loop():
    rng = np.random.default_rng(3)
    T, k, H, E = 9, 3, 5, 4
    idx = rng.integers(-1, E, size=(T, k))
    w = rng.random((T, k)).astype(np.float32)
    counts, offsets, pos, tok, row = mo.dispatch_layout(idx, E)
    y = rng.standard_normal((T * k, H)).astype(np.float32)
    got = mo.combine_rows(y, pos, w, k)
    for t in range(T):
        ref = np.zeros(H, dtype=np.float64)
        for j in range(k):
            if idx[t, j] >= 0:
                ref += float(w[t, j]) * y[pos[t * k + j]].astype(np.float64)
        np.testing.assert_allclose(got[t], ref, rtol=1e-6, atol=1e-6)


def test_gather_rows_selects_tokens():
    x = np.arange(12, dtype=np.float32).reshape(4, 3)
    out = mo.gather_rows(x, np.array([3, 0, 0, 2, -1]), 4)
    np.testing.assert_array_equal(out, x[[3, 0, 0, 2]])


def test_interleave_gate_up_columns():
    E, H, F = 2, 3, 64
    g = np.arange(E * H * F, dtype=np.float32).reshape(E, H, F)
    u = -g - 1
    w = mo.interleave_gate_up(g, u)
    for q in range(F // 32):
        for c in range(32):
            np.testing.assert_array_equal(w[:, :, 64 * q + c], g[:, :, 32 * q + c])
            np.testing.assert_array_equal(w[:, :, 64 * q + 32 + c], u[:, :, 32 * q + c])


def test_gelu_and_silu_match_torch():
    """The oracle's activations against torch's own (train:86-93 uses
    nn.GELU; SwiGLU's gate is F.silu) in float64, over [-100, 100] and out to
    where e^-x overflows (x < -709: silu's limit there is -0.0), plus the
    values the definitions fix: gelu(0) = silu(0) = 0, silu(x) -> x."""
    x = np.concatenate([np.linspace(-100.0, 100.0, 20001), [-800.0, -710.0, -709.0, 709.0, 800.0]])
    xt = torch.tensor(x, dtype=torch.float64)
    np.testing.assert_allclose(mo.gelu(x), torch.nn.functional.gelu(xt).numpy(),
                               rtol=1e-12, atol=1e-300)
    with np.errstate(over="ignore"):
        got = mo.silu(x)
    np.testing.assert_allclose(got, torch.nn.functional.silu(xt).numpy(), rtol=1e-13, atol=1e-300)
    assert mo.gelu(np.array([0.0]))[0] == 0.0 and mo.silu(np.array([0.0]))[0] == 0.0
    assert got[-1] == 800.0 and got[np.argmin(x)] == 0.0


def per_token_mlp(x, idx, w, w1, w2, activation):
    T, k = idx.shape
    out = np.zeros((T, w2.shape[2]))
    for t in range(T):
        for j in range(k):
            e = idx[t, j]
            if not 0 <= e < w1.shape[0]:
                continue
            h = x[t].astype(np.float64) @ w1[e].astype(np.float64)
            if activation == "gelu":
                h = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in h])
            else:
                F = h.size // 2
                gate = np.concatenate([h[64 * q: 64 * q + 32] for q in range(F // 32)])
                up = np.concatenate([h[64 * q + 32: 64 * q + 64] for q in range(F // 32)])
                h = torch.nn.functional.silu(torch.from_numpy(gate)).numpy() * up
            out[t] += w[t, j] * (h @ w2[e].astype(np.float64))
    return out


@pytest.mark.parametrize("activation", ["gelu", "swiglu"])
def test_expert_mlp_matches_per_token_loop(activation):
    rng = np.random.default_rng(5)
    T, k, E, H, F = 11, 2, 3, 8, 64
    x = rng.standard_normal((T, H))
    idx = rng.integers(-1, E, size=(T, k))
    w = rng.random((T, k))
    w1 = rng.standard_normal((E, H, 2 * F if activation == "swiglu" else F)) / math.sqrt(H)
    w2 = rng.standard_normal((E, F, H)) / math.sqrt(F)
    got = mo.expert_mlp(x, idx, w, w1, w2, activation)
    ref = per_token_mlp(x, idx, w, w1, w2, activation)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-10)


def test_expert_mlp_gelu_matches_torch_reference_experts():
    """The reference's ExpertMLP (train:86-93) is w2(gelu(w1(x))) with
    nn.Linear weights; with W1 = w1.weight^T stacked (train:187-191) the
    routed sum equals torch's per-expert modules applied per slot."""
    torch.manual_seed(0)
    T, k, E, H, F = 16, 2, 4, 32, 48
    experts = [torch.nn.Sequential(torch.nn.Linear(H, F, bias=False), torch.nn.GELU(),
                                   torch.nn.Linear(F, H, bias=False)).double() for _ in range(E)]
    x = torch.randn(T, H, dtype=torch.float64)
    probs = torch.softmax(torch.randn(T, E, dtype=torch.float64), -1)
    w, idx = torch.topk(probs, k, dim=-1)
    ref = torch.zeros(T, H, dtype=torch.float64)
    for j in range(k):
        for e in range(E):
            m = idx[:, j] == e
            if m.any():
                ref[m] += experts[e](x[m]) * w[m, j, None]
    w1 = torch.stack([m[0].weight.t() for m in experts]).detach().numpy()
    w2 = torch.stack([m[2].weight.t() for m in experts]).detach().numpy()
    got = mo.expert_mlp(x.numpy(), idx.numpy(), w.numpy(), w1, w2, "gelu")
    np.testing.assert_allclose(got, ref.detach().numpy(), rtol=1e-10, atol=1e-12)
