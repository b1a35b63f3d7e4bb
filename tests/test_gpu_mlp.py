"""GPU parity of the routed expert-MLP path (libmgg's dispatch layout, row
gather, fused-epilogue grouped GEMM and combine, all through the C ABI)
against the CPU oracle (oracle/expert_mlp_oracle.py) and plain fp32 torch.

Integer outputs (layout, gather) are bit-exact.  Floating point:
* fused epilogues: max |C - ref_fp32| <= 2 * tol(K), tol(K) = 2e-2 *
  sqrt(max(K, 512) / 512) as for the plain GEMM, doubled because the
  activation of two rounded accumulations (SwiGLU's silu(gate) * up) can
  carry both errors;
* combine: relative 2^-8 (one bf16 rounding of an fp32 sum);
* whole MLP: the hidden layer is rounded to bf16 between the GEMMs (as the
  reference's persistent_grouped_gemm output is), so the bound is that of
  the down GEMM over K = F plus the up GEMM's rounding carried through it:
  max-abs <= 2 * tol(F), and relative RMS error <= 1e-2.
"""
import math
import sys

import numpy as np
import pytest
import torch

import expert_mlp as mlp
import workloads
from oracle import expert_mlp_oracle as mo

pytestmark = pytest.mark.gpu


def tol(k):
    return 2e-2 * math.sqrt(max(k, 512) / 512)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def random_routing(T, k, E, masked_every=0, seed=0, dtype=torch.int64):
    gen = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, max(E, 1), (T, k), generator=gen)
    if masked_every:
        idx.view(-1)[::masked_every] = -1
    w = torch.rand(T, k, generator=gen)
    return idx.to(dtype), w


# (T, k, E, masked_every).  Paths: no assignments; the position pass with
# the scan inside it (chunks x experts <= 16384: the next four); the
# separate scan with the wide position pass (157 chunks x 256 experts); the
# one-wave position pass (E > 1024).
LAYOUT_CASES = [
    (0, 2, 4, 0),
    (1, 1, 1, 0),
    (37, 3, 5, 4),
    (1500, 2, 3, 0),
    (3000, 4, 300, 9),
    (20000, 8, 256, 7),
    (700, 8, 8192, 5),
]


@pytest.mark.parametrize("T,k,E,masked", LAYOUT_CASES)
@pytest.mark.parametrize("idx_dtype", [torch.int64, torch.int32])
def test_dispatch_layout_bit_exact(cuda_device, T, k, E, masked, idx_dtype):
    log(f"layout T={T} k={k} E={E} masked={masked} {idx_dtype}")
    idx, _ = random_routing(T, k, E, masked, seed=T + E, dtype=idx_dtype)
    lay = mlp.dispatch_layout(idx.to(cuda_device), E)
    torch.cuda.synchronize()
    counts, offsets, pos, tok, row = mo.dispatch_layout(idx.numpy(), E)
    M = int(offsets[-1])
    np.testing.assert_array_equal(lay.counts.cpu().numpy(), counts)
    np.testing.assert_array_equal(lay.offsets.cpu().numpy(), offsets)
    np.testing.assert_array_equal(lay.slot_position.cpu().numpy(), pos)
    np.testing.assert_array_equal(lay.token_index.cpu().numpy()[:M], tok[:M])
    np.testing.assert_array_equal(lay.row_assignment.cpu().numpy()[:M], row[:M])


@pytest.mark.parametrize("name,T,E,k", [("expert_mlp", 8192, 16, 2), ("fp8_fine", 4096, 64, 6)])
def test_dispatch_layout_baseline_routings(cuda_device, name, T, E, k):
    log(f"layout {name}")
    idx, _ = workloads.topk_routing(T, E, k, softmax=name == "expert_mlp")
    lay = mlp.dispatch_layout(idx.to(cuda_device), E)
    counts, offsets, pos, tok, row = mo.dispatch_layout(idx.numpy(), E)
    np.testing.assert_array_equal(lay.counts.cpu().numpy(), counts)
    np.testing.assert_array_equal(lay.slot_position.cpu().numpy(), pos)
    np.testing.assert_array_equal(lay.token_index.cpu().numpy(), tok)


def test_gather_rows_bit_exact(cuda_device):
    log("gather")
    T, k, E, H = 300, 3, 7, 264
    idx, _ = random_routing(T, k, E, masked_every=5)
    x = torch.randn(T, H).to(torch.bfloat16)
    lay = mlp.dispatch_layout(idx.to(cuda_device), E)
    xp = mlp.permute_tokens(x.to(cuda_device), lay).cpu()
    _, offsets, _, tok, _ = mo.dispatch_layout(idx.numpy(), E)
    M = int(offsets[-1])
    assert torch.equal(xp[:M], x[torch.from_numpy(tok[:M]).long()])
    # unaligned row length (element path)
    x2 = torch.randn(T, 13).to(torch.float16)
    xp2 = mlp.permute_tokens(x2.to(cuda_device), lay).cpu()
    assert torch.equal(xp2[:M], x2[torch.from_numpy(tok[:M]).long()])


@pytest.mark.parametrize("H", [256, 13])
# 1, 2: one slot at a time; 4, 10: slots loaded in groups of four (10: two
# groups and a partial one)
@pytest.mark.parametrize("k", [1, 2, 4, 10])
def test_combine_matches_oracle(cuda_device, H, k):
    log(f"combine H={H} k={k}")
    T, E = 257, 12
    idx, w = random_routing(T, k, E, masked_every=3)
    lay = mlp.dispatch_layout(idx.to(cuda_device), E)
    y = torch.randn(T * k, H).to(torch.bfloat16)
    got = mlp.combine_tokens(y.to(cuda_device), lay, w.to(cuda_device)).float().cpu().numpy()
    _, _, pos, _, _ = mo.dispatch_layout(idx.numpy(), E)
    ref = mo.combine_rows(y.float().numpy(), pos, w.numpy(), k, acc_dtype=np.float64)
    np.testing.assert_allclose(got, ref, rtol=2 ** -8, atol=1e-6)
    masked_tokens = (idx < 0).all(dim=1)
    if masked_tokens.any():
        assert np.all(got[masked_tokens.numpy()] == 0)


def fp32_epilogue_ref(a, b, offs, activation):
    out = []
    o = offs.cpu().tolist()
    for e in range(len(o) - 1):
        if o[e + 1] <= o[e]:
            continue
        h = a[o[e]:o[e + 1]].float() @ b[e].float()
        if activation == "gelu":
            h = torch.nn.functional.gelu(h)
        elif activation == "swiglu":
            hv = h.reshape(h.shape[0], -1, 64)
            h = (torch.nn.functional.silu(hv[..., :32]) * hv[..., 32:]).reshape(h.shape[0], -1)
        out.append((o[e], o[e + 1], h))
    return out


@pytest.mark.parametrize("activation", ["gelu", "swiglu"])
@pytest.mark.parametrize("block", [128, 256])
@pytest.mark.parametrize("atomic", [False, True])
def test_fused_epilogue_gemm(cuda_device, activation, block, atomic):
    log(f"epilogue {activation} block={block} atomic={atomic}")
    counts = [37, 0, 300, 5, 129]
    K, N = 512, 384
    gen = torch.Generator().manual_seed(7)
    M = sum(counts)
    a = torch.randn(M, K, generator=gen).to(torch.bfloat16).to(cuda_device)
    b = (torch.randn(len(counts), K, N, generator=gen) / math.sqrt(K)).to(torch.bfloat16).to(cuda_device)
    offs = torch.tensor([0] + list(np.cumsum(counts)), dtype=torch.int32, device=cuda_device)
    epi = mlp._EPILOGUES[activation]
    cols = N // 2 if activation == "swiglu" else N
    c = mlp._grouped_gemm_ex(a, b, offs, epi, cols, None, block, atomic).float()
    for s, t, h in fp32_epilogue_ref(a, b, offs, activation):
        err = (c[s:t] - h).abs().max().item()
        assert err <= 2 * tol(K), (activation, block, s, err)


@pytest.mark.parametrize("activation", ["gelu", "swiglu"])
def test_fp16_epilogues_and_mlp(cuda_device, activation):
    """The fp16 instantiations of the fused epilogues, and the routed MLP in
    fp16 (same bounds as bf16; fp16's finer mantissa only tightens them)."""
    log(f"fp16 {activation}")
    counts = [70, 0, 301, 9]
    K, N = 512, 256
    gen = torch.Generator().manual_seed(21)
    M = sum(counts)
    a = torch.randn(M, K, generator=gen).to(torch.float16).to(cuda_device)
    b = (torch.randn(len(counts), K, N, generator=gen) / math.sqrt(K)).to(torch.float16).to(cuda_device)
    offs = torch.tensor([0] + list(np.cumsum(counts)), dtype=torch.int32, device=cuda_device)
    cols = N // 2 if activation == "swiglu" else N
    for block in (128, 256):
        c = mlp._grouped_gemm_ex(a, b, offs, mlp._EPILOGUES[activation], cols, None, block, True)
        assert c.dtype == torch.float16
        for s0, t0, h in fp32_epilogue_ref(a, b, offs, activation):
            assert (c.float()[s0:t0] - h).abs().max().item() <= 2 * tol(K)
    T, k, E, H, F = 150, 2, 4, 128, 128
    idx, w = random_routing(T, k, E, masked_every=7, seed=8)
    x = torch.randn(T, H, generator=gen).to(torch.float16)
    w1 = (torch.randn(E, H, 2 * F if activation == "swiglu" else F, generator=gen) / math.sqrt(H)).to(torch.float16)
    w2 = (torch.randn(E, F, H, generator=gen) / math.sqrt(F)).to(torch.float16)
    got = mlp.expert_mlp_forward(x.to(cuda_device), idx.to(cuda_device), w.to(cuda_device),
                                 w1.to(cuda_device), w2.to(cuda_device), activation)
    assert got.dtype == torch.float16
    ref = mo.expert_mlp(x.float().numpy(), idx.numpy(), w.numpy(), w1.float().numpy(),
                        w2.float().numpy(), activation)
    err = np.abs(got.float().cpu().numpy() - ref)
    assert err.max() <= 2 * tol(F), err.max()


def test_fused_epilogue_rejects_unsupported_shapes(cuda_device):
    a = torch.zeros(64, 64, dtype=torch.bfloat16, device=cuda_device)
    b = torch.zeros(1, 64, 96, dtype=torch.bfloat16, device=cuda_device)
    offs = torch.tensor([0, 64], dtype=torch.int32, device=cuda_device)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        mlp._grouped_gemm_ex(a, b, offs, mlp._EPILOGUES["swiglu"], 48, None, 128, True)
    b2 = torch.zeros(1, 64, 128, dtype=torch.bfloat16, device=cuda_device)
    with pytest.raises(RuntimeError, match="block_m == block_n"):
        mlp._grouped_gemm_ex(a, b2, offs, mlp._EPILOGUES["gelu"], 128, None, 64, True)


@pytest.mark.parametrize("activation", ["gelu", "swiglu"])
def test_expert_mlp_small_matches_oracle(cuda_device, activation):
    log(f"mlp small {activation}")
    T, k, E, H, F = 200, 2, 5, 256, 256
    idx, w = random_routing(T, k, E, masked_every=11, seed=3)
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(T, H, generator=gen).to(torch.bfloat16)
    w1 = (torch.randn(E, H, 2 * F if activation == "swiglu" else F, generator=gen) / math.sqrt(H)).to(torch.bfloat16)
    w2 = (torch.randn(E, F, H, generator=gen) / math.sqrt(F)).to(torch.bfloat16)
    got = mlp.expert_mlp_forward(x.to(cuda_device), idx.to(cuda_device), w.to(cuda_device),
                                 w1.to(cuda_device), w2.to(cuda_device), activation,
                                 block=128).float().cpu().numpy()
    ref = mo.expert_mlp(x.float().numpy(), idx.numpy(), w.numpy(), w1.float().numpy(),
                        w2.float().numpy(), activation)
    err = np.abs(got - ref)
    assert err.max() <= 2 * tol(F), err.max()
    assert np.sqrt((err ** 2).mean() / max((ref ** 2).mean(), 1e-30)) <= 1e-2


@pytest.mark.parametrize("seed", range(6))
def test_expert_mlp_random_shapes(cuda_device, seed):
    """Seeded random routed MLPs (tokens, top-k, experts, hidden and FFN sizes,
    masked slots, both activations, both tile sizes) against the oracle."""
    rng = np.random.default_rng(200 + seed)
    T = int(rng.integers(1, 700))
    k = int(rng.integers(1, 5))
    E = int(rng.integers(1, 20))
    H = 64 * int(rng.integers(1, 9))
    F = 64 * int(rng.integers(1, 9))
    activation = ("gelu", "swiglu")[seed % 2]
    block = (128, 256)[(seed // 2) % 2]
    log(f"mlp random seed={seed} T={T} k={k} E={E} H={H} F={F} {activation} block={block}")
    idx, w = random_routing(T, k, E, masked_every=int(rng.integers(0, 6)), seed=seed)
    gen = torch.Generator().manual_seed(300 + seed)
    x = torch.randn(T, H, generator=gen).to(torch.bfloat16)
    w1 = (torch.randn(E, H, 2 * F if activation == "swiglu" else F, generator=gen) / math.sqrt(H)).to(torch.bfloat16)
    w2 = (torch.randn(E, F, H, generator=gen) / math.sqrt(F)).to(torch.bfloat16)
    got = mlp.expert_mlp_forward(x.to(cuda_device), idx.to(cuda_device), w.to(cuda_device),
                                 w1.to(cuda_device), w2.to(cuda_device), activation,
                                 block=block).float().cpu().numpy()
    ref = mo.expert_mlp(x.float().numpy(), idx.numpy(), w.numpy(), w1.float().numpy(),
                        w2.float().numpy(), activation)
    err = np.abs(got - ref)
    assert err.max() <= 2 * tol(F), err.max()
    assert np.sqrt((err ** 2).mean() / max((ref ** 2).mean(), 1e-30)) <= 1e-2


def test_expert_mlp_baseline_config(cuda_device):
    """benchmark expert-MLP config (8192 tokens, top-2 of 16, H 2048, SwiGLU F
    4096) against an fp32 torch computation of the same routed MLP."""
    log("mlp cfg4")
    case = workloads.make_expert_mlp_case(device=cuda_device)
    w1 = mlp.interleave_gate_up(case.w_gate, case.w_up)
    got = mlp.expert_mlp_forward(case.x, case.topk_idx, case.topk_weight, w1, case.w2, "swiglu")
    torch.cuda.synchronize()
    ref = torch.zeros(case.tokens, case.hidden, device=cuda_device)
    x32 = case.x.float()
    for e in range(case.experts):
        for j in range(case.top_k):
            sel = (case.topk_idx[:, j] == e).nonzero().flatten()
            if sel.numel() == 0:
                continue
            xe = x32[sel]
            h = torch.nn.functional.silu(xe @ case.w_gate[e].float()) * (xe @ case.w_up[e].float())
            # the product rounds the hidden layer to bf16 between the GEMMs
            y = h.to(torch.bfloat16).float() @ case.w2[e].float()
            ref[sel] += case.topk_weight[sel, j, None] * y
    err = (got.float() - ref).abs()
    rel_rms = (err.pow(2).mean() / ref.pow(2).mean()).sqrt().item()
    log(f"cfg4 max abs {err.max().item():.4g} rel rms {rel_rms:.3g}")
    assert err.max().item() <= 2 * tol(case.ffn)
    assert rel_rms <= 1e-2


def test_expert_mlp_graph_capture(cuda_device):
    """The whole routed MLP forward (layout, gathered up GEMM + SwiGLU, down
    GEMM, combine; atomic schedule) captured into a HIP graph replays
    correctly again and again: new token values copied into the captured
    input between replays, eager forwards and host syncs in between.  A
    captured atomic launch takes every tile whole, so each replay equals the
    eager striped forward bit for bit."""
    T, k, E, H, F = 1024, 2, 8, 256, 512
    idx, wts = random_routing(T, k, E, seed=5)
    gen = torch.Generator().manual_seed(5)
    xs = [torch.randn(T, H, generator=gen).to(torch.bfloat16).to(cuda_device) for _ in range(3)]
    w1 = (torch.randn(E, H, 2 * F, generator=gen) / math.sqrt(H)).to(torch.bfloat16).to(cuda_device)
    w2 = (torch.randn(E, F, H, generator=gen) / math.sqrt(F)).to(torch.bfloat16).to(cuda_device)
    idx, wts = idx.to(cuda_device), wts.to(cuda_device)
    assert mlp._gathered_ok(xs[0], w1, 256)
    x_in = xs[0].clone()
    fwd = lambda x, atomic: mlp.expert_mlp_forward(x, idx, wts, w1, w2, "swiglu",
                                                   use_atomic_queue=atomic)
    side = torch.cuda.Stream(device=cuda_device)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        fwd(x_in, True)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = fwd(x_in, True)
    for rep in range(6):
        x = xs[rep % 3]
        want = fwd(x, False)
        x_in.copy_(x)
        torch.cuda.synchronize()
        log(f"mlp graph replay {rep}")
        graph.replay()
        eager_atomic = fwd(x, True)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(captured, want), rep
        assert (eager_atomic.float() - want.float()).abs().max().item() <= 2 * tol(F), rep


def _activation_probe(values_a, cols_a, n, dtype, device):
    """One expert whose GEMM output C[r, :] is exactly a chosen pre-activation:
    A[r, c] = values_a[c][r] for the first columns, B[0] routes column c of A
    onto the output columns cols_a[c]."""
    m = values_a[0].numel()
    k = 64
    a = torch.zeros(m, k, dtype=dtype)
    b = torch.zeros(1, k, n, dtype=dtype)
    for c, (vals, cols) in enumerate(zip(values_a, cols_a)):
        a[:, c] = vals.to(dtype)
        b[0, c, cols] = 1.0
    offs = torch.tensor([0, m], dtype=torch.int32)
    return a.to(device), b.to(device), offs.to(device)


def _wide_inputs(m, lo, hi, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.linspace(lo, hi, m - 16)
    x = x + torch.rand(m - 16, generator=gen) * (hi - lo) / m
    special = torch.tensor([0.0, -0.0, 1e-3, -1e-3, 1e-20, -1e-20, 5.0, -5.0,
                            hi, lo, 88.0, -88.0, 89.0, -89.0, 0.70710678, -0.70710678])
    return torch.cat([x, special]).to(torch.bfloat16)


@pytest.mark.parametrize("block", [256, 128])
def test_gelu_epilogue_accuracy_over_wide_range(cuda_device, block):
    """The epilogue's erf (Abramowitz-Stegun 7.1.26 on the hardware exp2 and
    reciprocal) against float64 torch.gelu: within one bf16 rounding (2^-8
    relative) plus 2e-6 absolute, over pre-activations in [-100, 100] and the
    cases where erf saturates."""
    x = _wide_inputs(512, -100.0, 100.0, seed=1)
    n = 256
    a, b, offs = _activation_probe([x], [torch.arange(n)], n, torch.bfloat16, cuda_device)
    c = mlp._grouped_gemm_ex(a, b, offs, mlp._EPILOGUES["gelu"], n, None, block, False)
    torch.cuda.synchronize()
    ref = torch.nn.functional.gelu(x.double())[:, None].expand(-1, n).numpy()
    got = c.double().cpu().numpy()
    bound = 2.0 ** -8 * 1.01 * np.abs(ref) + 2e-6
    bad = np.abs(got - ref) > bound
    assert not bad.any(), (x[np.nonzero(bad)[0][:5]], got[bad][:5], ref[bad][:5])


@pytest.mark.parametrize("block", [256, 128])
def test_swiglu_epilogue_accuracy_over_wide_range(cuda_device, block):
    """silu(gate) * up on the hardware exp2 and reciprocal against float64,
    within one bf16 rounding plus 2e-6 absolute, for gates in [-100, 100]
    (e^-gate overflows below -88: the result is then 0, silu's limit)."""
    g = _wide_inputs(512, -100.0, 100.0, seed=2)
    gen = torch.Generator().manual_seed(3)
    u = (torch.randn(512, generator=gen) * 3).to(torch.bfloat16)
    n = 256  # interleaved: columns 64q..64q+31 gate, 64q+32..64q+63 up of outputs 32q..32q+31
    cols = torch.arange(n)
    gate_cols = cols[(cols % 64) < 32]
    up_cols = cols[(cols % 64) >= 32]
    a, b, offs = _activation_probe([g, u], [gate_cols, up_cols], n, torch.bfloat16, cuda_device)
    c = mlp._grouped_gemm_ex(a, b, offs, mlp._EPILOGUES["swiglu"], n // 2, None, block, False)
    torch.cuda.synchronize()
    gd, ud = g.double(), u.double()
    ref = (gd * torch.sigmoid(gd) * ud)[:, None].expand(-1, n // 2).numpy()
    got = c.double().cpu().numpy()
    bound = 2.0 ** -8 * 1.01 * np.abs(ref) + 2e-6
    bad = np.abs(got - ref) > bound
    assert not bad.any(), (g[np.nonzero(bad)[0][:5]], got[bad][:5], ref[bad][:5])
