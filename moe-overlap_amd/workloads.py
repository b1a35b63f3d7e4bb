"""Synthetic routed-token workloads of the benchmark configurations (fixed seeds).

Counts come from the routing recipes; tensors are N(0,1) activations and
N(0, 1/K) expert weights.  Tensors are drawn with a torch Generator seeded on
the target device (so a GPU run does not generate hundreds of MB on the host);
the same seed on the same device type gives the same tensors.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

# Per-expert counts of the skewed-routing config at its pinned recipe
# (8192 tokens, top-2 over 16 experts, logits N(0,1) with torch seed 0 plus a
# per-expert bias ln(Zipf(1.2)) drawn with numpy default_rng(0)).
SKEWED_COUNTS = (0, 0, 586, 3269, 7, 4331, 0, 0, 0, 0, 0, 0, 0, 8191, 0, 0)


@dataclass
class GroupedGemmCase:
    name: str
    counts: torch.Tensor  # int32 [E] (CPU)
    k: int
    n: int
    a: Optional[torch.Tensor] = None  # [M, K]
    b: Optional[torch.Tensor] = None  # [E, K, N]

    @property
    def num_experts(self) -> int:
        return int(self.counts.numel())

    @property
    def m(self) -> int:
        return int(self.counts.sum())

    @property
    def flops(self) -> int:
        return 2 * self.m * self.k * self.n

    def algorithmic_bytes(self, elem_size: int = 2) -> int:
        """A read once, B of every non-empty expert read once, C written once."""
        nonempty = int((self.counts > 0).sum())
        return (self.m * self.k + nonempty * self.k * self.n + self.m * self.n) * elem_size


def skewed_counts_from_recipe(tokens: int = 8192, experts: int = 16, top_k: int = 2) -> torch.Tensor:
    """Routing counts of the skewed config, recomputed from its recipe."""
    gen = torch.Generator().manual_seed(0)
    logits = torch.randn(tokens, experts, generator=gen)
    zipf = np.random.default_rng(0).zipf(1.2, experts)
    bias = torch.from_numpy(np.log(zipf.astype(np.float64))).float()
    idx = torch.topk(logits + bias, top_k, dim=1).indices
    return torch.bincount(idx.flatten(), minlength=experts).to(torch.int32)


def topk_counts(tokens: int, experts: int, top_k: int, softmax: bool = False) -> torch.Tensor:
    """Counts of top-k routing on N(0,1) logits (torch seed 0)."""
    gen = torch.Generator().manual_seed(0)
    logits = torch.randn(tokens, experts, generator=gen)
    if softmax:
        logits = torch.softmax(logits, dim=-1)
    idx = torch.topk(logits, top_k, dim=1).indices
    return torch.bincount(idx.flatten(), minlength=experts).to(torch.int32)


def topk_routing(tokens: int, experts: int, top_k: int, softmax: bool = True):
    """(topk_idx int64 [T, k], topk_weight fp32 [T, k]) of top-k routing on
    N(0,1) logits (torch seed 0, CPU generator), weights the softmax
    probabilities of the chosen experts as the reference's router gives them
    (src/train_moe_baseline.py:316-317).  Same draw as topk_counts."""
    gen = torch.Generator().manual_seed(0)
    logits = torch.randn(tokens, experts, generator=gen)
    probs = torch.softmax(logits, dim=-1) if softmax else logits
    weight, idx = torch.topk(probs, top_k, dim=1)
    return idx, weight.float()


@dataclass
class ExpertMlpCase:
    """The benchmark's expert-MLP configuration: T tokens routed top-k over E experts,
    hidden H, SwiGLU FFN of width F (gate|up 2F interleaved for the fused
    epilogue), weights N(0, 1/fan_in)."""

    tokens: int
    experts: int
    top_k: int
    hidden: int
    ffn: int
    x: Optional[torch.Tensor] = None  # [T, H]
    topk_idx: Optional[torch.Tensor] = None  # [T, k] int64
    topk_weight: Optional[torch.Tensor] = None  # [T, k] fp32
    w_gate: Optional[torch.Tensor] = None  # [E, H, F]
    w_up: Optional[torch.Tensor] = None  # [E, H, F]
    w2: Optional[torch.Tensor] = None  # [E, F, H]

    @property
    def flops(self) -> int:
        rows = int((self.topk_idx >= 0).sum())
        return 2 * rows * self.hidden * 2 * self.ffn + 2 * rows * self.ffn * self.hidden


def make_expert_mlp_case(tokens: int = 8192, experts: int = 16, top_k: int = 2,
                         hidden: int = 2048, ffn: int = 4096, device=None,
                         dtype: torch.dtype = torch.bfloat16, seed: int = 0) -> ExpertMlpCase:
    """Synthetic inputs of the expert-MLP configuration (defaults: 8192 tokens, top-2 of 16)."""
    case = ExpertMlpCase(tokens, experts, top_k, hidden, ffn)
    idx, w = topk_routing(tokens, experts, top_k)
    device = torch.device("cpu") if device is None else torch.device(device)
    case.topk_idx = idx.to(device)
    case.topk_weight = w.to(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    f32 = dict(generator=gen, device=device, dtype=torch.float32)
    case.x = torch.randn(tokens, hidden, **f32).to(dtype)
    case.w_gate = (torch.randn(experts, hidden, ffn, **f32) / math.sqrt(hidden)).to(dtype)
    case.w_up = (torch.randn(experts, hidden, ffn, **f32) / math.sqrt(hidden)).to(dtype)
    case.w2 = (torch.randn(experts, ffn, hidden, **f32) / math.sqrt(ffn)).to(dtype)
    return case


@dataclass
class Fp8Case:
    """The benchmark's fp8 configuration: per-token scaled e4m3 activations, per-output-
    channel scaled e4m3 expert weights stored [E, N, K] (K contiguous)."""

    counts: torch.Tensor  # int32 [E] (CPU)
    k: int
    n: int
    a: Optional[torch.Tensor] = None  # [M, K] float8_e4m3fn
    a_scale: Optional[torch.Tensor] = None  # [M] fp32
    b_nk: Optional[torch.Tensor] = None  # [E, N, K] float8_e4m3fn
    b_scale: Optional[torch.Tensor] = None  # [E, N] fp32
    a_ref: Optional[torch.Tensor] = None  # [M, K] fp32 before quantisation
    b_ref: Optional[torch.Tensor] = None  # [E, N, K] fp32 before quantisation

    @property
    def num_experts(self) -> int:
        return int(self.counts.numel())

    @property
    def m(self) -> int:
        return int(self.counts.sum())

    @property
    def flops(self) -> int:
        return 2 * self.m * self.k * self.n

    def algorithmic_bytes(self) -> int:
        """fp8 A and the non-empty experts' fp8 B read once, bf16 C written
        once, plus the fp32 scales (4M + 4 E_nonempty N)."""
        nonempty = int((self.counts > 0).sum())
        return (self.m * self.k + nonempty * self.k * self.n + 2 * self.m * self.n
                + 4 * self.m + 4 * nonempty * self.n)


def make_fp8_case(tokens: int = 4096, experts: int = 64, top_k: int = 6, k: int = 2048,
                  n: int = 1408, device=None, seed: int = 0, keep_reference: bool = False) -> Fp8Case:
    """Synthetic inputs of the fp8 configuration (defaults: 4096 tokens, top-6 of 64): counts of
    top-k routing on N(0,1) logits, X ~ N(0,1), W ~ N(0, 1/K), each quantised
    with scale = amax / 448 per token and per output channel."""
    counts = topk_counts(tokens, experts, top_k)
    case = Fp8Case(counts, k, n)
    device = torch.device("cpu") if device is None else torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(case.m, k, generator=gen, device=device, dtype=torch.float32)
    w = torch.randn(experts, n, k, generator=gen, device=device, dtype=torch.float32)
    w.mul_(1.0 / math.sqrt(k))

    def quant(t):
        amax = t.abs().amax(dim=-1, keepdim=True).clamp_min(1e-12)
        scale = amax / 448.0
        return (t / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn), scale.squeeze(-1)

    case.a, case.a_scale = quant(x)
    case.b_nk, case.b_scale = quant(w)
    if keep_reference:
        case.a_ref, case.b_ref = x, w
    return case


# The reference benchmark script's default problem (src/bench_triton_grouped_gemm.py:11-17,
# :36-42): 256 routed experts x 128 tokens each, hidden 7168, ffn 2048, uniform counts.
REFERENCE_BENCH = dict(experts=256, tokens_per_expert=128, k=7168, n=2048)


def uniform_case(experts: int, tokens_per_expert: int, k: int, n: int,
                 name: str = "uniform_custom") -> GroupedGemmCase:
    """Equal counts, as the reference benchmark's build_counts makes them (:36-42)."""
    return GroupedGemmCase(name, torch.full((experts,), tokens_per_expert, dtype=torch.int32), k, n)


def make_case(
    name: str,
    device: Optional[torch.device] = None,
    dtype: torch.dtype = torch.bfloat16,
    seed: int = 0,
    materialize: bool = True,
) -> GroupedGemmCase:
    """One of: cpu_plumbing (fp32, E=8), uniform (E=16, 512 rows each), skewed (16384 rows),
    reference_bench (the reference benchmark script's default: E=256 x 128 rows, K=7168,
    N=2048)."""
    if name == "reference_bench":
        case = uniform_case(name=name, **REFERENCE_BENCH)
    elif name == "cpu_plumbing":
        case = GroupedGemmCase(name, torch.full((8,), 128, dtype=torch.int32), 512, 1024)
    elif name == "uniform":
        case = GroupedGemmCase(name, torch.full((16,), 512, dtype=torch.int32), 2048, 4096)
    elif name == "skewed":
        case = GroupedGemmCase(name, torch.tensor(SKEWED_COUNTS, dtype=torch.int32), 2048, 4096)
    else:
        raise ValueError(f"unknown workload {name!r}")
    if materialize:
        fill_operands(case, device=device, dtype=dtype, seed=seed)
    return case


def fill_operands(case: GroupedGemmCase, device=None, dtype=torch.bfloat16, seed: int = 0) -> None:
    """a ~ N(0,1) [M, K], b ~ N(0, 1/K) [E, K, N], drawn in fp32 then cast (B one expert
    at a time, so no fp32 copy of a large weight tensor is ever whole)."""
    device = torch.device("cpu") if device is None else torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    a = torch.randn(case.m, case.k, generator=gen, device=device, dtype=torch.float32)
    case.a = a.to(dtype)
    del a
    case.b = torch.empty(case.num_experts, case.k, case.n, device=device, dtype=dtype)
    for e in range(case.num_experts):
        w = torch.randn(case.k, case.n, generator=gen, device=device, dtype=torch.float32)
        case.b[e] = w.mul_(1.0 / math.sqrt(case.k))
