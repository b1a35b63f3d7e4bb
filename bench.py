#!/usr/bin/env python3
"""Benchmark of the persistent expert-grouped GEMM on one MI355X.

A step is one ``persistent_grouped_gemm`` call (the full drop-in API: offsets
already on the device, output allocation, launch) over the benchmark metric's
workload: E=16 experts x 512 routed tokens, K=2048, N=4096, bf16 in, fp32
accumulate, bf16 out.  Inputs are synthetic (N(0,1) activations, N(0,1/K)
weights) and resident in HBM before the timed region.

Protocol:
1. ``--warmup`` untimed steps, then the clock is settled whatever ``--warmup``
   says: the card idles at a low clock and takes tens of milliseconds of work
   to reach its sustained clock, so steps run in windows of 10 (HIP events
   around each) until at least 50 ms of GPU time has passed and two
   consecutive windows' medians agree within 2% (``settle_*`` fields).
2. Exactly ``--steps`` steps between two device synchronisations: ``value`` is
   the algorithmic FLOPs (2*M*K*N) of those steps over that wall time.
   A HIP event pair on the launch stream brackets the same steps:
   ``roofline.achieved`` is the FLOPs over that GPU-side time per launch.
3. A pass of max(steps, 100) further back-to-back launches with HIP events
   around each batch of 10 gives the per-launch distribution
   (``kernel_ms_median`` / ``_min`` / ``_mean`` over the batches; the card's
   clock keeps drifting down under sustained load, so these read a little
   slower than the timed steps), and a pass of 50 more the kernel's own
   average shader clock (``clock``).
4. ``flushed``: 50 launches, each after a 512 MiB device write that evicts L2
   and the 256 MB MALL, HIP events around each launch only: the cache-cold
   time per launch with its own roofline fraction.

``--experts/--tokens-per-expert/--k/--n/--dtype`` (the reference benchmark
script's knobs; ``--num-routed-experts``, ``--hidden-size`` and
``--ffn-size`` are accepted as its names) time a uniform problem of that
shape instead, and ``--workload reference_bench`` the script's default (E=256
x 128 tokens, K=7168, N=2048).

Extra fields compare striped and atomic scheduling under uniform and skewed
routing, the reference's explicit 128x128 request, a cache-cold launch, the
per-expert torch loop on the GPU, the expert-MLP and fp8 configs, and the
per-expert torch loop on the host's cores (``cpu_baseline``).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "moe-overlap_amd"))
sys.path.insert(0, str(REPO))

METRIC = "grouped GEMM TFLOP/s + % bf16 MFMA peak, E=16 512 tok/expert K2048 N4096"
PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0
PEAK_FP8_TFLOPS = 5033.2  # MI355X dense fp8 MFMA
# (K per stage, LDS stages, waves) of the compiled 16-bit tiles bench.py names.
_TILE_CONFIG = {(256, 256): (32, 4, 8), (128, 512): (32, 3, 8), (128, 128): (64, 4, 4)}


def kernel_name(tile, dtype="bf16"):
    """The rocprofv3 name of the 16-bit kernel instance for `tile`."""
    cfg = _TILE_CONFIG.get(tuple(tile))
    if cfg is None:
        return "grouped_gemm_kernel"
    t = "Bf16" if dtype == "bf16" else "F16"
    return f"grouped_gemm_kernel<{tile[0]},{tile[1]},{cfg[0]},{cfg[1]},{cfg[2]},{t},0>"


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", default="uniform",
                   choices=["uniform", "skewed", "cpu_plumbing", "reference_bench", "expert_mlp", "fp8"],
                   help="uniform (the metric's config), skewed, cpu_plumbing, reference_bench (the "
                        "reference benchmark script's default problem); expert_mlp and fp8 "
                        "time the benchmark expert-MLP forward / fp8 GEMM configs instead")
    # The reference benchmark script's problem knobs (src/bench_triton_grouped_gemm.py:11-27):
    # a uniform problem, each unset one taken from the --workload's shape.
    p.add_argument("--experts", "--num-routed-experts", dest="experts", type=int, default=None)
    p.add_argument("--tokens-per-expert", type=int, default=None)
    p.add_argument("--k", "--hidden-size", dest="k", type=int, default=None)
    p.add_argument("--n", "--ffn-size", dest="n", type=int, default=None)
    p.add_argument("--dtype", default="bf16", choices=["bf16", "fp16"])
    # atomic by default, as the reference's API (persistent_grouped_gemm's use_atomic_queue=True,
    # src/triton_grouped_gemm.py:334; its benchmark script makes it opt-in, :28-32); the
    # comparison below times both schedules either way
    p.add_argument("--mode", default="atomic", choices=["atomic", "striped"])
    # The requested tile (the reference's block_m/block_n, default 128x128): it sets the queue
    # whose length the work counter reports; the kernel computes with --kernel-tile.
    p.add_argument("--block-m", type=int, default=128)
    p.add_argument("--block-n", type=int, default=128)
    p.add_argument("--kernel-tile", default=None,
                   help="compiled tile BMxBN to compute with (default: the library's choice)")
    p.add_argument("--num-sms", type=int, default=None)
    p.add_argument("--no-compare", action="store_true", help="skip the schedule/routing comparison")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="CPU baseline budget (cfg 1 and the fp32-upcast metric config together)")
    p.add_argument("--profile-only", action="store_true",
                   help="only the warmup, settle and timed steps (for rocprofv3 runs)")
    p.add_argument("--no-settle", action="store_true", help="skip the clock-settling phase")
    p.add_argument("--vendor-bmm", action="store_true",
                   help="with --profile-only and equal counts: run hipBLASLt's batched GEMM "
                        "(torch.bmm) on the same operands instead of the grouped GEMM, for "
                        "counter comparisons (analysis only)")
    # The benchmark's operands are random; the others keep every byte moved and every MFMA
    # issued but change the data, which shows how the card's power limit sets its clock.
    p.add_argument("--operands", default="random", choices=["random", "zero_a", "zero_b", "constant"],
                   help="operand data of the headline workload (analysis only; the metric uses random)")
    p.add_argument("--calibrate-copy-mib", type=int, default=0,
                   help="instead of the GEMM, run --steps plain device copies of this many MiB "
                        "(reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return p.parse_args()


def progress(msg):
    """A progress line on stderr (the JSON result line goes to stdout)."""
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def median(xs):
    ys = sorted(xs)
    if not ys:
        return float("nan")
    h = len(ys) // 2
    return ys[h] if len(ys) % 2 else 0.5 * (ys[h - 1] + ys[h])


def event_times_ms(fn, iters, flush=None):
    """Per-launch durations (ms) from HIP events on the current stream."""
    import torch

    times = []
    for _ in range(iters):
        if flush is not None:
            flush()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        times.append((s, e))
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in times]


def batched_times_ms(fn, launches=100, batch=10):
    """Per-launch durations (ms) of back-to-back launches: HIP events around
    each batch of `batch` launches on the current stream, divided by `batch`.
    An event pair around every single launch would also time the dispatch of
    each launch, which back-to-back launches overlap with the previous one."""
    import torch

    pairs = []
    for _ in range(max(1, launches // batch)):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(batch):
            fn()
        e.record()
        pairs.append((s, e))
    torch.cuda.synchronize()
    return [s.elapsed_time(e) / batch for s, e in pairs]


def settle_clock(fn, min_ms=50.0, window=10, rel=0.02, max_s=5.0):
    """Runs fn in windows of `window` launches until at least `min_ms` of GPU
    time has passed and two consecutive windows' median launch times agree
    within `rel` (the clock has stopped ramping), or `max_s` of wall time."""
    t0 = time.perf_counter()
    total_ms, launches, prev, last = 0.0, 0, None, None
    while True:
        ts = event_times_ms(fn, window)
        total_ms += sum(ts)
        launches += window
        last = median(ts)
        done = total_ms >= min_ms and prev is not None and abs(last - prev) <= rel * last
        if done or time.perf_counter() - t0 > max_s:
            return {"settle_launches": launches, "settle_ms": round(total_ms, 2),
                    "settle_window_ms_median": round(last, 5), "settled": bool(done)}
        prev = last


def clock_pass(fn, launches=50):
    """s_memtime ticks per microsecond over `launches` back-to-back launches
    of fn (libmgg's clock probe: the ticks eight workgroups live, over the
    per-launch time from HIP events around the pass).  On gfx950 s_memtime
    does not count shader clocks (an MFMA-only probe at 97.6% of peak read
    1244), so this is only a relative reading between runs of one box, not
    the clock; rocprofv3's GRBM_GUI_ACTIVE gives cycle counts.  A pass of
    its own, so the probe stays out of the other timings."""
    import torch

    import mgg_native as nat

    probe = torch.zeros(2, dtype=torch.int64, device="cuda")
    lib = nat.lib()
    settle_clock(fn)  # the card drops its clock in any idle gap before this pass
    nat.check(lib.mgg_debug_set_clock_probe(probe.data_ptr()))
    try:
        ms = sum(batched_times_ms(fn, launches=launches, batch=launches))
    finally:
        nat.check(lib.mgg_debug_set_clock_probe(None))
    ticks, readers = probe.tolist()
    mhz = ticks / readers / (ms * 1e3) if readers > 0 and ms > 0 else None
    return {"s_memtime_ticks_per_us": round(mhz, 1) if mhz else None, "launches": launches,
            "ms_per_launch": round(ms, 5),
            "source": "s_memtime ticks of a workgroup's lifetime / HIP-event time per launch "
                      "(a relative reading: s_memtime is not the shader clock on gfx950)"}


PROFILE_SUMMARY = REPO / "profiles" / "grouped_gemm_256x256_bf16_uniform.md"
FP8_PROFILE_SUMMARY = REPO / "profiles" / "grouped_gemm_fp8_cfg5.md"
REFBENCH_PROFILE_SUMMARY = REPO / "profiles" / "grouped_gemm_128x512_bf16_reference_bench.md"


def recorded_traffic(mode, workload, kernel_tile):
    """HBM bytes per launch from a committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
    (calibrated against a plain copy), when one covers this configuration; else None."""
    if workload == "uniform" and kernel_tile == (256, 256):
        path, key = PROFILE_SUMMARY, f"traffic_bytes_per_launch_{mode}:"
    elif workload == "reference_bench" and kernel_tile == (128, 512):
        path, key = REFBENCH_PROFILE_SUMMARY, f"traffic_bytes_per_launch_reference_bench_{mode}:"
    elif workload == "fp8" and kernel_tile in ((256, 256), (256, 128), (192, 128)):
        path, key = FP8_PROFILE_SUMMARY, f"traffic_bytes_per_launch_fp8_{kernel_tile[0]}x{kernel_tile[1]}_{mode}:"
    else:
        return None
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith(key):
            return int(line.split(":", 1)[1])
    return None


def expert_mlp_summary(dev, steps: int = 20):
    """The benchmark expert-MLP config (8192 tokens top-2 of 16, H 2048, SwiGLU
    F 4096): whole forward (layout, up GEMM with the gather fused + SwiGLU,
    down GEMM, combine) and each launch alone, from HIP events on the current
    stream; also the separate gather and plain up GEMM the fused launch
    replaces."""
    import torch

    import expert_mlp as mlp
    import workloads

    case = workloads.make_expert_mlp_case(device=dev)
    w1 = mlp.interleave_gate_up(case.w_gate, case.w_up)
    case.w_gate = case.w_up = None
    fwd = lambda: mlp.expert_mlp_forward(case.x, case.topk_idx, case.topk_weight, w1, case.w2,
                                         "swiglu")
    settle_clock(fwd)
    t_fwd = median(event_times_ms(fwd, steps))
    lay = mlp.dispatch_layout(case.topk_idx, case.experts)
    xp = mlp.permute_tokens(case.x, lay)
    h = mlp._grouped_gemm_ex(xp, w1, lay.offsets, mlp._EPILOGUES["swiglu"], case.ffn, None, 256, True)
    y = mlp._grouped_gemm_ex(h, case.w2, lay.offsets, mlp._EPILOGUES["none"], case.hidden, None, 256, True)
    parts = {
        "dispatch_layout": lambda: mlp.dispatch_layout(case.topk_idx, case.experts),
        "up_gemm_gathered_swiglu": lambda: mlp._grouped_gemm_gathered(
            case.x, lay, w1, mlp._EPILOGUES["swiglu"], case.ffn, None, True),
        "gather_unfused": lambda: mlp.permute_tokens(case.x, lay),
        "up_gemm_swiglu_unfused": lambda: mlp._grouped_gemm_ex(
            xp, w1, lay.offsets, mlp._EPILOGUES["swiglu"], case.ffn, None, 256, True),
        "down_gemm": lambda: mlp._grouped_gemm_ex(h, case.w2, lay.offsets, mlp._EPILOGUES["none"],
                                                 case.hidden, None, 256, True),
        "combine": lambda: mlp.combine_tokens(y, lay, case.topk_weight),
    }
    rows = case.tokens * case.top_k
    up_flops = 2 * rows * case.hidden * 2 * case.ffn
    down_flops = 2 * rows * case.ffn * case.hidden
    out = {"config": f"T={case.tokens} top-{case.top_k} of E={case.experts}, H={case.hidden}, "
                     f"SwiGLU F={case.ffn}, bf16",
           "forward_ms_median": round(t_fwd, 4),
           "forward_tflops": round(case.flops / (t_fwd * 1e-3) / 1e12, 1),
           "launch_ms_median": {}}
    # Interleaved rounds, so a clock that drifts during the measurement
    # weighs on every launch alike.
    times = {name: [] for name in parts}
    for name, fn in parts.items():
        event_times_ms(fn, 10)
    for rnd in range(4):
        order = list(parts.items()) if rnd % 2 == 0 else list(parts.items())[::-1]
        for name, fn in order:
            times[name] += event_times_ms(fn, max(steps // 4, 5))
    for name in parts:
        out["launch_ms_median"][name] = round(median(times[name]), 4)
    lm = out["launch_ms_median"]
    out["up_gemm_tflops"] = round(up_flops / (lm["up_gemm_gathered_swiglu"] * 1e-3) / 1e12, 1)
    out["down_gemm_tflops"] = round(down_flops / (lm["down_gemm"] * 1e-3) / 1e12, 1)
    del case, w1, lay, xp, h, y
    torch.cuda.empty_cache()
    return out


def fp8_summary(dev, steps: int = 40):
    """The benchmark fp8 config (E=64, M=24576, K=2048, N=1408, e4m3 with
    per-token x per-channel scales, bf16 out), HBM-bound by its algorithmic
    bytes: each kernel tile and schedule, kernel time from HIP events."""
    import grouped_gemm as gg
    import workloads

    case = workloads.make_fp8_case(device=dev)
    offs = gg.expert_offsets_from_recv_counts(case.counts, device=dev)
    b_kn = case.b_nk.transpose(1, 2)
    t_bytes = case.algorithmic_bytes()
    t_flop_bound = case.flops / (PEAK_FP8_TFLOPS * 1e12)
    t_hbm_bound = t_bytes / (PEAK_HBM_GBPS * 1e9)
    out = {"config": f"E={case.num_experts}, M={case.m}, K={case.k}, N={case.n}, e4m3 in, bf16 out",
           "algorithmic_bytes": t_bytes, "t_bound_us": round(max(t_flop_bound, t_hbm_bound) * 1e6, 2),
           "runs": {}}
    out["default_tile"] = "{}x{}".format(*gg._default_fp8_kernel_tile(case.m, case.num_experts))
    best = None
    for tile in ((256, 256), (256, 128), (192, 128), (128, 128)):
        for mode in ("striped", "atomic"):
            fn = lambda: gg.persistent_grouped_gemm(case.a, b_kn, offs, kernel_tile=tile,
                                                    use_atomic_queue=mode == "atomic",
                                                    a_scale=case.a_scale, b_scale=case.b_scale)
            settle_clock(fn)
            t = median(event_times_ms(fn, steps))
            r = {"kernel_ms_median": round(t, 4),
                 "tflops": round(case.flops / (t * 1e-3) / 1e12, 1),
                 "hbm_gbps_at_algorithmic_bytes": round(t_bytes / (t * 1e-3) / 1e9, 1)}
            name = f"{tile[0]}x{tile[1]}_{mode}"
            out["runs"][name] = r
            if best is None or t < best[1]:
                best = (name, t)
    out["best"] = best[0]
    out["best_frac_of_hbm_roofline"] = round(t_hbm_bound * 1e3 / best[1], 4)
    out["best_pct_fp8_peak"] = round(100 * case.flops / (best[1] * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 2)
    return out


def overlap_summary(case, offs, dev, iters: int = 60):
    """What one GPU shows of the multi-GPU overlap design, per launch over a pipeline of
    `iters` iterations timed by the host clock: (1) the GEMM with CUs held back for
    communication kernels (num_sms < 256, the analogue of the reference's DeepEP SM
    reservation); (2) each iteration's GEMM on one created stream while a copy of the
    micro-batch's tokens (the local memory traffic of a dispatch, 2 x 32 MiB) runs on
    another, joined at the iteration's end, against the two back to back on one stream.
    Both streams are created streams: the legacy default stream would serialise them."""
    import torch

    import grouped_gemm as gg

    src = torch.empty_like(case.a)
    dst = torch.empty_like(case.a)
    s_main = torch.cuda.Stream(device=dev)
    s_side = torch.cuda.Stream(device=dev)

    def copies():
        dst.copy_(src)
        src.copy_(dst)

    def pipeline(sms, mode, n):
        for _ in range(n):
            if mode != "copy":
                with torch.cuda.stream(s_main):
                    gg.persistent_grouped_gemm(case.a, case.b, offs, num_sms=sms)
            if mode == "serial":
                with torch.cuda.stream(s_main):
                    copies()
            elif mode in ("overlapped", "copy"):
                with torch.cuda.stream(s_side):
                    copies()
                s_main.wait_stream(s_side)
                s_side.wait_stream(s_main)

    def per_iter_us(sms, mode):
        pipeline(sms, mode, 20)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        pipeline(sms, mode, iters)
        torch.cuda.synchronize()
        return round((time.perf_counter() - t0) / iters * 1e6, 1)

    out = {"unit": "µs per iteration"}
    for sms in (256, 240, 224, 192):
        out[f"gemm_alone_{sms}"] = per_iter_us(sms, "gemm")
    for sms in (256, 224):
        out[f"serial_{sms}"] = per_iter_us(sms, "serial")
        out[f"overlapped_{sms}"] = per_iter_us(sms, "overlapped")
    out["copy_alone"] = per_iter_us(0, "copy")
    out["note"] = ("copy = 2 x 32 MiB device copies; overlapped = GEMM and copy on two created "
                   "streams of default priority, joined every iteration")
    return out


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or platform.machine()


def cpu_baseline(case, budget_s):
    """The reference's comparison loop, a per-expert torch matmul over each
    expert's rows (src/triton_grouped_gemm.py:446-457, restated as
    grouped_gemm.reference_grouped_gemm), on the host's cores in fp32: the
    CPU-plumbing config (E=8, 128 tokens/expert, K=512, N=1024; >= 20 timed
    iterations, median) and the metric's config with its bf16 inputs upcast
    to fp32 (>= 3 timed iterations, median).  Threads: torch's default, which
    follows OMP_NUM_THREADS (the GPU box's CPU share)."""
    import torch

    import grouped_gemm as gg
    import workloads

    threads = torch.get_num_threads()

    def timed(a, b, offs, min_iters, budget):
        gg.reference_grouped_gemm(a, b, offs)  # warm-up (allocator, thread pool)
        ts = []
        t_end = time.perf_counter() + budget
        while len(ts) < min_iters or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            gg.reference_grouped_gemm(a, b, offs)
            ts.append(time.perf_counter() - t0)
        return ts

    small = workloads.make_case("cpu_plumbing", device="cpu", dtype=torch.float32)
    small_offs = gg.expert_offsets_from_recv_counts(small.counts)
    ts_small = timed(small.a, small.b, small_offs, 20, 0.2 * budget_s)
    a32 = case.a.float().cpu()
    b32 = case.b.float().cpu()
    offs = gg.expert_offsets_from_recv_counts(case.counts)
    ts_big = timed(a32, b32, offs, 3, 0.6 * budget_s)
    t_big = median(ts_big)
    t_small = median(ts_small)
    return {
        "value": round(case.flops / t_big / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": int(threads),
        "kind": "port",
        "sample": f"{case.name} config (E={case.num_experts}, M={case.m}, K={case.k}, N={case.n}) with "
                  f"its bf16 inputs upcast to fp32: per-expert torch matmul loop, median of "
                  f"{len(ts_big)} iterations of {t_big * 1e3:.1f} ms",
        "cpu_plumbing": {"config": f"E={small.num_experts}, M={small.m}, K={small.k}, N={small.n}, fp32",
                         "ms_median": round(t_small * 1e3, 4), "iterations": len(ts_small),
                         "tflops": round(small.flops / t_small / 1e12, 5)},
        "threads": int(threads),
        "host_cpus": os.cpu_count(),
        "cpu_model": _cpu_model(),
        "torch_version": torch.__version__,
    }


FLUSH_BYTES = 512 * 1024 * 1024  # > the 256 MB MALL + 8 x 4 MB L2


def flushed_times_ms(step, dev, launches=50):
    """Per-launch durations (ms) of `launches` launches, each after a 512 MiB
    device write that evicts L2 and the MALL (HIP events around the launch
    only)."""
    import torch

    scratch = torch.empty(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)
    fill = lambda: scratch.fill_(1.0)
    event_times_ms(step, 5, flush=fill)
    t = event_times_ms(step, launches, flush=fill)
    del scratch
    return t


def reference_bench_summary(dev, dtype, num_sms=None, steps=30):
    """The reference benchmark script's default problem (E=256 x 128 tokens,
    K=7168, N=2048, uniform counts; src/bench_triton_grouped_gemm.py:11-17):
    7.5 GB of weights make it HBM-bound (119 FLOP/B against the bf16 ridge of
    315).  Warm and flushed kernel times per schedule."""
    import torch

    import grouped_gemm as gg
    import workloads

    case = workloads.make_case("reference_bench", device=dev, dtype=dtype)
    offs = gg.expert_offsets_from_recv_counts(case.counts, device=dev)
    nbytes = case.algorithmic_bytes()
    t_hbm = nbytes / (PEAK_HBM_GBPS * 1e9) * 1e3
    out = {"config": f"E={case.num_experts} x {int(case.counts[0])} tokens, K={case.k}, N={case.n}, "
                     f"{'bf16' if dtype == torch.bfloat16 else 'fp16'}",
           "algorithmic_flops": case.flops, "algorithmic_bytes": nbytes,
           "t_hbm_bound_ms": round(t_hbm, 4), "runs": {}}
    for mode in ("atomic", "striped"):
        fn = lambda: gg.persistent_grouped_gemm(case.a, case.b, offs, num_sms=num_sms,
                                                use_atomic_queue=mode == "atomic")
        settle_clock(fn)
        t = median(event_times_ms(fn, steps))
        tc = median(flushed_times_ms(fn, dev, launches=20))
        out["runs"][mode] = {"kernel_ms_median": round(t, 4), "tflops": round(case.flops / (t * 1e-3) / 1e12, 1),
                             "hbm_gbps_at_algorithmic_bytes": round(nbytes / (t * 1e-3) / 1e9, 1),
                             "frac_of_hbm_roofline": round(t_hbm / t, 4),
                             "flushed_kernel_ms_median": round(tc, 4),
                             "flushed_frac_of_hbm_roofline": round(t_hbm / tc, 4)}
    # The vendor library's batched GEMM (torch.bmm -> hipBLASLt) on the same
    # operands (equal counts make the problem one batched GEMM), for reference.
    a3 = case.a.view(case.num_experts, int(case.counts[0]), case.k)
    bmm = lambda: torch.bmm(a3, case.b)
    settle_clock(bmm)
    tb = median(event_times_ms(bmm, steps))
    out["hipblaslt_bmm"] = {"kernel_ms_median": round(tb, 4),
                            "frac_of_hbm_roofline": round(t_hbm / tb, 4)}
    out["kernel_tile"] = "{}x{}".format(*gg._default_kernel_tile(
        case.m, case.num_experts, case.n, num_sms or gg._cu_count(dev.index or 0)))
    c = gg.persistent_grouped_gemm(case.a, case.b, offs, num_sms=num_sms)
    rows = torch.arange(0, case.m, 509, device=dev)
    e_of = torch.div(rows, int(case.counts[0]), rounding_mode="floor")
    ref = torch.bmm(case.a[rows].float().unsqueeze(1), case.b[e_of].float()).squeeze(1)
    out["sampled_rows"] = int(rows.numel())
    out["max_abs_diff_vs_fp32_sampled"] = round((c[rows].float() - ref).abs().max().item(), 6)
    out["tolerance"] = round(2e-2 * math.sqrt(case.k / 512), 6)
    del case, c, ref
    torch.cuda.empty_cache()
    return out


def _kernel_tile_arg(text):
    if text is None:
        return None
    m, n = text.lower().split("x")
    return int(m), int(n)


def run_protocol(step, args, flops):
    """Warmup, clock settling, the timed steps (wall clock) and the event
    pass; returns the timing fields of the result line."""
    import torch

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    settle = {"settle_launches": 0, "settle_ms": 0.0} if args.no_settle else settle_clock(step)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # The timed steps' launches back to back on the stream, from the GPU's clock.
    out = {"wall_s": wall, "timed_ms_per_launch": ev0.elapsed_time(ev1) / args.steps, **settle}
    if args.profile_only:
        return out
    kernel_ms = batched_times_ms(step, launches=max(args.steps, 100), batch=10)
    out.update(kernel_ms=kernel_ms, clock=clock_pass(step))
    return out


def secondary_main(args, dev):
    """--workload expert_mlp | fp8: time one step of that config (the same
    warmup / settle / timed-steps / event protocol as the headline) and print
    its line."""
    import expert_mlp as mlp
    import grouped_gemm as gg
    import workloads

    if args.workload == "expert_mlp":
        case = workloads.make_expert_mlp_case(device=dev)
        w1 = mlp.interleave_gate_up(case.w_gate, case.w_up)
        case.w_gate = case.w_up = None
        step = lambda: mlp.expert_mlp_forward(case.x, case.topk_idx, case.topk_weight, w1, case.w2,
                                              "swiglu", num_sms=args.num_sms,
                                              use_atomic_queue=args.mode == "atomic")
        flops, nbytes, bound, peak, dtype = case.flops, None, "mfma", PEAK_BF16_TFLOPS, "bf16"
        metric = "expert-MLP forward TFLOP/s (SwiGLU, T=8192 top-2 of 16, H2048 F4096)"
        tile = (256, 256)
        kernel = "grouped_gemm_kernel<256,256,32,4,8,Bf16,2> (up, SwiGLU) and <256,256,32,4,8,Bf16,0> (down)"
        config = {"workload": f"expert_mlp: T={case.tokens}, top-{case.top_k} of E={case.experts}, "
                              f"H={case.hidden}, F={case.ffn}, SwiGLU", "mode": args.mode}
    else:
        case = workloads.make_fp8_case(device=dev)
        offs = gg.expert_offsets_from_recv_counts(case.counts, device=dev)
        b_kn = case.b_nk.transpose(1, 2)
        tile = _kernel_tile_arg(args.kernel_tile) or gg._default_fp8_kernel_tile(case.m, case.num_experts)
        step = lambda: gg.persistent_grouped_gemm(case.a, b_kn, offs, num_sms=args.num_sms,
                                                  block_m=args.block_m, block_n=args.block_n,
                                                  kernel_tile=tile,
                                                  use_atomic_queue=args.mode == "atomic",
                                                  a_scale=case.a_scale, b_scale=case.b_scale)
        flops, nbytes, bound, peak, dtype = case.flops, case.algorithmic_bytes(), "hbm", PEAK_HBM_GBPS, "fp8_e4m3"
        metric = "fp8 grouped GEMM TFLOP/s, E=64 M=24576 K2048 N1408 (per-token x per-channel scales)"
        config = {"workload": f"fp8: E={case.num_experts}, M={case.m}, K={case.k}, N={case.n}",
                  "mode": args.mode, "kernel_tile": f"{tile[0]}x{tile[1]}"}
        stages = 2 if tile == (256, 256) else (4 if tile[0] == 128 else 3)
        kernel = f"grouped_gemm_kernel<{tile[0]},{tile[1]},128,{stages},8,Fp8,0>"
    r = run_protocol(step, args, flops)
    wall = r["wall_s"]
    if args.profile_only:
        print(json.dumps({"profile_only": True, "workload": args.workload,
                          "ms_per_step": wall / args.steps * 1e3,
                          "settle_launches": r["settle_launches"]}))
        return
    k_med = median(r["kernel_ms"])
    k_timed = r["timed_ms_per_launch"]
    value = flops * args.steps / wall / 1e12
    if bound == "hbm":
        achieved, unit = nbytes / (k_timed * 1e-3) / 1e9, "GB/s"
    else:
        achieved, unit = flops / (k_timed * 1e-3) / 1e12, "TFLOP/s"
    print(json.dumps({
        "metric": metric, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall / args.steps * 1e3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic (benchmark recipe, random init)", "config": config,
        "settle_launches": r["settle_launches"], "settle_ms": r["settle_ms"],
        "kernel_ms_timed_mean": round(k_timed, 5),
        "kernel_ms_median": round(k_med, 5), "kernel_ms_min": round(min(r["kernel_ms"]), 5),
        "kernel_ms_mean": round(sum(r["kernel_ms"]) / len(r["kernel_ms"]), 5),
        "clock": r["clock"],
        "roofline": {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 4),
                     "traffic": recorded_traffic(args.mode, args.workload, tile),
                     "kernel": kernel,
                     "algorithmic_flops_per_step": flops, "algorithmic_bytes_per_step": nbytes},
    }), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the grouped GEMM shards by expert across GPUs; one GPU's share is what runs here).",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import grouped_gemm as gg
    import workloads

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.calibrate_copy_mib:
        n = args.calibrate_copy_mib * 1024 * 1024 // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": n * 4, "copies": args.warmup + args.steps}))
        return
    if args.workload in ("expert_mlp", "fp8"):
        secondary_main(args, dev)
        return
    dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    shape_flags = (args.experts, args.tokens_per_expert, args.k, args.n)
    if any(v is not None for v in shape_flags):
        base = workloads.make_case(args.workload, materialize=False)
        if args.workload not in ("uniform", "reference_bench", "cpu_plumbing"):
            print("--experts/--tokens-per-expert/--k/--n make a uniform problem: use them with "
                  "--workload uniform or reference_bench", file=sys.stderr)
            sys.exit(2)
        case = workloads.uniform_case(args.experts or base.num_experts,
                                      args.tokens_per_expert or int(base.counts[0]),
                                      args.k or base.k, args.n or base.n)
        workloads.fill_operands(case, device=dev, dtype=dtype)
    else:
        case = workloads.make_case(args.workload, device=dev, dtype=dtype)
    is_metric_config = (case.name == "uniform" and dtype == torch.bfloat16)
    if args.operands == "zero_a":
        case.a.zero_()
    elif args.operands == "zero_b":
        case.b.zero_()
    elif args.operands == "constant":
        case.a.fill_(1.0)
        case.b.fill_(1.0 / 64)
    offs = gg.expert_offsets_from_recv_counts(case.counts, device=dev)
    atomic = args.mode == "atomic"
    kernel_tile = (_kernel_tile_arg(args.kernel_tile)
                   or gg._default_kernel_tile(case.m, case.num_experts, case.n,
                                              args.num_sms or gg._cu_count(0)))
    kw = dict(num_sms=args.num_sms, block_m=args.block_m, block_n=args.block_n,
              use_atomic_queue=atomic, kernel_tile=kernel_tile)

    def step():
        return gg.persistent_grouped_gemm(case.a, case.b, offs, **kw)

    if args.vendor_bmm:
        counts_l = case.counts.tolist()
        if not args.profile_only or len(set(counts_l)) != 1 or counts_l[0] <= 0:
            print("--vendor-bmm needs --profile-only and equal, non-zero counts", file=sys.stderr)
            sys.exit(2)
        a3 = case.a.view(case.num_experts, counts_l[0], case.k)

        def step():  # noqa: F811 (the vendor library's kernel on the same operands)
            return torch.bmm(a3, case.b)

    flops = case.flops
    nbytes = case.algorithmic_bytes()
    # MFMA-bound when the problem's FLOP per algorithmic byte is above the
    # bf16/fp16 ridge (peak FLOP/s over HBM bytes/s), else HBM-bound.
    hbm_bound = flops / nbytes < PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBPS * 1e9)
    progress(f"headline {case.name} E={case.num_experts} M={case.m} K={case.k} N={case.n} {args.dtype} "
             f"{args.mode}: warmup, settle, {args.steps} timed steps")
    r = run_protocol(step, args, flops)
    wall = r["wall_s"]
    if args.profile_only:
        print(json.dumps({"profile_only": True, "ms_per_step": wall / args.steps * 1e3,
                          "settle_launches": r["settle_launches"]}))
        return
    kernel_ms = r["kernel_ms"]
    value = flops * args.steps / wall / 1e12
    k_med = median(kernel_ms)
    k_mean = sum(kernel_ms) / len(kernel_ms)
    k_timed = r["timed_ms_per_launch"]
    progress(f"timed {k_timed * 1e3:.1f} us per launch; flushed pass")
    flushed = flushed_times_ms(step, dev)
    k_flushed = median(flushed)

    def roof(ms):
        if hbm_bound:
            return nbytes / (ms * 1e-3) / 1e9, PEAK_HBM_GBPS, "GB/s"
        return flops / (ms * 1e-3) / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s"

    achieved, peak, roof_unit = roof(k_timed)
    achieved_fl, _, _ = roof(k_flushed)

    # Correctness of the timed configuration against an fp32 torch loop
    # (every row up to 64 Mi output elements, else a row sample).
    c = step()
    if case.m * case.n <= 64 * 2 ** 20:
        ref = gg.reference_grouped_gemm(case.a.float(), case.b.float(), offs)
        max_abs = (c.float() - ref).abs().max().item()
    else:
        rows = torch.arange(0, case.m, 509, device=dev)
        bounds = torch.cumsum(case.counts, 0).to(dev)
        e_of = torch.searchsorted(bounds, rows, right=True)
        ref = torch.bmm(case.a[rows].float().unsqueeze(1), case.b[e_of].float()).squeeze(1)
        max_abs = (c[rows].float() - ref).abs().max().item()
    del ref
    tolerance = 2e-2 * math.sqrt(max(case.k, 512) / 512)

    extra = {}
    if not args.no_compare:
        # The reference's own call (its benchmark passes block_m = block_n = 128 explicitly,
        # src/bench_triton_grouped_gemm.py:19-20, :83-91) against the library default.
        legs = {}
        for name, extra_kw in (("default_call", {}),
                               ("explicit_128x128", dict(block_m=128, block_n=128)),
                               ("kernel_tile_128x128", dict(kernel_tile=(128, 128)))):
            fn = lambda: gg.persistent_grouped_gemm(case.a, case.b, offs, use_atomic_queue=atomic,
                                                    **extra_kw)
            settle_clock(fn)
            t = median(event_times_ms(fn, 50))
            legs[name] = {"kernel_ms_median": round(t, 5),
                          "tflops": round(flops / (t * 1e-3) / 1e12, 1)}
        extra["reference_calls"] = legs
        progress("expert MLP leg")
        extra["expert_mlp"] = expert_mlp_summary(dev)
        progress("fp8 leg")
        extra["fp8"] = fp8_summary(dev)
        progress("schedules leg")
        sched = {}
        for wl in ("uniform", "skewed"):
            cs = case if (wl == case.name and is_metric_config) else workloads.make_case(wl, device=dev)
            o = gg.expert_offsets_from_recv_counts(cs.counts, device=dev)
            for mode in ("striped", "atomic"):
                fn = lambda: gg.persistent_grouped_gemm(
                    cs.a, cs.b, o, num_sms=args.num_sms, kernel_tile=kernel_tile,
                    use_atomic_queue=(mode == "atomic"))
                settle_clock(fn)
                t = event_times_ms(fn, 50)
                sched[f"{wl}_{mode}"] = {
                    "kernel_ms_median": round(median(t), 4), "kernel_ms_min": round(min(t), 4),
                    "tflops": round(cs.flops / (median(t) * 1e-3) / 1e12, 1)}
            if cs is not case:
                del cs
        extra["schedules"] = sched
        # The reference API's per-expert torch loop on the GPU (hipBLASLt GEMMs).
        loop = lambda: gg.reference_grouped_gemm(case.a, case.b, offs)
        event_times_ms(loop, 3)
        tl = event_times_ms(loop, 10)
        extra["torch_loop_gpu_ms_median"] = round(median(tl), 4)
        extra["torch_loop_gpu_tflops"] = round(flops / (median(tl) * 1e-3) / 1e12, 1)
        counts_l = case.counts.tolist()
        if len(set(counts_l)) == 1 and counts_l[0] > 0:
            # Equal counts make the problem one batched GEMM: the vendor library's batched
            # kernel (torch.bmm -> hipBLASLt) on the same operands, for reference.
            e, c_e = len(counts_l), counts_l[0]
            a3 = case.a[: e * c_e].view(e, c_e, case.k)
            bmm = lambda: torch.bmm(a3, case.b)
            settle_clock(bmm)
            tb = event_times_ms(bmm, 50)
            extra["hipblaslt_bmm_ms_median"] = round(median(tb), 4)
            extra["hipblaslt_bmm_tflops"] = round(flops / (median(tb) * 1e-3) / 1e12, 1)
        # N not a multiple of 8 is read and written in place: N = 4092 and the
        # odd N = 4095 (its own kernel instance) against N = 4096 on the
        # metric's other dimensions, timed in rotating batches so a drifting
        # clock weighs on all alike.
        progress("odd-N leg")
        ns = (4096, 4092, 4095)
        legs_n = {}
        for n_odd in ns:
            co = workloads.uniform_case(case.num_experts, int(case.counts[0]), case.k, n_odd)
            workloads.fill_operands(co, device=dev, dtype=dtype)
            oo = gg.expert_offsets_from_recv_counts(co.counts, device=dev)
            legs_n[n_odd] = (co, (lambda co=co, oo=oo: gg.persistent_grouped_gemm(
                co.a, co.b, oo, num_sms=args.num_sms, use_atomic_queue=atomic)))
        settle_clock(legs_n[4096][1])
        times_n = {n_odd: [] for n_odd in ns}
        for rnd in range(12):
            for n_odd in ns[rnd % 3:] + ns[:rnd % 3]:
                times_n[n_odd] += batched_times_ms(legs_n[n_odd][1], launches=20, batch=10)
        odd = {f"n{n_odd}": {"kernel_ms_median": round(median(t), 5),
                             "tflops": round(legs_n[n_odd][0].flops / (median(t) * 1e-3) / 1e12, 1)}
               for n_odd, t in times_n.items()}
        odd["ratio_4092_over_4096"] = round(median(times_n[4092]) / median(times_n[4096]), 4)
        odd["ratio_4095_over_4096"] = round(median(times_n[4095]) / median(times_n[4096]), 4)
        del legs_n
        extra["n_not_multiple_of_8"] = odd
        progress("overlap leg")
        extra["overlap"] = overlap_summary(case, offs, dev)
        progress("reference benchmark default problem leg")
        extra["reference_bench_default"] = reference_bench_summary(dev, dtype, args.num_sms)

    progress("cpu baseline")
    cpu = None if args.no_cpu_baseline else cpu_baseline(case, args.cpu_seconds)

    metric = METRIC if is_metric_config else (
        f"grouped GEMM TFLOP/s, E={case.num_experts} {int(case.counts.max())} tok/expert "
        f"K{case.k} N{case.n} ({args.dtype})")
    result = {
        "metric": metric,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": ("synthetic (N(0,1) tokens, N(0,1/K) weights, random init)" if args.operands == "random"
                 else f"synthetic, operands {args.operands} (power analysis, not the metric)"),
        "config": {
            "workload": f"{case.name}: E={case.num_experts}, M={case.m}, K={case.k}, N={case.n}",
            "mode": args.mode,
            "block_m": args.block_m,
            "block_n": args.block_n,
            "kernel_tile": f"{kernel_tile[0]}x{kernel_tile[1]}",
            "num_sms": args.num_sms or "all CUs",
            "queue": "device",
        },
        "settle_launches": r["settle_launches"],
        "settle_ms": r["settle_ms"],
        "settled": r.get("settled"),
        "pct_bf16_peak": round(100 * value / PEAK_BF16_TFLOPS, 2),
        "kernel_ms_timed_mean": round(k_timed, 5),
        "event_launches": 10 * len(kernel_ms),
        "kernel_ms_median": round(k_med, 5),
        "kernel_ms_min": round(min(kernel_ms), 5),
        "kernel_ms_mean": round(k_mean, 5),
        "clock": r["clock"],
        "max_abs_diff_vs_fp32": round(max_abs, 6),
        "tolerance": round(tolerance, 6),
        "flushed": {
            "kernel_ms_median": round(k_flushed, 5),
            "kernel_ms_min": round(min(flushed), 5),
            "launches": len(flushed),
            "flush_bytes_per_launch": FLUSH_BYTES,
            "tflops": round(flops / (k_flushed * 1e-3) / 1e12, 1),
            "roofline_achieved": round(achieved_fl, 2),
            "roofline_frac": round(achieved_fl / peak, 4),
            "protocol": "a 512 MiB device write before each launch (L2 and MALL evicted), "
                        "HIP events around the launch",
        },
        "roofline": {
            "bound": "hbm" if hbm_bound else "mfma",
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": roof_unit,
            "frac": round(achieved / peak, 4),
            "achieved_from": "HIP events around the timed steps (GPU time per launch), warm caches; "
                             "the flushed field has the cache-cold fraction",
            "traffic": recorded_traffic(args.mode, case.name, kernel_tile),
            "traffic_source": "rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0 (copy-calibrated), "
                              + ("profiles/grouped_gemm_128x512_bf16_reference_bench.md"
                                 if case.name == "reference_bench"
                                 else "profiles/grouped_gemm_256x256_bf16_uniform.md"),
            "kernel": kernel_name(kernel_tile, args.dtype),
            "algorithmic_flops_per_launch": flops,
            "algorithmic_bytes_per_launch": nbytes,
            "hbm_gbps_at_algorithmic_bytes": round(nbytes / (k_timed * 1e-3) / 1e9, 1),
        },
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
