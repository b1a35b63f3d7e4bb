"""Writes the committed fixtures in tests/golden/ (run from the repo root).

* ``routing_counts.json`` -- per-expert counts of the benchmark configs, from
  their routing recipes (the skewed recipe reproduces the counts pinned in the
  build's survey).
* ``queues.npz`` -- expert offsets and the (expert, tile_m, tile_n) queue of
  every config at several tile shapes, written by a scalar triple loop (the
  enumeration order of src/triton_grouped_gemm.py:277-292).
* ``tiny_gemm.json`` -- small integer-valued grouped GEMMs whose fp32 results
  are exact, computed with Python integers.

The reference publishes no vectors for this path; these fixtures freeze the
restated algorithm so later changes to the oracle or the kernels are caught.
"""
from __future__ import annotations

import json
import random
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO / "moe-overlap_amd"))

import workloads  # noqa: E402

TILES = ((128, 128), (256, 128), (128, 256), (256, 256), (64, 64))


def routing_counts() -> dict:
    return {
        "cpu_plumbing": [128] * 8,
        "uniform": [512] * 16,
        "skewed": workloads.skewed_counts_from_recipe().tolist(),
        "expert_mlp": workloads.topk_counts(8192, 16, 2, softmax=True).tolist(),
        "fp8_fine": workloads.topk_counts(4096, 64, 6).tolist(),
    }


N_SIZES = {
    "cpu_plumbing": (1024,),
    "uniform": (4096,),
    "skewed": (4096,),
    "expert_mlp": (8192, 2048),
    "fp8_fine": (1408,),
}


def scalar_queue(offsets, n_size, bm, bn):
    we, wm, wn = [], [], []
    tiles_n = (n_size + bn - 1) // bn
    for e in range(len(offsets) - 1):
        cnt = max(offsets[e + 1] - offsets[e], 0)
        for tm in range((cnt + bm - 1) // bm):
            for tn in range(tiles_n):
                we.append(e)
                wm.append(tm)
                wn.append(tn)
    return [np.array(x, dtype=np.int32) for x in (we, wm, wn)]


def tiny_gemm_cases() -> list:
    rng = random.Random(1234)
    cases = []
    for counts, k, n in (([2, 0, 3], 4, 3), ([1, 4], 8, 5), ([0, 0], 3, 2), ([3, 1, 0, 2], 5, 4)):
        offs = [0]
        for c in counts:
            offs.append(offs[-1] + c)
        m = offs[-1] + 1  # one trailing row outside every expert range
        a = [[rng.randint(-3, 3) for _ in range(k)] for _ in range(m)]
        b = [[[rng.randint(-3, 3) for _ in range(n)] for _ in range(k)] for _ in counts]
        c = [[None] * n for _ in range(m)]
        for e in range(len(counts)):
            for i in range(offs[e], offs[e + 1]):
                for j in range(n):
                    c[i][j] = sum(a[i][kk] * b[e][kk][j] for kk in range(k))
        cases.append({"offsets": offs, "a": a, "b": b, "c": c})
    return cases


def main() -> None:
    counts = routing_counts()
    (HERE / "routing_counts.json").write_text(json.dumps(counts, indent=1) + "\n")
    arrays = {}
    for name, cs in counts.items():
        offs = [0]
        for c in cs:
            offs.append(offs[-1] + c)
        arrays[f"{name}__offsets"] = np.array(offs, dtype=np.int32)
        for n_size in N_SIZES[name]:
            for bm, bn in TILES:
                we, wm, wn = scalar_queue(offs, n_size, bm, bn)
                tag = f"{name}__n{n_size}__{bm}x{bn}"
                arrays[f"{tag}__expert"] = we
                arrays[f"{tag}__tile_m"] = wm
                arrays[f"{tag}__tile_n"] = wn
    np.savez_compressed(HERE / "queues.npz", **arrays)
    (HERE / "tiny_gemm.json").write_text(json.dumps(tiny_gemm_cases()) + "\n")


if __name__ == "__main__":
    main()
