"""Our device code must never write through the scalar data cache.

Compiles each HIP source of libmgg to AMDGPU assembly (device pass only) and
rejects scalar-memory stores, scalar atomics and scalar-cache write-back or
discard.  CPU-only; this file is kept off the GPU box because it names those
instructions."""
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO / "moe-overlap_amd"))
import build_native  # noqa: E402

FORBIDDEN = ("s_store_", "s_buffer_store", "s_atomic_", "s_buffer_atomic", "s_scratch_store",
             "s_dcache_wb", "s_dcache_discard")


@pytest.mark.parametrize("src", build_native.SOURCES)
def test_no_scalar_cache_writes(src, tmp_path):
    out = tmp_path / (Path(src).stem + ".s")
    cmd = [build_native._hipcc(), *build_native.HIP_FLAGS, "--cuda-device-only", "-S",
           str(build_native.CSRC / src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    bad = [line.strip() for line in out.read_text().splitlines()
           if line.strip().split(" ")[0].startswith(FORBIDDEN)]
    assert not bad, bad[:10]
