"""include/mgg.h as a C caller sees it: a C99 program (gcc -Wall -Werror)
includes the header, takes the address of every entry point it declares,
links against libmgg.so and runs the host-side calls (ABI version, error
message, the host offsets builder and a rejected launch), without a GPU.
This is the boundary a non-Python binding (cgo, JNI, a C++ runtime) would
use in place of src/triton_grouped_gemm.py's module functions."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

import mgg_native as nat

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "mgg.h"
LIB = REPO / "moe-overlap_amd" / "libmgg.so"
ROCM_LIB = Path("/opt/rocm/lib")


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mgg_\w+)\s*\(", text)))


PROGRAM = r"""
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include "mgg.h"

typedef void (*any_fn)(void);
static any_fn entry_points[] = {
%(entries)s
};

int main(void) {
  int32_t counts[4] = {3, 0, 5, 2};
  int32_t offsets[5] = {-1, -1, -1, -1, -1};
  size_t i;
  for (i = 0; i < sizeof(entry_points) / sizeof(entry_points[0]); ++i)
    if (entry_points[i] == NULL) return 10;
  if (mgg_abi_version() != %(abi)d) return 11;
  if (mgg_expert_offsets_from_counts_host(counts, MGG_INT32, 4, offsets, MGG_INT32) != MGG_OK)
    return 12;
  if (offsets[0] != 0 || offsets[1] != 3 || offsets[2] != 3 || offsets[3] != 8 || offsets[4] != 10)
    return 13;
  /* A launch with an unsupported tile is rejected before any device work. */
  if (mgg_grouped_gemm(MGG_DTYPE_BF16, (void*)16, (void*)16, (void*)16, (const int32_t*)16,
                       64, 64, 64, 1, 64, 4096, 64, 64, NULL, NULL, NULL, -1, 96, 128, 4, 0,
                       NULL, 0, 0, NULL) != MGG_ERR_UNSUPPORTED)
    return 14;
  if (strstr(mgg_last_error(), "block_m") == NULL) return 15;
  printf("ok %%d\n", mgg_abi_version());
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")
def test_c_program_links_and_runs(tmp_path):
    assert LIB.exists(), "build libmgg.so first (__graft_entry__.build())"
    names = declared_functions()
    assert len(names) >= 15
    entries = "\n".join(f"  (any_fn)&{n}," for n in names)
    src = tmp_path / "caller.c"
    src.write_text(PROGRAM % {"entries": entries, "abi": nat.ABI_VERSION})
    exe = tmp_path / "caller"
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-Wno-pedantic",
           f"-I{REPO / 'include'}", str(src), "-o", str(exe), str(LIB),
           f"-Wl,-rpath,{LIB.parent}", f"-Wl,-rpath-link,{ROCM_LIB}", f"-L{ROCM_LIB}"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, (run.returncode, run.stderr[-2000:])
    assert run.stdout.strip() == f"ok {nat.ABI_VERSION}"
