"""Import-compatible alias of the reference's module name.

Callers written against ``src/triton_grouped_gemm.py`` (``from
triton_grouped_gemm import persistent_grouped_gemm, reference_grouped_gemm``)
run unchanged with this directory on ``sys.path``.  Everything here is the
HIP implementation in ``grouped_gemm``; no Triton is involved.
"""
from grouped_gemm import (  # noqa: F401
    _WORK_QUEUE_CACHE,
    _WORK_QUEUE_CACHE_MAX,
    _build_work_queue,
    expert_offsets_from_recv_counts,
    grouped_gemm_flops,
    persistent_grouped_gemm,
    reference_grouped_gemm,
)
