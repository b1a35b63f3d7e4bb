"""The allocation-free dispatch layout (mgg_dispatch_layout_noalloc, workspace
in the library's device scratch array) against mgg_dispatch_layout with a
caller workspace, through the C ABI: bit-exact integer outputs on two calls
in a row, the second smaller, plus the oracle's layout (train:219-237) and
the rejection of layouts whose workspace exceeds the scratch array."""
import ctypes
import sys

import numpy as np
import pytest
import torch

import mgg_native as nat
from oracle import expert_mlp_oracle as mo

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _outputs(T, k, E, dev):
    i32 = dict(dtype=torch.int32, device=dev)
    return [torch.full((E,), -7, **i32), torch.full((E + 1,), -7, **i32)] + \
           [torch.full((T * k,), -7, **i32) for _ in range(3)]


def _routing(T, k, E, seed):
    gen = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, E, (T, k), generator=gen, dtype=torch.int64)
    idx[torch.rand(T, k, generator=gen) < 0.05] = -1  # masked slots
    return idx


def _layout_with_workspace(idx, E, dev, stream):
    T, k = idx.shape
    outs = _outputs(T, k, E, dev)
    lib = nat.lib()
    ws_bytes = int(lib.mgg_dispatch_layout_workspace_bytes(T, k, E))
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=dev)
    nat.check(lib.mgg_dispatch_layout(_p(idx), nat.MGG_INT64, T, k, E, *map(_p, outs), _p(ws),
                                      ws_bytes, stream))
    return outs


def _layout_noalloc(idx, E, dev, stream):
    T, k = idx.shape
    outs = _outputs(T, k, E, dev)
    nat.check(nat.lib().mgg_dispatch_layout_noalloc(_p(idx), nat.MGG_INT64, T, k, E,
                                                    *map(_p, outs), stream))
    return outs


def test_noalloc_layout_matches_workspace_layout(cuda_device):
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # Second call smaller than the first (fewer chunks and experts): what the
    # first call left in the scratch array must not leak into it.
    for T, k, E, seed in ((8192, 6, 64, 0), (1500, 2, 16, 1), (40000, 6, 100, 2)):
        print(f"noalloc layout T={T} k={k} E={E}", file=sys.stderr, flush=True)
        idx = _routing(T, k, E, seed).to(cuda_device)
        got = _layout_noalloc(idx, E, cuda_device, stream)
        want = _layout_with_workspace(idx, E, cuda_device, stream)
        torch.cuda.synchronize()
        counts, offsets, pos, tok, row = (t.cpu().numpy() for t in got)
        rows = int(offsets[-1])
        for g, w in zip(got[:3], want[:3]):
            assert torch.equal(g, w)
        for g, w in zip(got[3:], want[3:]):
            assert torch.equal(g[:rows], w[:rows])
        o_counts, o_offsets, o_pos, o_tok, o_row = mo.dispatch_layout(idx.cpu().numpy(), E)
        np.testing.assert_array_equal(counts, o_counts)
        np.testing.assert_array_equal(offsets, o_offsets)
        np.testing.assert_array_equal(pos, o_pos)
        np.testing.assert_array_equal(tok[:rows], o_tok[:rows])
        np.testing.assert_array_equal(row[:rows], o_row[:rows])


def test_noalloc_layout_rejects_oversized_workspace(cuda_device):
    lib = nat.lib()
    # 300000 assignments over 1024 experts need 293 * 1024 * 4 bytes > 1 MiB.
    assert lib.mgg_dispatch_layout_workspace_bytes(300000, 1, 1024) > 1 << 20
    # Null pointers: the size check must reject the call before any pointer
    # is used (were it skipped, the null checks behind it would answer
    # MGG_ERR_INVALID instead, still without a launch).
    rc = lib.mgg_dispatch_layout_noalloc(None, nat.MGG_INT64, 300000, 1, 1024, None, None, None,
                                         None, None, None)
    assert rc == nat.MGG_ERR_UNSUPPORTED
    assert b"1 MiB" in lib.mgg_last_error()
    # The largest layout that fits (256 chunks x 1024 experts = 1 MiB) is accepted.
    assert lib.mgg_dispatch_layout_workspace_bytes(262144, 1, 1024) == 1 << 20
