"""gsx_l1_fwd_noalloc (the entry point that allocates nothing) against
gsx_l1_fwd, called through the C ABI: bit-identical results on two calls in
a row, the second with a smaller input, and the size limit refused before
any launch."""

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import cu, say
from mlx3d_amd import _lib

pytestmark = pytest.mark.gpu


def _l1_workspace(L, x, y, dev):
    n = x.numel()
    ws = torch.empty(int(L.gsx_l1_workspace_bytes(n)), dtype=torch.uint8, device=dev)
    out = torch.empty(2, dtype=torch.float32, device=dev)
    rc = L.gsx_l1_fwd(n, _lib.ptr(x), _lib.ptr(y), _lib.ptr(ws), ws.numel(), _lib.ptr(out),
                      _lib.stream_handle(dev))
    assert rc == 0, _lib.load().gsx_strerror(rc)
    return out


def _l1_noalloc(L, x, y, dev):
    out = torch.empty(2, dtype=torch.float32, device=dev)
    rc = L.gsx_l1_fwd_noalloc(x.numel(), _lib.ptr(x), _lib.ptr(y), _lib.ptr(out),
                              _lib.stream_handle(dev))
    assert rc == 0, _lib.load().gsx_strerror(rc)
    return out


def test_noalloc_matches_workspace_entry_point():
    L = _lib.load()
    dev = torch.device("cuda")
    rng = np.random.default_rng(7)
    # two calls in a row on the shared scratch, the second smaller: its
    # result must not see the first call's partials
    for n, off in [(1920 * 1080 * 3, 0), (1000 * 37 + 5, 1)]:
        a = rng.uniform(0, 1, n + off).astype(np.float32)
        b = rng.uniform(0, 1, n + off).astype(np.float32)
        x, y = cu(a)[off:], cu(b)[off:]  # off = 1: unaligned (scalar-load path)
        got = _l1_noalloc(L, x, y, dev)
        ref = _l1_workspace(L, x, y, dev)
        torch.cuda.synchronize()
        g, r = got.cpu().numpy(), ref.cpu().numpy()
        exact = np.abs(a[off:].astype(np.float64) - b[off:]).mean()
        say(f"n={n}: noalloc {g[0]!r} workspace {r[0]!r} float64 {exact!r}")
        assert g[0].view(np.int32) == r[0].view(np.int32)
        assert abs(float(g[0]) - exact) <= 1e-6 * exact


def test_noalloc_size_limit_refused_before_launch():
    L = _lib.load()
    dev = torch.device("cuda")
    x = torch.zeros(16, dtype=torch.float32, device=dev)
    out = torch.zeros(2, dtype=torch.float32, device=dev)
    limit = int(L.gsx_l1_noalloc_max_elements())
    assert limit == 1 << 28
    # the host check returns before anything is enqueued (n is never read)
    rc = L.gsx_l1_fwd_noalloc(limit + 1, _lib.ptr(x), _lib.ptr(x), _lib.ptr(out),
                              _lib.stream_handle(dev))
    assert rc == -4  # GSX_ERR_TOO_LARGE
    assert float(out[0]) == 0.0
