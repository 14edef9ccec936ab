"""Tile binning (``src/mlx3d/splatting/tiles.py:19-182``).

``bin_gaussians`` keeps the reference's signature and outputs: ``sorted_ids``
(D,) int32 in (tile, depth, index) order and ``tile_ranges`` (tiles, 2)
int32 with (0, 0) for empty tiles.  The work runs in ``gsx_bin_prepare`` and
``gsx_bin_sort`` (device radix sorts); the only host sync is the 8-byte
readback of D that the reference also does (tiles.py:68).
"""

from __future__ import annotations

import ctypes
import threading

import torch

from .. import _lib

TILE_SIZE = 16

__all__ = ["TILE_SIZE", "bin_gaussians"]


class _Workspace:
    """Grow-only scratch buffer for gsx_bin_sort, one per (device, stream)."""

    def __init__(self):
        self.buf = None
        self.n = -1
        self.cap = -1
        self.last_dups = 0

    def get(self, dev, n: int, cap: int, num_tiles: int) -> torch.Tensor:
        need = int(_lib.load().gsx_bin_workspace_bytes(n, cap, num_tiles))
        if self.buf is None or self.buf.numel() < need:
            self.buf = torch.empty(int(need * 1.1) + 4096, dtype=torch.uint8, device=dev)
        return self.buf


_workspaces: dict = {}
_ws_lock = threading.Lock()


def _workspace_for(dev, stream) -> _Workspace:
    key = (dev, stream.value)
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None:
            ws = _workspaces[key] = _Workspace()
    return ws


def _bin_sort(counts, dkeys, rects, width: int, height: int):
    """gsx_bin_sort with a capacity guess from the previous call; retried
    once with the exact duplicate count when the guess is too small."""
    dev = counts.device
    n = counts.shape[0]
    tiles_x = (width + TILE_SIZE - 1) // TILE_SIZE
    tiles_y = (height + TILE_SIZE - 1) // TILE_SIZE
    T = tiles_x * tiles_y
    ranges = torch.empty((T, 2), dtype=torch.int32, device=dev)
    st = _lib.stream_handle(dev)
    ws = _workspace_for(dev, st)
    cap = max(1024, int(ws.last_dups * 1.25), 4 * n)
    L = _lib.load()
    for _ in range(2):
        buf = ws.get(dev, n, cap, T)
        ids = torch.empty((cap,), dtype=torch.int32, device=dev)
        nd = ctypes.c_int64(0)
        rc = _lib.check(L.gsx_bin_sort(n, _lib.ptr(counts), _lib.ptr(dkeys), _lib.ptr(rects), width,
                                       height, _lib.ptr(buf), buf.numel(), cap, _lib.ptr(ids),
                                       _lib.ptr(ranges), ctypes.byref(nd), st), "gsx_bin_sort")
        D = int(nd.value)
        ws.last_dups = D
        if rc == _lib.GSX_OK:
            return ids[:D], ranges
        cap = D + D // 8 + 1024
    raise _lib.GsxError("gsx_bin_sort: capacity retry failed")


def bin_gaussians(means2d: torch.Tensor, radii: torch.Tensor, depths: torch.Tensor, width: int,
                  height: int, conics: torch.Tensor | None = None):
    """Assign Gaussians to 16x16 tiles and sort by (tile, depth) (tiles.py:19-182).

    Returns ``(sorted_ids, tile_ranges, tiles_x, tiles_y)``.  Inputs carry no
    gradient (tiles.py:44-47).
    """
    if conics is not None:
        raise NotImplementedError("refine_tiles (conic tile rejection, tiles.py:91-164) is "
                                  "not implemented yet")
    n = means2d.shape[0]
    if means2d.shape != (n, 2) or radii.shape != (n,) or depths.shape != (n,):
        raise ValueError("means2d must be (N, 2), radii and depths (N,).")
    dev = _lib.require_device(means2d, radii, depths)
    m = _lib.f32c(means2d.detach())
    r = _lib.f32c(radii.detach())
    d = _lib.f32c(depths.detach())
    counts = torch.empty((n,), dtype=torch.int32, device=dev)
    dkeys = torch.empty((n,), dtype=torch.int32, device=dev)
    rects = torch.empty((n, 2), dtype=torch.int32, device=dev)
    L = _lib.load()
    _lib.check(L.gsx_bin_prepare(n, _lib.ptr(m), _lib.ptr(r), _lib.ptr(d), width, height,
                                 _lib.ptr(counts), _lib.ptr(dkeys), _lib.ptr(rects),
                                 _lib.stream_handle(dev)), "gsx_bin_prepare")
    ids, ranges = _bin_sort(counts, dkeys, rects, width, height)
    tiles_x = (width + TILE_SIZE - 1) // TILE_SIZE
    tiles_y = (height + TILE_SIZE - 1) // TILE_SIZE
    return ids, ranges, tiles_x, tiles_y
