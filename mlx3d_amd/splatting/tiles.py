"""Tile binning (``src/mlx3d/splatting/tiles.py:19-182``).

``bin_gaussians`` keeps the reference's signature and outputs: ``sorted_ids``
(D,) int32 in (tile, depth, index) order and ``tile_ranges`` (tiles, 2)
int32 with (0, 0) for empty tiles.  The work runs in ``gsx_bin_prepare`` and
``gsx_bin_sort_async`` (device radix sorts); the only host sync is the
8-byte readback of D that the reference also does (tiles.py:68), and the
renderer places it after the rasterizer has been enqueued.
"""

from __future__ import annotations

import ctypes
import threading

import numpy as np
import torch

from .. import _lib

TILE_SIZE = 16

__all__ = ["TILE_SIZE", "bin_gaussians"]


class _Workspace:
    """Grow-only scratch buffer for gsx_bin_sort_async, one per (device, stream)."""

    def __init__(self):
        self.buf = None
        self.last_dups = 0

    def get(self, dev, n: int, cap: int, num_tiles: int) -> torch.Tensor:
        need = int(_lib.load().gsx_bin_workspace_bytes(n, cap, num_tiles))
        if need < 0:
            raise ValueError(f"bad binning sizes: n={n}, capacity={cap}")
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


class BinJob:
    """One binning on the device with the duplicate count D left there.

    ``ids`` (capacity,) and ``ranges`` are usable by kernels enqueued behind
    the job right away.  The two status words (D, error bits) are copied to
    pinned host memory right behind the binning kernels, so ``finish()``
    (the one host sync, as tiles.py:68 does) waits for the binning only,
    not for work the caller enqueued after it.  It reports whether the
    capacity sufficed; when it did not, ``retry()`` re-enqueues the binning
    with room for D and the caller re-enqueues what it ran on the
    incomplete result.
    """

    def __init__(self, counts, dkeys, rects, width: int, height: int, refine=None):
        """``refine`` = (means2d (N,2), conics (N,k>=3)) enables refine_tiles."""
        self.dev = counts.device
        self.args = (counts, dkeys, rects)
        self.refine = refine
        self.n = counts.shape[0]
        self.width, self.height = int(width), int(height)
        self.tiles_x = (self.width + TILE_SIZE - 1) // TILE_SIZE
        self.tiles_y = (self.height + TILE_SIZE - 1) // TILE_SIZE
        self.stream = _lib.stream_handle(self.dev)
        self.ws = _workspace_for(self.dev, self.stream)
        self.ranges = torch.empty((self.tiles_x * self.tiles_y, 2), dtype=torch.int32,
                                  device=self.dev)
        self.status = torch.empty((4,), dtype=torch.int32, device=self.dev)
        self.num_dups = None
        self._enqueue(max(1024, int(self.ws.last_dups * 1.25), 4 * self.n))

    def _enqueue(self, cap: int):
        counts, dkeys, rects = self.args
        self.cap = int(cap)
        buf = self.ws.get(self.dev, self.n, self.cap, self.tiles_x * self.tiles_y)
        self.ids = torch.empty((self.cap,), dtype=torch.int32, device=self.dev)
        m2, co = self.refine if self.refine is not None else (None, None)
        _lib.check(_lib.load().gsx_bin_sort_async(
            self.n, _lib.ptr(counts), _lib.ptr(dkeys), _lib.ptr(rects), _lib.ptr(m2),
            _lib.ptr(co), 0 if co is None else co.shape[1], self.width, self.height,
            _lib.ptr(buf), buf.numel(), self.cap, _lib.ptr(self.ids), _lib.ptr(self.ranges),
            _lib.ptr(self.status), self.stream), "gsx_bin_sort_async")
        self.host = torch.empty((4,), dtype=torch.int32, pin_memory=True)
        self.host.copy_(self.status, non_blocking=True)
        self.ready = torch.cuda.Event()
        self.ready.record()

    def finish(self) -> bool:
        """Read D back; True if the binning is complete (num_dups = duplicates
        kept), False if retry() is due (num_dups = capacity needed)."""
        self.ready.synchronize()
        host = np.ascontiguousarray(self.host.numpy().view(np.uint32))
        nd = ctypes.c_int64(0)
        rc = _lib.check(_lib.load().gsx_bin_status_check(
            host.ctypes.data_as(ctypes.c_void_p), self.cap, ctypes.byref(nd)),
            "gsx_bin_sort_async")
        self.num_dups = int(nd.value)
        self.ws.last_dups = self.num_dups
        return rc == _lib.GSX_OK

    def retry(self):
        self._enqueue(self.num_dups + self.num_dups // 8 + 1024)
        self.num_dups = None

    def result(self):
        """(sorted_ids (D,), tile_ranges) once finish() returned True."""
        return self.ids[:self.num_dups], self.ranges


def _bin_sort(counts, dkeys, rects, width: int, height: int, refine=None):
    """Binning with the capacity guessed from the previous call; one retry
    with room for the exact duplicate count when the guess was short."""
    job = BinJob(counts, dkeys, rects, width, height, refine)
    if not job.finish():
        job.retry()
        if not job.finish():
            raise _lib.GsxError("gsx_bin_sort_async: capacity retry failed")
    return job.result()


def bin_gaussians(means2d: torch.Tensor, radii: torch.Tensor, depths: torch.Tensor, width: int,
                  height: int, conics: torch.Tensor | None = None):
    """Assign Gaussians to 16x16 tiles and sort by (tile, depth) (tiles.py:19-182).

    With ``conics`` (N, 3) the tiles of each Gaussian's square bbox whose
    rectangle the conic's 3.46-sigma ellipse (q <= 12) does not reach are
    dropped (refine_tiles, tiles.py:91-164).  Returns ``(sorted_ids,
    tile_ranges, tiles_x, tiles_y)``.  Inputs carry no gradient
    (tiles.py:44-47).
    """
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
    refine = None
    if conics is not None:
        if conics.shape != (n, 3):
            raise ValueError("conics must be (N, 3).")
        _lib.require_device(conics)
        refine = (m, _lib.f32c(conics.detach()))
    ids, ranges = _bin_sort(counts, dkeys, rects, width, height, refine)
    tiles_x = (width + TILE_SIZE - 1) // TILE_SIZE
    tiles_y = (height + TILE_SIZE - 1) // TILE_SIZE
    return ids, ranges, tiles_x, tiles_y
