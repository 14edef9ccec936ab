"""Tile binning (``src/mlx3d/splatting/tiles.py:19-182``).

``bin_gaussians`` keeps the reference's signature and outputs: ``sorted_ids``
(D,) int32 in (tile, depth, index) order and ``tile_ranges`` (tiles, 2)
int32 with (0, 0) for empty tiles.  The work runs in ``gsx_bin_prepare`` and
``gsx_bin_count_async`` / ``gsx_bin_depth_async`` / ``gsx_bin_tiles_async``
(device radix sorts).  The host reads the duplicate count (the sum of the tile
counts, which the reference reads at tiles.py:68) while the depth sort still
runs, and sizes the tile phase's buffers exactly from it.
"""

from __future__ import annotations

import ctypes
import threading

import numpy as np
import torch

from .. import _lib

TILE_SIZE = 16
_BIN_ERR_OVERFLOW = 2  # gsx_bin_error
_ERR_TOO_LARGE = -4    # gsx_status
_ERR_DEVICE = -5

__all__ = ["TILE_SIZE", "bin_gaussians"]


class _Workspace:
    """Grow-only scratch buffers of the binning phases and the persistent
    bin_status words, one set per (device, stream)."""

    def __init__(self, dev):
        self.depth = None
        self.tiles = None
        # device error bits accumulate here across jobs (gsx_bin_count_async
        # leaves word 1 alone), so each job's count readback also reports
        # the checks of the jobs before it
        self.status = torch.zeros((4,), dtype=torch.int32, device=dev)

    @staticmethod
    def _grow(buf, dev, need: int, what: str) -> torch.Tensor:
        if need < 0:
            raise ValueError(f"bad binning sizes for the {what} workspace")
        if buf is None or buf.numel() < need:
            buf = torch.empty(int(need * 1.1) + 4096, dtype=torch.uint8, device=dev)
        return buf

    def get_depth(self, dev, n: int) -> torch.Tensor:
        self.depth = self._grow(self.depth, dev, int(_lib.load().gsx_bin_depth_workspace_bytes(n)),
                                "depth")
        return self.depth

    def get_tiles(self, dev, cap: int, num_tiles: int) -> torch.Tensor:
        need = int(_lib.load().gsx_bin_tile_workspace_bytes(cap, num_tiles))
        self.tiles = self._grow(self.tiles, dev, need, "tile")
        return self.tiles


_workspaces: dict = {}
_ws_lock = threading.Lock()


def _workspace_for(dev, stream) -> _Workspace:
    key = (dev, stream.value)
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None:
            ws = _workspaces[key] = _Workspace(dev)
    return ws


def _pinned_status(status: torch.Tensor):
    """Copy of the 4 status words into pinned host memory behind the work
    enqueued so far, and the event that marks it."""
    host = torch.empty((4,), dtype=torch.int32, pin_memory=True)
    host.copy_(status, non_blocking=True)
    ev = torch.cuda.Event()
    ev.record()
    return host, ev


def _raise_on_errors(ws: _Workspace, err: int, what: str) -> None:
    if err == 0:
        return
    ws.status[1:2].zero_()  # report once
    if err & _BIN_ERR_OVERFLOW:
        _lib.check(_ERR_TOO_LARGE, f"{what} (more than 2^30 - 1 duplicates)")
    _lib.check(_ERR_DEVICE, f"{what} (a device-side check of this or an earlier binning "
                            "on this stream)")


class BinJob:
    """One binning on the device, sized exactly.

    gsx_bin_count_async sums the tile counts, the number of duplicates
    emission writes; the job copies the status words to pinned memory,
    enqueues the depth sort (gsx_bin_depth_async, which keeps the device
    busy meanwhile) and waits for that copy only, allocates ``ids`` with
    exactly that capacity and enqueues the rest (gsx_bin_tiles_async).
    ``ids`` and ``ranges`` are usable by kernels enqueued behind the job
    right away.  Without refine_tiles D is that count and no second host
    sync is needed.  Every job copies its final status words to pinned
    memory behind the tile phase (no wait); ``check()`` waits for that copy
    and raises on a device-side error bit of the tile phase.  ``result()``
    calls it when D is unknown (refine_tiles); the render backward calls it
    after enqueuing its kernels, so a failed binning raises before the
    gradients reach an optimizer.  A job nobody checks has its error bits
    reported by the next job's count readback on the same stream.
    """

    def __init__(self, counts, dkeys, rects, width: int, height: int, refine=None,
                 final: bool = False):
        """``refine`` = (means2d (N,2), conics (N,k>=3)) enables refine_tiles."""
        self.dev = counts.device
        self.n = n = counts.shape[0]
        self.width, self.height = int(width), int(height)
        self.tiles_x = (self.width + TILE_SIZE - 1) // TILE_SIZE
        self.tiles_y = (self.height + TILE_SIZE - 1) // TILE_SIZE
        num_tiles = self.tiles_x * self.tiles_y
        stream = _lib.stream_handle(self.dev)
        ws = self.ws = _workspace_for(self.dev, stream)
        status = ws.status
        self.ranges = torch.empty((num_tiles, 2), dtype=torch.int32, device=self.dev)
        L = _lib.load()
        dws = ws.get_depth(self.dev, n)
        _lib.check(L.gsx_bin_count_async(
            n, _lib.ptr(counts), _lib.ptr(dkeys), self.width, self.height, _lib.ptr(dws),
            dws.numel(), _lib.ptr(self.ranges), _lib.ptr(status), stream),
            "gsx_bin_count_async")
        host, ev = _pinned_status(status)
        _lib.check(L.gsx_bin_depth_async(n, _lib.ptr(dkeys), _lib.ptr(dws), dws.numel(),
                                         _lib.ptr(status), stream), "gsx_bin_depth_async")
        ev.synchronize()
        words = host.numpy().view(np.uint32)
        _raise_on_errors(ws, int(words[1]), "gsx_bin_count_async")
        self.cap = int(words[3])
        tws = ws.get_tiles(self.dev, self.cap, num_tiles)
        self.ids = torch.empty((self.cap,), dtype=torch.int32, device=self.dev)
        m2, co = refine if refine is not None else (None, None)
        _lib.check(L.gsx_bin_tiles_async(
            n, _lib.ptr(counts), _lib.ptr(rects), _lib.ptr(m2), _lib.ptr(co),
            0 if co is None else co.shape[1], self.width, self.height, _lib.ptr(dws),
            dws.numel(), _lib.ptr(tws), tws.numel(), self.cap, _lib.ptr(self.ids),
            _lib.ptr(self.ranges), _lib.ptr(status), stream), "gsx_bin_tiles_async")
        self.host, self.ready = _pinned_status(status)
        self.num_dups = None if (refine is not None or final) else self.cap

    def check(self) -> None:
        """With a final status copy: wait for the binning, raise GsxError if
        a device-side check failed and set num_dups (duplicates kept)."""
        if self.ready is None:
            return
        self.ready.synchronize()
        self.ready = None
        words = np.ascontiguousarray(self.host.numpy().view(np.uint32))
        _raise_on_errors(self.ws, int(words[1]), "gsx_bin_tiles_async")
        nd = ctypes.c_int64(0)
        rc = _lib.check(_lib.load().gsx_bin_status_check(
            words.ctypes.data_as(ctypes.c_void_p), self.cap, ctypes.byref(nd)),
            "gsx_bin_tiles_async")
        if rc != _lib.GSX_OK:  # not reached: the capacity is the emitted count
            raise _lib.GsxError("gsx_bin_tiles_async: duplicates exceed the exact capacity")
        if self.num_dups is None:
            self.num_dups = int(nd.value)

    def result(self):
        """(sorted_ids (D,), tile_ranges); waits for the binning only when D
        is not yet known (refine_tiles)."""
        if self.num_dups is None:
            self.check()
        return self.ids[:self.num_dups], self.ranges


def _bin_sort(counts, dkeys, rects, width: int, height: int, refine=None):
    """Binning with the exact capacity, reading the final status (the
    reference also syncs here, tiles.py:68)."""
    job = BinJob(counts, dkeys, rects, width, height, refine, final=True)
    job.check()
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
