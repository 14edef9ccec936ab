"""Tile binning (``src/mlx3d/splatting/tiles.py:19-182``).

``bin_gaussians`` keeps the reference's signature and outputs: ``sorted_ids``
(D,) int32 in (tile, depth, index) order and ``tile_ranges`` (tiles, 2)
int32 with (0, 0) for empty tiles.  The work runs in ``gsx_bin_prepare`` and
``gsx_bin_count_async`` / ``gsx_bin_depth_async`` / ``gsx_bin_tiles_async``
(device radix passes and row placement).  The duplicate count D (the sum of
the tile counts, which the reference reads at tiles.py:68) reaches the host
without a copy or an event: the depth sort's first kernel writes the status
words into pinned host memory, which the host polls.  A render enqueues the
tile phase with a capacity guessed from the stream's latest counts and reads
D after its rasterizer has been enqueued, so nothing waits between kernels;
a count above the guess re-runs that frame's binning with the exact size.
"""

from __future__ import annotations

import collections
import ctypes
import threading
import time
import weakref

import numpy as np
import torch

from .. import _lib

TILE_SIZE = 16
_BIN_ERR_OVERFLOW = 2  # gsx_bin_error
_ERR_TOO_LARGE = -4    # gsx_status
_ERR_DEVICE = -5
_STATUS_WORDS = 8
_WAIT_LIMIT_S = 120.0  # a device that never publishes is reported, not waited on forever
_HINT_WINDOW = 16      # jobs whose duplicate counts size the next capacity guess

__all__ = ["TILE_SIZE", "bin_gaussians"]


class _HostStatus:
    """Two pinned host targets of 8 status words each (count phase, final
    status), which the binning's kernels write as (seq << 32 | word)."""

    def __init__(self):
        L = _lib.load()
        p = ctypes.c_void_p()
        _lib.check(L.gsx_host_status_alloc(ctypes.byref(p)), "gsx_host_status_alloc")
        self.addr = p.value
        self.words = np.ctypeslib.as_array(
            (ctypes.c_uint64 * (2 * _STATUS_WORDS)).from_address(self.addr))
        weakref.finalize(self, L.gsx_host_status_free, ctypes.c_void_p(self.addr))

    def slot(self, k: int):
        return ctypes.c_void_p(self.addr + 8 * _STATUS_WORDS * k)

    def wait(self, k: int, seq: int) -> tuple[np.ndarray, int]:
        """The words of target k once they carry `seq` or a later sequence
        number (kernels of one stream publish in order), and that number."""
        w = self.words[_STATUS_WORDS * k:_STATUS_WORDS * (k + 1)]
        t0 = None
        spins = 0
        while True:
            v = w.copy()
            tags = (v >> np.uint64(32)).astype(np.uint32)
            ahead = (tags - np.uint32(seq)).astype(np.uint32)  # modular: >= seq
            if (ahead < np.uint32(1 << 31)).all() and (tags == tags[0]).all():
                return (v & np.uint64(0xFFFFFFFF)).astype(np.uint32), int(tags[0])
            spins += 1
            if spins % 4096 == 0:
                t0 = t0 or time.perf_counter()
                if time.perf_counter() - t0 > _WAIT_LIMIT_S:
                    _lib.check(_ERR_DEVICE, "binning status (no status from the device)")


class _Workspace:
    """Grow-only scratch buffers of the binning phases, the persistent
    bin_status words and their pinned host targets, one set per (device,
    stream)."""

    def __init__(self, dev):
        self.depth = None
        self.tiles = None
        # device error bits accumulate here across jobs (gsx_bin_count_async
        # leaves word 1 alone), so each job's count readback also reports
        # the checks of the jobs before it
        self.status = torch.zeros((_STATUS_WORDS,), dtype=torch.int32, device=dev)
        self.host = _HostStatus()
        self.seq = 0
        self.recent = collections.deque(maxlen=_HINT_WINDOW)  # D of the latest jobs

    def capacity_hint(self) -> int | None:
        """Duplicate capacity for a job whose D is not read yet: 1.25x the
        largest D of the latest jobs on this stream (None before the first)."""
        if not self.recent:
            return None
        d = max(self.recent)
        return d + d // 4 + 1024

    def note_dups(self, d: int) -> None:
        self.recent.append(int(d))

    def next_seq(self) -> int:
        self.seq = (self.seq + 1) & 0xFFFFFFFF
        return self.seq

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


def _raise_on_errors(ws: _Workspace, err: int, what: str) -> None:
    if err == 0:
        return
    ws.status[1:2].zero_()  # report once
    if err & _BIN_ERR_OVERFLOW:
        _lib.check(_ERR_TOO_LARGE, f"{what} (more than 2^30 - 1 duplicates)")
    _lib.check(_ERR_DEVICE, f"{what} (a device-side check of this or an earlier binning "
                            "on this stream)")


class BinJob:
    """One binning on the device.

    gsx_bin_count_async sums the tile counts, the number of duplicates D
    emission writes; gsx_bin_depth_async's first kernel copies the status
    words (D among them) to the workspace's pinned host target.  When the
    stream has binned before (and without refine_tiles or ``final``), the
    tile phase is enqueued at once with a guessed capacity (1.25x the
    largest D of the latest jobs) and ``ids`` of that length: nothing waits
    between the phases, and ``ids`` and ``ranges`` are usable by kernels
    enqueued behind the job right away.  ``settle()`` then reads D from the
    host target; if D exceeds the guess the tile phase has written an
    in-bounds, empty binning (all ranges (0, 0)), and the whole binning is
    enqueued again with the exact capacity -- ``settle()`` returns True and
    the caller enqueues its consumers again.  Otherwise (the first job on a
    stream, refine_tiles, ``final``) the host polls for D before it
    enqueues the tile phase with exactly that capacity.  The tile phase's
    last kernel writes the final status words to the second target;
    ``check()`` waits for them and raises on a device-side error bit.
    ``result()`` calls it when D is unknown (refine_tiles); the render
    backward calls it after enqueuing its kernels, so a failed binning
    raises before the gradients reach an optimizer.  A job nobody checks
    has its error bits reported by the next job's count readback on the
    same stream.
    """

    def __init__(self, counts, dkeys, rects, width: int, height: int, refine=None,
                 final: bool = False, tile_order=None):
        """``refine`` = (means2d (N,2), conics (N,k>=3)) enables refine_tiles;
        ``tile_order`` (tile_order_buffer) receives the forward rasterizer's
        tile order for the ranges (gsx_raster_fwd then runs with order_ready)."""
        self.dev = counts.device
        self.n = counts.shape[0]
        self.width, self.height = int(width), int(height)
        self.tiles_x = (self.width + TILE_SIZE - 1) // TILE_SIZE
        self.tiles_y = (self.height + TILE_SIZE - 1) // TILE_SIZE
        self.stream = _lib.stream_handle(self.dev)
        self.ws = _workspace_for(self.dev, self.stream)
        self.ranges = torch.empty((self.tiles_x * self.tiles_y, 2), dtype=torch.int32,
                                  device=self.dev)
        self.inputs = (counts, dkeys, rects, refine)
        self.tile_order = tile_order
        self.exact = refine is not None or final  # D read before the tile phase, kept as is
        self._enqueue(None if self.exact else self.ws.capacity_hint())

    def _enqueue(self, guess: int | None) -> None:
        """Count phase, depth sort and tile phase, with capacity `guess`, or
        with the D read back in between when `guess` is None."""
        counts, dkeys, rects, refine = self.inputs
        n, ws, stream = self.n, self.ws, self.stream
        status = ws.status
        L = _lib.load()
        dws = ws.get_depth(self.dev, n)
        _lib.check(L.gsx_bin_count_async(
            n, _lib.ptr(counts), _lib.ptr(dkeys), _lib.ptr(rects), self.width, self.height,
            _lib.ptr(dws), dws.numel(), _lib.ptr(self.ranges), _lib.ptr(status), stream),
            "gsx_bin_count_async")
        self.seq = seq = ws.next_seq()
        self.cap = 0
        self.guessed = False
        if n > 0:
            _lib.check(L.gsx_bin_depth_async(n, _lib.ptr(dkeys), _lib.ptr(dws), dws.numel(),
                                             _lib.ptr(status), ws.host.slot(0), seq, stream),
                       "gsx_bin_depth_async")
            if guess is None:
                self.cap = self._read_count()
            else:
                self.cap, self.guessed = int(guess), True
        tws = ws.get_tiles(self.dev, self.cap, self.tiles_x * self.tiles_y)
        self.ids = torch.empty((self.cap,), dtype=torch.int32, device=self.dev)
        m2, co = refine if refine is not None else (None, None)
        _lib.check(L.gsx_bin_tiles_async(
            n, _lib.ptr(counts), _lib.ptr(rects), _lib.ptr(m2), _lib.ptr(co),
            0 if co is None else co.shape[1], self.width, self.height, _lib.ptr(dws),
            dws.numel(), _lib.ptr(tws), tws.numel(), self.cap, _lib.ptr(self.ids),
            _lib.ptr(self.ranges), _lib.ptr(status), ws.host.slot(1), seq,
            _lib.ptr(self.tile_order), stream),
            "gsx_bin_tiles_async")
        self.ready = n > 0  # n == 0 launches nothing after the count phase
        self.num_dups = None if (self.exact or self.guessed) else self.cap
        if n == 0:
            self.num_dups = 0

    def _read_count(self) -> int:
        """D of this job from the count phase's status words (first host
        target), which raises on device-side error bits."""
        words, tag = self.ws.host.wait(0, self.seq)
        if tag != self.seq:  # a later job on the stream overwrote the counts
            raise _lib.GsxError("gsx_bin_count_async: count read after a later binning")
        _raise_on_errors(self.ws, int(words[1]), "gsx_bin_count_async")
        d = int(words[3])
        self.ws.note_dups(d)
        return d

    def settle(self) -> bool:
        """Read D when the capacity was guessed.  Returns True when it
        exceeded the guess and the binning has been enqueued again with the
        exact capacity: work enqueued behind the first run (which saw empty
        ranges) must be enqueued again.  False otherwise, and for jobs sized
        exactly from the start."""
        if not self.guessed:
            return False
        self.guessed = False
        d = self._read_count()
        if d <= self.cap:
            self.num_dups = d
            return False
        self._enqueue(None)
        return True

    def check(self) -> None:
        """Wait for the final status, raise GsxError if a device-side check
        failed and set num_dups (duplicates kept)."""
        if not self.ready:
            return
        self.ready = False
        words, seq = self.ws.host.wait(1, self.seq)
        _raise_on_errors(self.ws, int(words[1]), "gsx_bin_tiles_async")
        if self.num_dups is not None:
            return
        if seq != self.seq:  # a later job on the stream overwrote the counts
            raise _lib.GsxError("gsx_bin_tiles_async: status read after a later binning")
        nd = ctypes.c_int64(0)
        rc = _lib.check(_lib.load().gsx_bin_status_check(
            words.ctypes.data_as(ctypes.c_void_p), self.cap, ctypes.byref(nd)),
            "gsx_bin_tiles_async")
        if rc != _lib.GSX_OK:  # not reached: the capacity is the emitted count
            raise _lib.GsxError("gsx_bin_tiles_async: duplicates exceed the exact capacity")
        self.num_dups = int(nd.value)

    def result(self):
        """(sorted_ids (D,), tile_ranges); reads D first when the capacity
        was guessed (see settle()) and waits for the whole binning when D
        is not known before it ends (refine_tiles)."""
        self.settle()
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
