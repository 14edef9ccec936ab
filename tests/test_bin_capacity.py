"""Host protocol of the render's binning (splatting/tiles.py BinJob) on the
CPU: the tile phase is enqueued with a guessed capacity before the duplicate
count is read, and a count above the guess re-runs the binning with the exact
capacity.  The device library is replaced by a recorder that publishes the
count words the way gsx_bin_depth_async's first kernel does (seq << 32 |
word into the pinned host target), so no GPU is involved."""

from __future__ import annotations

import ctypes

import pytest
import torch

from mlx3d_amd import _lib
from mlx3d_amd.splatting import tiles


class _FakeLib:
    """Records the binning calls; the count phase's D is `dups`."""

    def __init__(self):
        self.host = (ctypes.c_uint64 * 16)()
        self.base = ctypes.addressof(self.host)
        self.calls = []
        self.dups = 0

    def gsx_host_status_alloc(self, pp):
        pp._obj.value = self.base
        return 0

    def gsx_host_status_free(self, p):
        return 0

    def gsx_bin_depth_workspace_bytes(self, n):
        return 256

    def gsx_bin_tile_workspace_bytes(self, cap, tiles):
        return 256

    def gsx_strerror(self, status):
        return b"fake error"

    def _publish(self, slot, seq, words):
        k = (slot.value - self.base) // 64
        for i, w in enumerate(words):
            self.host[8 * k + i] = (seq << 32) | w

    def gsx_bin_count_async(self, n, counts, dkeys, rects, w, h, dws, nb, ranges, status, st):
        self.calls.append(("count",))
        return 0

    def gsx_bin_depth_async(self, n, dkeys, dws, nb, status, slot, seq, st):
        self.calls.append(("depth", seq))
        self._publish(slot, seq, [0, 0, 0, self.dups, 0, 0, 0, 0])
        return 0

    def gsx_bin_tiles_async(self, n, counts, rects, m2, co, cs, w, h, dws, dnb, tws, tnb, cap,
                            ids, ranges, status, slot, seq, order, st):
        self.calls.append(("tiles", cap, seq))
        fits = cap >= self.dups
        self._publish(slot, seq, [self.dups if fits else 0, 0, 0, self.dups, 0, 0, 0, 0])
        return 0


@pytest.fixture
def fake(monkeypatch):
    f = _FakeLib()
    monkeypatch.setattr(_lib, "load", lambda: f)
    monkeypatch.setattr(_lib, "stream_handle", lambda dev: ctypes.c_void_p(0x5EED))
    monkeypatch.setattr(tiles, "_workspaces", {})
    return f


def _job(n=64):
    z = torch.zeros
    return tiles.BinJob(z(n, dtype=torch.int32), z(n, dtype=torch.int32),
                        z(n, 2, dtype=torch.int32), 64, 48)


def test_first_job_reads_the_count_before_the_tile_phase(fake):
    fake.dups = 1000
    job = _job()
    assert [c[0] for c in fake.calls] == ["count", "depth", "tiles"]
    assert fake.calls[2][1] == 1000  # exact capacity
    assert job.settle() is False
    ids, ranges = job.result()
    assert ids.shape == (1000,) and ranges.shape == (4 * 3, 2)


def test_guess_then_overflow_retry(fake):
    fake.dups = 1000
    _job().result()
    fake.calls.clear()

    # within the guess: one enqueue, tile phase sized by the guess, D read after
    fake.dups = 1100
    job = _job()
    guess = 1000 + 1000 // 4 + 1024
    assert [c[0] for c in fake.calls] == ["count", "depth", "tiles"]
    assert fake.calls[2][1] == guess
    assert job.ids.shape == (guess,)  # consumers may be enqueued on this buffer now
    assert job.settle() is False
    ids, _ = job.result()
    assert ids.shape == (1100,)
    fake.calls.clear()

    # above the guess: the tile phase ran short, settle() re-runs the binning
    # with the exact capacity and a new sequence number
    fake.dups = 5000
    job = _job()
    guess = 1100 + 1100 // 4 + 1024
    assert fake.calls[2][:2] == ("tiles", guess)
    first_seq = fake.calls[2][2]
    assert job.settle() is True
    assert [c[0] for c in fake.calls] == ["count", "depth", "tiles"] * 2
    assert fake.calls[5][1] == 5000 and fake.calls[5][2] != first_seq
    assert job.settle() is False  # settled once
    ids, _ = job.result()
    assert ids.shape == (5000,)
    job.check()  # the final status of the second run carries its sequence number
    fake.calls.clear()

    # the next guess covers the largest recent count
    fake.dups = 4000
    job = _job()
    assert fake.calls[2][1] == 5000 + 5000 // 4 + 1024
    assert job.result()[0].shape == (4000,)


def test_final_and_empty_jobs_are_exact(fake):
    fake.dups = 300
    _job().result()
    fake.calls.clear()
    fake.dups = 200
    job = tiles.BinJob(torch.zeros(8, dtype=torch.int32), torch.zeros(8, dtype=torch.int32),
                       torch.zeros(8, 2, dtype=torch.int32), 64, 48, final=True)
    assert fake.calls[2][1] == 200  # read before the tile phase despite the hint
    assert job.settle() is False
    fake.calls.clear()
    job = _job(n=0)
    assert [c[0] for c in fake.calls] == ["count", "tiles"]
    assert job.result()[0].shape == (0,)
