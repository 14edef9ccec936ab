"""The C ABI library loads and exports exactly what include/gsx.h declares
(no compute call: this runs without a GPU)."""

import ctypes
import os
import re

import numpy as np
import pytest

from mlx3d_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "gsx.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b(gsx_\w+)\s*\(", src))


def test_header_symbols_exported():
    L = _lib.load()
    names = _declared()
    assert len(names) >= 16
    for n in sorted(names):
        assert hasattr(L, n), f"{n} declared in gsx.h but not exported"


def test_python_binding_covers_header():
    assert _declared() == set(_lib.SIGNATURES), "ctypes signatures drift from gsx.h"


def test_status_strings_and_version():
    L = _lib.load()
    assert L.gsx_abi_version() == 7
    assert _lib.strerror(0) == "ok"
    assert "invalid" in _lib.strerror(-1)
    assert "capacity" in _lib.strerror(1)


def test_camera_struct_layout():
    # 9 + 3 + 3 + 4 + 2 + 1 floats, 2 int32; lens: 2 int32 + 8 floats
    assert ctypes.sizeof(_lib.GsxCamera) == 4 * 34
    from oracle import oracle as O

    assert ctypes.sizeof(O.OrcCamera) == ctypes.sizeof(_lib.GsxCamera)
    assert [f[0] for f in O.OrcCamera._fields_] == [f[0] for f in _lib.GsxCamera._fields_]


def test_workspace_query_is_host_only():
    L = _lib.load()
    a = L.gsx_bin_workspace_bytes(1000, 5000, 100)
    b = L.gsx_bin_workspace_bytes(1000, 50000, 100)
    assert 0 < a < b
    assert L.gsx_bin_workspace_bytes(-1, 0, 1) < 0
    # the one-call workspace is the depth phase's followed by the tile phase's
    dn = L.gsx_bin_depth_workspace_bytes(1000)
    assert dn > 0 and dn % 256 == 0
    assert a == dn + L.gsx_bin_tile_workspace_bytes(5000, 100)
    assert b == dn + L.gsx_bin_tile_workspace_bytes(50000, 100)
    assert L.gsx_bin_depth_workspace_bytes(-1) < 0
    assert L.gsx_bin_tile_workspace_bytes(-1, 100) < 0
    assert L.gsx_bin_tile_workspace_bytes(10, 0) < 0
    # the rasterizers' tile-order buffer: T bounds + 16 ceil(T / 8) order entries
    assert L.gsx_tile_order_words(328, 200) == 21 * 13 + 16 * 35
    assert L.gsx_tile_order_words(16, 16) == 1 + 16
    assert L.gsx_tile_order_words(0, 16) == 0


def test_invalid_arguments_rejected_before_launch():
    L = _lib.load()
    # null camera / negative sizes fail fast without touching a device
    assert L.gsx_project_fwd(None, 10, None, None, None, 0.3, 0, None, None, None, None, None,
                             None) == -1
    assert L.gsx_eval_sh_fwd(-1, 16, 3, 3, None, None, None, None) == -1
    assert L.gsx_eval_sh_fwd(10, 4, 3, 3, None, None, None, None) == -1  # K < (deg+1)^2
    # the no-allocation L1 refuses sizes beyond its fixed scratch on the host
    # (the pointers are never dereferenced)
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    limit = L.gsx_l1_noalloc_max_elements()
    assert limit == 1 << 28
    assert L.gsx_l1_fwd_noalloc(limit + 1, p, p, p, None) == -4
    assert L.gsx_l1_fwd_noalloc(0, p, p, p, None) == -1
    assert L.gsx_l1_fwd_noalloc(10, None, p, p, None) == -1
    # the sign-keeping L1 pair checks its arguments before any launch
    assert L.gsx_l1_fwd_signs(0, p, p, p, 64, p, p, None) == -1
    assert L.gsx_l1_fwd_signs(10, p, p, p, 64, None, p, None) == -1
    assert L.gsx_l1_fwd_signs(10, p, p, p, 0, p, p, None) == -3  # workspace too small
    assert L.gsx_l1_bwd_signs(10, None, p, p, p, p, None) == -1
    assert L.gsx_l1_bwd_signs(-1, p, p, p, p, p, None) == -1


def test_bin_status_check_is_host_only():
    """gsx_bin_status_check interprets the status words of
    gsx_bin_sort_async: duplicates emitted, error bits (1 = wait bound,
    2 = overflow), duplicates dropped by refine_tiles."""
    L = _lib.load()

    def chk(words, cap):
        h = np.array(words, dtype=np.uint32)
        nd = ctypes.c_int64(-7)
        rc = L.gsx_bin_status_check(h.ctypes.data_as(ctypes.c_void_p), cap, ctypes.byref(nd))
        return rc, nd.value

    assert chk([123, 0, 0, 0, 0, 0, 0, 0], 123) == (0, 123)
    assert chk([123, 0, 20, 0, 0, 0, 0, 0], 123) == (0, 103)   # kept = emitted - dropped
    assert chk([124, 0, 0, 0, 0, 0, 0, 0], 123) == (1, 124)    # capacity needed
    assert chk([5, 2, 0, 0, 0, 0, 0, 0], 100)[0] == -4
    assert chk([5, 1, 0, 0, 0, 0, 0, 0], 100)[0] == -5
    assert L.gsx_strerror(-5).decode().startswith("device-side check")
    # binning entry points reject bad sizes before any launch
    nd = ctypes.c_int64(0)
    assert L.gsx_bin_sort(-1, None, None, None, None, None, 0, 64, 64, None, 0, 0, None, None,
                          ctypes.byref(nd), None) == -1
    assert L.gsx_bin_sort(10, None, None, None, None, None, 0, 64, 64, None, 0, 1 << 30, None,
                          None, ctypes.byref(nd), None) == -4
    assert L.gsx_bin_sort_async(10, None, None, None, None, None, 0, 64, 64, None, 0, 100, None,
                                None, None, None) == -1
    # the three phases: null outputs / inputs, negative sizes, a short workspace
    assert L.gsx_bin_count_async(10, None, None, None, 64, 64, None, 0, None, None, None) == -1
    assert L.gsx_bin_count_async(-1, None, None, None, 64, 64, None, 0, None, None, None) == -1
    assert L.gsx_bin_depth_async(-1, None, None, 0, None, None, 0, None) == -1
    assert L.gsx_bin_depth_async(10, None, None, 0, None, None, 0, None) == -1
    assert L.gsx_bin_depth_async(1 << 30, None, None, 0, None, None, 0, None) == -4
    st = np.zeros(8, np.uint32)
    rg = np.zeros(32, np.int32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731  (never dereferenced)
    assert L.gsx_bin_tiles_async(10, p(st), p(st), None, None, 0, 64, 64, p(st), 16, p(st), 16,
                                 100, p(rg), p(rg), p(st), None, 0, None, None) == -3
    assert L.gsx_bin_tiles_async(10, None, None, None, None, 0, 64, 64, None, 0, None, 0, 100,
                                 None, p(rg), p(st), None, 0, None, None) == -1
    assert L.gsx_bin_tiles_async(10, None, None, None, None, 0, 64, 64, None, 0, None, 0,
                                 1 << 30, None, p(rg), p(st), None, 0, None, None) == -4
    assert L.gsx_host_status_alloc(None) == -1
    assert L.gsx_host_status_free(None) == 0


def test_no_kernel_spills_registers():
    """build() records the compiler's per-kernel resource usage; no kernel
    may use scratch memory (register spills)."""
    import json
    import os

    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                        "mlx3d_amd", "_build", "resource_usage.json")
    if not os.path.exists(path):
        pytest.skip("libgsx.so was not built in this tree")
    usage = json.load(open(path))
    assert len(usage) > 50
    spills = {k: v["ScratchSize"] for k, v in usage.items() if v.get("ScratchSize", 0)}
    assert not spills, spills
