"""The C ABI library loads and exports exactly what include/gsx.h declares
(no compute call: this runs without a GPU)."""

import ctypes
import os
import re

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
    assert L.gsx_abi_version() == 1
    assert _lib.strerror(0) == "ok"
    assert "invalid" in _lib.strerror(-1)
    assert "capacity" in _lib.strerror(1)


def test_camera_struct_layout():
    # 9 + 3 + 3 + 4 + 2 + 1 floats, 2 int32
    assert ctypes.sizeof(_lib.GsxCamera) == 4 * 24


def test_workspace_query_is_host_only():
    L = _lib.load()
    a = L.gsx_bin_workspace_bytes(1000, 5000, 100)
    b = L.gsx_bin_workspace_bytes(1000, 50000, 100)
    assert 0 < a < b
    assert L.gsx_bin_workspace_bytes(-1, 0, 1) < 0


def test_invalid_arguments_rejected_before_launch():
    L = _lib.load()
    # null camera / negative sizes fail fast without touching a device
    assert L.gsx_project_fwd(None, 10, None, None, None, 0.3, 0, None, None, None, None, None,
                             None) == -1
    assert L.gsx_eval_sh_fwd(-1, 16, 3, 3, None, None, None, None) == -1
    assert L.gsx_eval_sh_fwd(10, 4, 3, 3, None, None, None, None) == -1  # K < (deg+1)^2
