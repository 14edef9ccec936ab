"""ctypes binding of ``libgsx.so`` (the C ABI declared in ``include/gsx.h``).

The library is the only compute path: there is no CPU or eager-PyTorch
fallback.  If the shared object is missing, or a tensor is not on a ROCm
device, the call raises instead of silently computing something else.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgsx.so")

GSX_OK = 0
LOG_SCALES = 1
LOGIT_OPACITY = 2
ANTIALIAS = 4
PROJECT_UT = 8


class GsxError(RuntimeError):
    """A gsx entry point returned an error status."""


class GsxCamera(ctypes.Structure):
    """Mirror of ``gsx_camera`` (include/gsx.h)."""

    _fields_ = [
        ("R", ctypes.c_float * 9),
        ("t", ctypes.c_float * 3),
        ("center", ctypes.c_float * 3),
        ("fx", ctypes.c_float),
        ("fy", ctypes.c_float),
        ("cx", ctypes.c_float),
        ("cy", ctypes.c_float),
        ("lim_x", ctypes.c_float),
        ("lim_y", ctypes.c_float),
        ("znear", ctypes.c_float),
        ("width", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("orthographic", ctypes.c_int32),
        ("lens", ctypes.c_int32),
        ("dist", ctypes.c_float * 8),
    ]


ADAM_MAX_GROUPS = 8  # GSX_ADAM_MAX_GROUPS


class GsxAdamGroup(ctypes.Structure):
    """gsx_adam_group of include/gsx.h."""

    _fields_ = [
        ("param", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("m", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("n", ctypes.c_int64),
        ("lr", ctypes.c_float),
    ]


TABLE_MAX = 20  # GSX_TABLE_MAX
ROW_PARAM = 1
ROW_MOMENT = 2


class GsxRowTable(ctypes.Structure):
    """gsx_row_table of include/gsx.h."""

    _fields_ = [
        ("count", ctypes.c_int32),
        ("width", ctypes.c_int32 * TABLE_MAX),
        ("role", ctypes.c_int32 * TABLE_MAX),
        ("src", ctypes.c_void_p * TABLE_MAX),
        ("dst", ctypes.c_void_p * TABLE_MAX),
    ]


def row_table(columns) -> GsxRowTable:
    """GsxRowTable of ``[(src, dst, role), ...]``: (N, ...) float32
    contiguous tensors, width = elements per row."""
    if not 0 < len(columns) <= TABLE_MAX:
        raise ValueError(f"a row table holds 1..{TABLE_MAX} tensors")
    t = GsxRowTable()
    t.count = len(columns)
    for k, (src, dst, role) in enumerate(columns):
        for x in (src, dst):
            if x.dtype != torch.float32 or not x.is_contiguous():
                raise ValueError("row-table tensors must be contiguous float32")
        t.width[k] = int(src[0].numel()) if src.shape[0] else int(dst[0].numel())
        t.role[k] = role
        t.src[k] = src.data_ptr()
        t.dst[k] = dst.data_ptr()
    return t


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_U32 = ctypes.c_uint32
_F = ctypes.c_float
_CAM = ctypes.POINTER(GsxCamera)

# name -> (restype, argtypes); the order follows include/gsx.h.
SIGNATURES = {
    "gsx_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "gsx_abi_version": (ctypes.c_int, []),
    "gsx_device_check": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int]),
    "gsx_project_fwd": (ctypes.c_int, [_CAM, _I64, _P, _P, _P, _F, _I32, _P, _P, _P, _P, _P, _P]),
    "gsx_project_bwd": (ctypes.c_int, [_CAM, _I64, _P, _P, _P, _F, _I32, _P, _P, _P, _P, _P, _P,
                                       _P, _P]),
    "gsx_project_ut_fwd": (ctypes.c_int, [_CAM, _I64, _P, _P, _P, _F, _I32, _P, _P, _P, _P, _P,
                                          _P]),
    "gsx_project_ut_bwd": (ctypes.c_int, [_CAM, _I64, _P, _P, _P, _F, _I32, _P, _P, _P, _P, _P,
                                          _P, _P, _P]),
    "gsx_eval_sh_fwd": (ctypes.c_int, [_I64, _I32, _I32, _I32, _P, _P, _P, _P]),
    "gsx_eval_sh_bwd": (ctypes.c_int, [_I64, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P]),
    "gsx_preprocess_fwd": (ctypes.c_int, [_CAM, _I64, _P, _P, _P, _P, _P, _I64, _P, _I64, _I32,
                                          _I32, _U32, _F, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                          _P]),
    "gsx_preprocess_bwd": (ctypes.c_int, [_CAM, _I64, _P, _P, _P, _P, _P, _I32, _I32, _U32, _F,
                                          _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                                          _P, _I64, _I32, _P]),
    "gsx_bin_prepare": (ctypes.c_int, [_I64, _P, _P, _P, _I32, _I32, _P, _P, _P, _P]),
    "gsx_bin_workspace_bytes": (_I64, [_I64, _I64, _I32]),
    "gsx_bin_sort": (ctypes.c_int, [_I64, _P, _P, _P, _P, _P, _I64, _I32, _I32, _P, _I64, _I64,
                                    _P, _P, ctypes.POINTER(_I64), _P]),
    "gsx_bin_sort_async": (ctypes.c_int, [_I64, _P, _P, _P, _P, _P, _I64, _I32, _I32, _P, _I64,
                                          _I64, _P, _P, _P, _P]),
    "gsx_bin_depth_workspace_bytes": (_I64, [_I64]),
    "gsx_bin_tile_workspace_bytes": (_I64, [_I64, _I32]),
    "gsx_bin_count_async": (ctypes.c_int, [_I64, _P, _P, _P, _I32, _I32, _P, _I64, _P, _P, _P]),
    "gsx_bin_depth_async": (ctypes.c_int, [_I64, _P, _P, _I64, _P, _P, _U32, _P]),
    "gsx_bin_tiles_async": (ctypes.c_int, [_I64, _P, _P, _P, _P, _I64, _I32, _I32, _P, _I64, _P,
                                           _I64, _I64, _P, _P, _P, _P, _U32, _P, _P]),
    "gsx_bin_status_check": (ctypes.c_int, [_P, _I64, ctypes.POINTER(_I64)]),
    "gsx_host_status_alloc": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p)]),
    "gsx_host_status_free": (ctypes.c_int, [_P]),
    "gsx_pack_conic_opacity": (ctypes.c_int, [_I64, _P, _P, _P, _P]),
    "gsx_raster_fwd": (ctypes.c_int, [_I64, _I32, _P, _P, _P, _P, _P, _I64, _P, _P, _I32, _I32,
                                      _P, _P, _P, _P, _P, _P, _I32, _P]),
    "gsx_tile_order_words": (_I64, [_I32, _I32]),
    "gsx_raster_bwd": (ctypes.c_int, [_I64, _I32, _P, _P, _P, _P, _I64, _P, _P, _I32, _I32, _P,
                                      _P, _P, _P, _P, _P, _P, _P, _I32, _P, _P]),
    "gsx_photometric_workspace_bytes": (_I64, [_I32, _I32, _I32]),
    "gsx_photometric_fwd": (ctypes.c_int, [_I32, _I32, _I32, _P, _P, _I32, _F, _F, _P, _I64, _P,
                                           _P]),
    "gsx_photometric_bwd": (ctypes.c_int, [_I32, _I32, _I32, _P, _P, _I32, _F, _P, _I64, _P, _P,
                                           _P]),
    "gsx_photometric_loss_fwd": (ctypes.c_int, [_I32, _I32, _I32, _P, _P, _I32, _F, _F,
                                                ctypes.c_double, _P, _I64, _P, _P]),
    "gsx_photometric_loss_bwd": (ctypes.c_int, [_I32, _I32, _I32, _P, _P, _I32, _F,
                                                ctypes.c_double, _P, _I64, _P, _P, _P]),
    "gsx_l1_workspace_bytes": (_I64, [_I64]),
    "gsx_l1_fwd": (ctypes.c_int, [_I64, _P, _P, _P, _I64, _P, _P]),
    "gsx_l1_noalloc_max_elements": (_I64, []),
    "gsx_l1_fwd_noalloc": (ctypes.c_int, [_I64, _P, _P, _P, _P]),
    "gsx_l1_bwd": (ctypes.c_int, [_I64, _P, _P, _P, _P, _P]),
    "gsx_l1_fwd_signs": (ctypes.c_int, [_I64, _P, _P, _P, _I64, _P, _P, _P]),
    "gsx_l1_bwd_signs": (ctypes.c_int, [_I64, _P, _P, _P, _P, _P, _P]),
    "gsx_adam_step": (ctypes.c_int, [_I32, ctypes.c_void_p, _F, _F, _F, _P]),
    "gsx_preprocess_bwd_adam": (ctypes.c_int, [_CAM, _I64, _P, _P, _P, _P, _P, _P, _P, _I32,
                                               _I32, _U32, _F, _P, _P, _P, _P, _P, _P, _P,
                                               ctypes.c_void_p, _F, _F, _F, _I32, _P]),
    "gsx_accum_screen_grads": (ctypes.c_int, [_I64, _P, _P, _I32, _I32, _P, _P, _I32, _P]),
    "gsx_knn_log_scale": (ctypes.c_int, [_I64, _P, _I64, _P, _I32, _F, _P, _P]),
    "gsx_density_workspace_bytes": (_I64, [_I64]),
    "gsx_density_classify": (ctypes.c_int, [_I64, _P, _P, _P, _P, _F, _F, _F, _F, _P, _I64,
                                            _P, _P]),
    "gsx_density_emit": (ctypes.c_int, [_I64, _P, _I64, _P, ctypes.POINTER(GsxRowTable), _I32,
                                        _I32, _I32, _P, _F, _P]),
    "gsx_relocate_scores": (ctypes.c_int, [_I64, _P, _P, _P, _F, _P, _P, _P, _P]),
    "gsx_density_relocate": (ctypes.c_int, [_I64, _P, _P, ctypes.POINTER(GsxRowTable), _I32,
                                            _I32, _I32, _P, _F, _F, _F, _P, _I64, _P]),
    "gsx_geom_features": (ctypes.c_int, [_I64, _P, _P, _P, _P, _P, _P]),
    "gsx_geom_features_bwd": (ctypes.c_int, [_I64, _P, _P, _P, _P, _P, _P, _P, _P]),
    "gsx_geom_loss_workspace_bytes": (_I64, [_I32, _I32]),
    "gsx_geom_loss_fwd": (ctypes.c_int, [_I32, _I32, _P, _P, _P, _P, _F, _F, _F, _P, _I64, _P,
                                         _P]),
    "gsx_geom_loss_bwd": (ctypes.c_int, [_I32, _I32, _P, _P, _P, _P, _F, _F, _F, _P, _P, _P,
                                         _P]),
    "gsx_mesh_raster": (ctypes.c_int, [_I64, _P, _P, _P, _I64, _P, _I32, _I32, _F, _P, _P, _P]),
    "gsx_debug_expf": (ctypes.c_int, [_I64, _P, _P, _P]),
    "gsx_debug_atanf": (ctypes.c_int, [_I64, _P, _P, _P]),
}

_lib = None
_lock = threading.Lock()


def load():
    """Load libgsx.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"mlx3d_amd: {LIB_PATH} is missing. Build it with "
                    "`python mlx3d_amd/csrc/build.py` (or __graft_entry__.build()); "
                    "there is no fallback compute path.")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def strerror(status: int) -> str:
    return load().gsx_strerror(status).decode()


def check(status: int, what: str) -> int:
    if status < 0:
        raise GsxError(f"{what} failed: {strerror(status)} (status {status})")
    return status


def ptr(t: torch.Tensor | None):
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream_handle(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_device(*tensors: torch.Tensor | None) -> torch.device:
    """All tensors must live on one ROCm GPU (torch device type 'cuda')."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(
                "mlx3d_amd kernels run on the GPU only; got a tensor on "
                f"{t.device}. Move inputs to a ROCm device (e.g. .cuda()).")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor inputs")
    return dev


def f32c(t: torch.Tensor) -> torch.Tensor:
    """float32, contiguous (the layout every entry point expects)."""
    if t.dtype != torch.float32:
        t = t.float()
    return t.contiguous()
