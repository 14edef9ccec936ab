"""numpy/ctypes front end of the CPU oracle (``libgsx_oracle.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, by ``bench.py``'s
``cpu_baseline`` leg and by ``__graft_entry__.smoke()`` as the checker.  The
product package ``mlx3d_amd`` never imports this module.

Every function takes and returns float32/int32 numpy arrays on the host and
mirrors the reference function named in ``gsx_oracle.h``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libgsx_oracle.so")
_lib = None

LOG_SCALES = 1
LOGIT_OPACITY = 2
ANTIALIAS = 4
PROJECT_UT = 8


class OrcCamera(ctypes.Structure):
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


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc + OpenMP)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "all"], cwd=_HERE, check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_U32 = ctypes.c_uint32


def _declare(L):
    L.orc_expf.argtypes = [_F]
    L.orc_expf.restype = _F
    L.orc_expf_array.argtypes = [_I64, _P, _P]
    L.orc_splat_expf_array.argtypes = [_I64, _P, _P]
    L.orc_splat_power.argtypes = [_F, _F, _F, _F, _F]
    L.orc_splat_power.restype = _F
    L.orc_project.argtypes = [_P, _I64, _P, _P, _P, _F, _I, _P, _P, _P, _P, _P, _I]
    L.orc_project_bwd.argtypes = [_P, _I64, _P, _P, _P, _F, _I, _P, _P, _P, _P, _P, _P, _P, _I]
    L.orc_eval_sh.argtypes = [_I64, _I, _I, _I, _P, _P, _P, _I]
    L.orc_eval_sh_bwd.argtypes = [_I64, _I, _I, _I, _P, _P, _P, _P, _P, _I]
    L.orc_preprocess_fwd.argtypes = [_P, _I64, _P, _P, _P, _P, _P, _I, _I, _U32, _F,
                                     _P, _P, _P, _P, _P, _P, _P, _I]
    L.orc_preprocess_bwd.argtypes = [_P, _I64, _P, _P, _P, _P, _P, _I, _I, _U32, _F,
                                     _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I]
    L.orc_bin.argtypes = [_I64, _P, _P, _P, _P, _I64, _I, _I, _P, _I64, _P, _I]
    L.orc_bin.restype = _I64
    L.orc_raster_fwd.argtypes = [_I64, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I,
                                 _P, _P, _P, _P, _P, _I64, _I]
    L.orc_raster_fwd_arith.argtypes = L.orc_raster_fwd.argtypes + [_I]
    L.orc_literal_power.argtypes = [_F, _F, _F, _F, _F]
    L.orc_literal_power.restype = _F
    L.orc_raster_bwd.argtypes = [_I64, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _P, _P,
                                 _P, _P, _P, _P, _P, _P, _I]
    L.orc_atanf.argtypes = [_F]
    L.orc_atanf.restype = _F
    L.orc_project_ut.argtypes = [_P, _I64, _P, _P, _P, _F, _I, _P, _P, _P, _P, _P, _I]
    L.orc_project_ut_bwd.argtypes = [_P, _I64, _P, _P, _P, _F, _I, _P, _P, _P, _P, _P, _P, _P,
                                     _I]
    L.orc_mesh_raster.argtypes = [_I64, _P, _P, _P, _P, _I, _I, _F, _P, _P, _I]
    _D = ctypes.c_double
    L.orc_photometric.argtypes = [_I, _I, _I, _P, _P, _I, _D, _D, _D, _D, _P, _P]
    L.orc_adam.argtypes = [_I64, _P, _P, _P, _P, _F, _F, _F, _F]
    L.orc_accum_screen_grads.argtypes = [_I64, _P, _P, _I, _I, _P, _P]


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _i32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def default_threads() -> int:
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def make_camera(R, t, center, fx, fy, cx, cy, lim_x, lim_y, znear, width, height,
                orthographic=0, lens=0, dist=None) -> OrcCamera:
    cam = OrcCamera()
    cam.R[:] = [float(v) for v in np.asarray(R, np.float32).reshape(9)]
    cam.t[:] = [float(v) for v in np.asarray(t, np.float32).reshape(3)]
    cam.center[:] = [float(v) for v in np.asarray(center, np.float32).reshape(3)]
    cam.fx, cam.fy, cam.cx, cam.cy = fx, fy, cx, cy
    cam.lim_x, cam.lim_y, cam.znear = lim_x, lim_y, znear
    cam.width, cam.height = int(width), int(height)
    cam.orthographic, cam.lens = int(orthographic), int(lens)
    cam.dist[:] = [float(v) for v in (dist if dist is not None else [0.0] * 8)]
    return cam


def expf(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_expf_array(x.size, _ptr(x), _ptr(y))
    return y


def splat_expf(x):
    """The compositing loops' exp (orc_splat_expf)."""
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_splat_expf_array(x.size, _ptr(x), _ptr(y))
    return y


def splat_power(a, b, c, dx, dy):
    """The compositing loops' power for one (conic, offset) (orc_splat_power)."""
    return float(lib().orc_splat_power(a, b, c, dx, dy))


def project(cam, means, quats, scales, blur=0.3, antialias=False, threads=1):
    means, quats, scales = _f32(means), _f32(quats), _f32(scales)
    n = means.shape[0]
    out = dict(
        means2d=np.empty((n, 2), np.float32),
        conics=np.empty((n, 3), np.float32),
        depths=np.empty((n,), np.float32),
        radii=np.empty((n,), np.float32),
        compensation=np.empty((n,), np.float32),
    )
    lib().orc_project(ctypes.byref(cam), n, _ptr(means), _ptr(quats), _ptr(scales), blur,
                      int(antialias), _ptr(out["means2d"]), _ptr(out["conics"]),
                      _ptr(out["depths"]), _ptr(out["radii"]), _ptr(out["compensation"]),
                      threads)
    return out


def project_bwd(cam, means, quats, scales, g_means2d=None, g_conics=None, g_depths=None,
                g_comp=None, blur=0.3, antialias=False, threads=1, ut=False):
    means, quats, scales = _f32(means), _f32(quats), _f32(scales)
    n = means.shape[0]
    gm = np.empty((n, 3), np.float32)
    gq = np.empty((n, 4), np.float32)
    gs = np.empty((n, 3), np.float32)
    conv = [None if a is None else _f32(a) for a in (g_means2d, g_conics, g_depths, g_comp)]
    fn = lib().orc_project_ut_bwd if ut else lib().orc_project_bwd
    fn(ctypes.byref(cam), n, _ptr(means), _ptr(quats), _ptr(scales), blur, int(antialias),
       *[_ptr(a) for a in conv], _ptr(gm), _ptr(gq), _ptr(gs), threads)
    return gm, gq, gs


def atanf(r):
    """The oracle's arctan (r >= 0), element by element."""
    return np.array([lib().orc_atanf(float(v)) for v in np.asarray(r, np.float32).ravel()],
                    np.float32).reshape(np.shape(r))


def project_ut(cam, means, quats, scales, blur=0.3, antialias=False, threads=1):
    """project_gaussians_ut (projection.py:149-205)."""
    means, quats, scales = _f32(means), _f32(quats), _f32(scales)
    n = means.shape[0]
    out = dict(
        means2d=np.empty((n, 2), np.float32),
        conics=np.empty((n, 3), np.float32),
        depths=np.empty((n,), np.float32),
        radii=np.empty((n,), np.float32),
        compensation=np.empty((n,), np.float32),
    )
    lib().orc_project_ut(ctypes.byref(cam), n, _ptr(means), _ptr(quats), _ptr(scales), blur,
                         int(antialias), _ptr(out["means2d"]), _ptr(out["conics"]),
                         _ptr(out["depths"]), _ptr(out["radii"]), _ptr(out["compensation"]),
                         threads)
    return out


def eval_sh(degree, sh, dirs, threads=1):
    sh, dirs = _f32(sh), _f32(dirs)
    n, K, C = sh.shape
    out = np.empty((n, C), np.float32)
    lib().orc_eval_sh(n, K, C, degree, _ptr(sh), _ptr(dirs), _ptr(out), threads)
    return out


def eval_sh_bwd(degree, sh, dirs, g_out, threads=1):
    sh, dirs, g_out = _f32(sh), _f32(dirs), _f32(g_out)
    n, K, C = sh.shape
    g_sh = np.empty_like(sh)
    g_dirs = np.empty((n, 3), np.float32)
    lib().orc_eval_sh_bwd(n, K, C, degree, _ptr(sh), _ptr(dirs), _ptr(g_out), _ptr(g_sh),
                          _ptr(g_dirs), threads)
    return g_sh, g_dirs


def preprocess_fwd(cam, means, quats, scales, opacities, sh=None, degree=0, flags=0,
                   blur=0.3, threads=1):
    means, quats, scales, opacities = map(_f32, (means, quats, scales, opacities))
    n = means.shape[0]
    K = 0
    if sh is not None:
        sh = _f32(sh)
        K = sh.shape[1]
    out = dict(
        means2d=np.empty((n, 2), np.float32),
        conics=np.empty((n, 3), np.float32),
        depths=np.empty((n,), np.float32),
        radii=np.empty((n,), np.float32),
        compensation=np.empty((n,), np.float32),
        opac_eff=np.empty((n,), np.float32),
        colors=np.empty((n, 3), np.float32) if sh is not None else None,
    )
    lib().orc_preprocess_fwd(ctypes.byref(cam), n, _ptr(means), _ptr(quats), _ptr(scales),
                             _ptr(opacities), _ptr(sh), K, degree, flags, blur,
                             _ptr(out["means2d"]), _ptr(out["conics"]), _ptr(out["depths"]),
                             _ptr(out["radii"]), _ptr(out["compensation"]),
                             _ptr(out["opac_eff"]), _ptr(out["colors"]), threads)
    return out


def preprocess_bwd(cam, means, quats, scales, opacities, colors_out, K, degree, flags,
                   g_means2d, g_conics, g_opac_eff, g_colors, g_depths=None, g_comp=None,
                   blur=0.3, threads=1):
    means, quats, scales, opacities = map(_f32, (means, quats, scales, opacities))
    n = means.shape[0]
    conv = [None if a is None else _f32(a)
            for a in (colors_out, g_means2d, g_conics, g_opac_eff, g_colors, g_depths, g_comp)]
    gm = np.empty((n, 3), np.float32)
    gq = np.empty((n, 4), np.float32)
    gs = np.empty((n, 3), np.float32)
    go = np.empty((n,), np.float32)
    gsh = np.empty((n, K, 3), np.float32) if colors_out is not None else None
    lib().orc_preprocess_bwd(ctypes.byref(cam), n, _ptr(means), _ptr(quats), _ptr(scales),
                             _ptr(opacities), _ptr(conv[0]), K, degree, flags, blur,
                             *[_ptr(a) for a in conv[1:]], _ptr(gm), _ptr(gq), _ptr(gs),
                             _ptr(go), _ptr(gsh), threads)
    return dict(means=gm, quats=gq, scales=gs, opacities=go, sh=gsh)


def bin_gaussians(means2d, radii, depths, width, height, threads=1, conics=None):
    """tiles.py:19-182; with ``conics`` (N,3) the refine_tiles pass (:91-164)."""
    means2d, radii, depths = _f32(means2d), _f32(radii), _f32(depths)
    n = means2d.shape[0]
    co = None if conics is None else _f32(conics)
    cs = 0 if co is None else co.shape[1]
    tx, ty = (width + 15) // 16, (height + 15) // 16
    ranges = np.empty((tx * ty, 2), np.int32)
    D = lib().orc_bin(n, _ptr(means2d), _ptr(radii), _ptr(depths), _ptr(co), cs, width, height,
                      None, 0, _ptr(ranges), threads)
    ids = np.empty((max(D, 0),), np.int32)
    if D > 0:
        D2 = lib().orc_bin(n, _ptr(means2d), _ptr(radii), _ptr(depths), _ptr(co), cs, width,
                           height, _ptr(ids), D, _ptr(ranges), threads)
        assert D2 == D
    return ids, ranges, tx, ty


# arithmetic variants of raster_fwd (gsx_oracle.h ORC_ARITH_*): the
# reference's literal expressions, for measurement only
ARITH_LITERAL_POWER, ARITH_SEPARATE_ACC, ARITH_ROUNDED_EXP = 1, 2, 4


def literal_power(a, b, c, dx, dy):
    """rasterize.py:75-76's power as written, op by op in float32."""
    return lib().orc_literal_power(a, b, c, dx, dy)


def raster_fwd(means2d, conics, opacities, feats, sorted_ids, tile_ranges, width, height,
               bg=None, depths=None, tiles=None, threads=1, arith=0):
    means2d, conics, opacities, feats = map(_f32, (means2d, conics, opacities, feats))
    sorted_ids, tile_ranges = _i32(sorted_ids), _i32(tile_ranges)
    n, C = feats.shape
    bg = None if bg is None else _f32(bg)
    depths = None if depths is None else _f32(depths)
    tiles = None if tiles is None else _i32(tiles)
    out = np.zeros((height, width, C), np.float32)
    final_T = np.zeros((height, width), np.float32)
    n_contrib = np.zeros((height, width), np.int32)
    depth_out = np.zeros((height, width), np.float32) if depths is not None else None
    lib().orc_raster_fwd_arith(n, C, _ptr(means2d), _ptr(conics), _ptr(opacities),
                               _ptr(feats), _ptr(depths), _ptr(sorted_ids), _ptr(tile_ranges),
                               _ptr(bg), width, height, _ptr(out), _ptr(final_T),
                               _ptr(n_contrib), _ptr(depth_out), _ptr(tiles),
                               0 if tiles is None else tiles.size, threads, int(arith))
    return dict(image=out, final_T=final_T, n_contrib=n_contrib, depth=depth_out)


def raster_bwd(means2d, conics, opacities, feats, sorted_ids, tile_ranges, width, height,
               final_T, n_contrib, grad_out, grad_final_T=None, bg=None, threads=1):
    means2d, conics, opacities, feats = map(_f32, (means2d, conics, opacities, feats))
    sorted_ids, tile_ranges = _i32(sorted_ids), _i32(tile_ranges)
    final_T, n_contrib, grad_out = _f32(final_T), _i32(n_contrib), _f32(grad_out)
    grad_final_T = None if grad_final_T is None else _f32(grad_final_T)
    bg = None if bg is None else _f32(bg)
    n, C = feats.shape
    g_m = np.empty((n, 2), np.float32)
    g_c = np.empty((n, 3), np.float32)
    g_f = np.empty((n, C), np.float32)
    g_o = np.empty((n,), np.float32)
    lib().orc_raster_bwd(n, C, _ptr(means2d), _ptr(conics), _ptr(opacities), _ptr(feats),
                         _ptr(sorted_ids), _ptr(tile_ranges), _ptr(bg), width, height,
                         _ptr(final_T), _ptr(n_contrib), _ptr(grad_out), _ptr(grad_final_T),
                         _ptr(g_m), _ptr(g_c), _ptr(g_f), _ptr(g_o), threads)
    return dict(means2d=g_m, conics=g_c, features=g_f, opacities=g_o)


# ------------------------------------------------------------ training step


def photometric(pred, target, window_size=11, sigma=1.5, max_val=1.0, g_l1=0.0, g_ssim=0.0,
                grad=False):
    """(mean L1, mean SSIM[, gradient]) of (H, W, C) images in float64
    (losses/image_metrics.py:23-55, 66-85; trainer.py:303)."""
    pred, target = _f32(pred), _f32(target)
    if pred.ndim == 2:
        pred, target = pred[..., None], target[..., None]
    H, W, C = pred.shape
    out = np.zeros(2, np.float64)
    g = np.zeros(pred.shape, np.float64) if grad else None
    lib().orc_photometric(H, W, C, _ptr(pred), _ptr(target), int(window_size), float(sigma),
                          float(max_val), float(g_l1), float(g_ssim), _ptr(out), _ptr(g))
    return (out[0], out[1], g) if grad else (out[0], out[1])


def adam(param, grad, m, v, lr, beta1=0.9, beta2=0.999, eps=1e-15):
    """One mlx.optimizers.Adam update (bias_correction off); returns new
    (param, m, v) as float32 arrays."""
    p, m, v = _f32(param).copy(), _f32(m).copy(), _f32(v).copy()
    g = _f32(grad)
    lib().orc_adam(p.size, _ptr(p), _ptr(g), _ptr(m), _ptr(v), float(np.float32(lr)),
                   float(np.float32(beta1)), float(np.float32(beta2)), float(np.float32(eps)))
    return p, m, v


def accum_screen_grads(g_means2d, radii, width, height, accum, count):
    """trainer.py:357-365; returns new (accum, count)."""
    g, r = _f32(g_means2d), _f32(radii)
    a, c = _f32(accum).copy(), _f32(count).copy()
    lib().orc_accum_screen_grads(r.size, _ptr(g), _ptr(r), int(width), int(height), _ptr(a),
                                 _ptr(c))
    return a, c


# ------------------------------------------------------------- mesh raster


def mesh_raster(tri_xy, tri_z, sorted_ids, tile_ranges, width, height, znear=0.01, threads=1):
    """(pix_to_face (H, W) int32, zbuf (H, W)) of renderer/rasterizer.py:29-87."""
    tri_xy, tri_z = _f32(tri_xy).reshape(-1, 6), _f32(tri_z).reshape(-1, 3)
    ids, ranges = _i32(sorted_ids), _i32(tile_ranges)
    p2f = np.empty((height, width), np.int32)
    zb = np.empty((height, width), np.float32)
    lib().orc_mesh_raster(tri_xy.shape[0], _ptr(tri_xy), _ptr(tri_z), _ptr(ids), _ptr(ranges),
                          int(width), int(height), float(np.float32(znear)), _ptr(p2f),
                          _ptr(zb), threads)
    return p2f, zb
