"""Projection + binning + rasterization (``src/mlx3d/splatting/render.py:14-220``).

The render functions run the fused pipeline

    gsx_preprocess_fwd -> gsx_bin_count_async -> gsx_bin_depth_async
        -> gsx_bin_tiles_async -> gsx_raster_fwd -> (read the duplicate count)
    gsx_raster_bwd -> gsx_preprocess_bwd            (backward)

inside one ``torch.autograd.Function``: activations, projection, opacity
compensation, view-dependent SH colour and the tile rectangles are one
kernel per Gaussian, and the backward is the analytic VJP of the same
expressions (what MLX autodiff computes for the reference).
"""

from __future__ import annotations

import ctypes

from dataclasses import dataclass

import torch

from .. import _lib
from ..cameras import Camera
from ..profiling import count, stage
from .rasterize import (background_tensor, raster_backward, raster_forward, t_cotangent,
                        tile_order_buffer)
from .sh import num_sh_bases
from .tiles import BinJob

__all__ = ["render_gaussians", "render_gaussian_depth", "render_gaussian_features"]


@dataclass
class _Cfg:
    cam: object          # GsxCamera
    width: int
    height: int
    flags: int
    blur: float
    degree: int
    K: int
    sh_mode: str | None  # "packed" (N,K,3) tensor, "split" (dc, rest) tensors, None = colours
    return_depth: bool
    refine: bool = False  # refine_tiles: drop bbox tiles the conic never reaches
    # (grad_accum, grad_count): the backward adds the density-control
    # statistics of dL/dmeans2d (trainer.py:357-365) to these in place.
    screen_stats: tuple | None = None
    # optim.FusedAdam: the backward applies this Adam update to the six
    # parameter groups itself (gsx_preprocess_bwd_adam) and returns no
    # parameter gradients
    adam: object | None = None


def _sh_views(cfg: _Cfg, sh_a, sh_b):
    """(sh0 pointer tensor, sh0 stride, sh_rest address, sh_rest stride) in floats."""
    if cfg.sh_mode == "packed":
        s = cfg.K * 3
        rest = sh_a.data_ptr() + 12 if cfg.K > 1 else None
        return sh_a, s, rest, s
    if cfg.sh_mode == "split":
        rest = sh_b.data_ptr() if cfg.K > 1 else None
        return sh_a, 3, rest, 3 * (cfg.K - 1)
    return None, 0, None, 0


def _forward(cfg: _Cfg, means, quats, scales, opacities, sh_a, sh_b, colors, background):
    dev = means.device
    n = means.shape[0]
    f = lambda *s: torch.empty(s, dtype=torch.float32, device=dev)  # noqa: E731
    i = lambda *s: torch.empty(s, dtype=torch.int32, device=dev)  # noqa: E731
    means2d, depths, radii, comp, co = f(n, 2), f(n), f(n), f(n), f(n, 4)
    colors_out = f(n, 3) if cfg.sh_mode else None
    counts, dkeys, rects = i(n), i(n), i(n, 2)
    sh0, s0, shr, sr = _sh_views(cfg, sh_a, sh_b)
    L = _lib.load()
    st = _lib.stream_handle(dev)
    with stage("preprocess_fwd"):
        _lib.check(L.gsx_preprocess_fwd(
            cfg.cam, n, _lib.ptr(means), _lib.ptr(quats), _lib.ptr(scales), _lib.ptr(opacities),
            _lib.ptr(sh0), s0, shr, sr, cfg.K, cfg.degree, cfg.flags, cfg.blur,
            _lib.ptr(means2d), _lib.ptr(depths), _lib.ptr(radii), _lib.ptr(comp), _lib.ptr(co),
            _lib.ptr(colors_out), _lib.ptr(counts), _lib.ptr(dkeys), _lib.ptr(rects), st),
            "gsx_preprocess_fwd")
    feats = colors_out if cfg.sh_mode else colors
    # the binning's placement launch writes the forward's tile order too
    order = tile_order_buffer(cfg.width, cfg.height, dev)
    with stage("binning"):
        job = BinJob(counts, dkeys, rects, cfg.width, cfg.height,
                     refine=(means2d, co) if cfg.refine else None, tile_order=order)

    def raster(ids):
        with stage("raster_fwd"):
            return raster_forward(means2d, co, feats, ids, job.ranges, background, cfg.width,
                                  cfg.height, depths=depths if cfg.return_depth else None,
                                  tile_order=order, order_ready=True)

    # The rasterizer runs on the id buffer (its ranges never reach past D)
    # and is enqueued before the host reads D.  If D exceeded the guessed
    # capacity, the first run saw empty ranges and the binning has been
    # enqueued again with the exact capacity: the rasterizer runs again
    # behind it.  Only refine_tiles needs the final status for D, read after
    # everything has been enqueued.
    image, final_T, n_contrib, depth_map, alpha = raster(job.ids)
    if job.settle():
        image, final_T, n_contrib, depth_map, alpha = raster(job.ids)
    ids, ranges = job.result()
    count("duplicates", ids.shape[0])
    return dict(means2d=means2d, depths=depths, radii=radii, compensation=comp, conic_opac=co,
                feats=feats, sorted_ids=ids, tile_ranges=ranges, image=image, final_T=final_T,
                alpha=alpha, n_contrib=n_contrib, depth=depth_map, job=job, tile_order=order)


class _RenderFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means, quats, scales, opacities, sh_a, sh_b, colors, background, cfg):
        r = _forward(cfg, means, quats, scales, opacities, sh_a, sh_b, colors, background)
        ctx.cfg = cfg
        ctx.bin_job = r["job"]
        ctx.save_for_backward(means, quats, scales, opacities, sh_a, sh_b, r["feats"],
                              r["means2d"], r["conic_opac"], r["sorted_ids"], r["tile_ranges"],
                              r["final_T"], r["n_contrib"], background, r["radii"],
                              r["tile_order"])
        depth = r["depth"] if r["depth"] is not None else r["final_T"].new_empty((0,))
        ctx.mark_non_differentiable(r["radii"], r["n_contrib"], depth, r["sorted_ids"],
                                    r["tile_ranges"])
        ctx.set_materialize_grads(False)  # unused outputs: no zero-filled cotangents
        return (r["image"], r["final_T"], r["alpha"], r["n_contrib"], r["means2d"], r["depths"],
                r["radii"], r["compensation"], depth, r["sorted_ids"], r["tile_ranges"])

    @staticmethod
    def backward(ctx, g_image, g_final_T, g_alpha, _g_nc, g_means2d, g_depths, _g_radii, g_comp,
                 _g_depth, _g_ids, _g_ranges):
        (means, quats, scales, opacities, sh_a, sh_b, feats, means2d, co, ids, ranges, final_T,
         n_contrib, background, radii, order) = ctx.saved_tensors
        cfg = ctx.cfg
        dev = means.device
        n = means.shape[0]
        # The rasterizer's gradients go into one record per Gaussian, which
        # the screen statistics and the preprocess VJP read in place.  A
        # feature render hands its feature gradient to autograd instead: a
        # strided view of the record would be copied there, so it takes the
        # four-array layout (a contiguous (N, C) feature gradient).
        record = bool(cfg.sh_mode) or cfg.adam is not None
        with stage("raster_bwd"):
            r = raster_backward(
                means2d, co, feats, ids, ranges, background, cfg.width, cfg.height, final_T,
                n_contrib, g_image, t_cotangent(g_final_T, g_alpha), record=record,
                tile_order=order)
        if record:
            _, _, g_feat, _, grec, gstride = r
            g_in = (grec, None, None)  # g_means2d (the record), g_conics, g_opac_eff
        else:
            g_m2r, g_con, g_feat, g_op = r
            gstride = 0
            g_in = (g_m2r, g_con, g_op)
        if cfg.screen_stats is not None:
            acc, cnt = cfg.screen_stats
            _lib.check(_lib.load().gsx_accum_screen_grads(
                n, _lib.ptr(g_in[0]), _lib.ptr(radii), cfg.width, cfg.height, _lib.ptr(acc),
                _lib.ptr(cnt), gstride, _lib.stream_handle(dev)), "gsx_accum_screen_grads")
        c = lambda t: None if t is None else _lib.f32c(t)  # noqa: E731
        # The contiguous copies of the output cotangents (a stride-0 expand
        # from .sum() is copied) must outlive the enqueued kernel: only their
        # addresses cross the ABI, so they are bound to locals here.
        gm2_in, gdep_in, gcomp_in = c(g_means2d), c(g_depths), c(g_comp)
        L = _lib.load()
        # The binning's final device status was copied behind it in the
        # forward; a failed device-side check raises here, before any
        # gradient or parameter update is produced.
        ctx.bin_job.check()
        if cfg.adam is not None:
            opt = cfg.adam
            with stage("preprocess_bwd_adam"):
                _lib.check(L.gsx_preprocess_bwd_adam(
                    cfg.cam, n, _lib.ptr(means), _lib.ptr(quats), _lib.ptr(scales),
                    _lib.ptr(opacities), _lib.ptr(sh_a), _lib.ptr(sh_b), _lib.ptr(feats), cfg.K,
                    cfg.degree, cfg.flags, cfg.blur, *[_lib.ptr(t) for t in g_in], None,
                    _lib.ptr(gm2_in), _lib.ptr(gdep_in),
                    _lib.ptr(gcomp_in), ctypes.cast(opt.records, ctypes.c_void_p),
                    opt.betas[0], opt.betas[1], opt.eps, gstride, _lib.stream_handle(dev)),
                    "gsx_preprocess_bwd_adam")
            opt.commit()
            return None, None, None, None, None, None, None, None, None
        f = lambda *s: torch.empty(s, dtype=torch.float32, device=dev)  # noqa: E731
        g_means, g_quats, g_scales, g_opac = f(n, 3), f(n, 4), f(n, 3), f(n)
        g_sh_a = g_sh_b = None
        if cfg.sh_mode:
            g_sh_a = torch.empty_like(sh_a)
            g_sh_b = torch.empty_like(sh_b) if cfg.sh_mode == "split" else None
        gs0, s0, gshr, sr = _sh_views(cfg, g_sh_a, g_sh_b)
        with stage("preprocess_bwd"):
            _lib.check(L.gsx_preprocess_bwd(
                cfg.cam, n, _lib.ptr(means), _lib.ptr(quats), _lib.ptr(scales),
                _lib.ptr(opacities), _lib.ptr(feats if cfg.sh_mode else None), cfg.K, cfg.degree,
                cfg.flags, cfg.blur, *[_lib.ptr(t) for t in g_in], None, _lib.ptr(gm2_in),
                _lib.ptr(gdep_in), _lib.ptr(gcomp_in), _lib.ptr(g_means),
                _lib.ptr(g_quats), _lib.ptr(g_scales), _lib.ptr(g_opac), _lib.ptr(gs0), s0, gshr,
                sr, gstride, _lib.stream_handle(dev)), "gsx_preprocess_bwd")
        g_colors = None if cfg.sh_mode else g_feat
        return g_means, g_quats, g_scales, g_opac, g_sh_a, g_sh_b, g_colors, None, None


def _check_common(projection: str) -> int:
    """Flag bits of the projection (render.py:14-26)."""
    if projection not in ("ewa", "ut"):
        raise ValueError("projection must be 'ewa' or 'ut'.")
    return _lib.PROJECT_UT if projection == "ut" else 0


def _stats(screen_stats, n, dev):
    if screen_stats is None:
        return None
    acc, cnt = screen_stats
    for t in (acc, cnt):
        if t.shape != (n,) or t.dtype != torch.float32 or not t.is_contiguous() or t.device != dev:
            raise ValueError("screen_stats tensors must be contiguous float32 (N,) on the "
                             "render device")
    return acc, cnt


def _run(camera: Camera, means, quats, scales, opacities, *, sh_a=None, sh_b=None,
         sh_mode=None, K=0, degree=0, colors=None, background=None, flags=0, antialias=False,
         blur=0.3, return_depth=False, refine_tiles=False, screen_stats=None, adam=None):
    n = means.shape[0]
    if means.ndim != 2 or means.shape[1] != 3:
        raise ValueError("means must have shape (N, 3).")
    if quats.shape != (n, 4) or scales.shape != (n, 3) or opacities.shape != (n,):
        raise ValueError("quats must be (N, 4), scales (N, 3), opacities (N,).")
    dev = _lib.require_device(means, quats, scales, opacities, sh_a, sh_b, colors)
    channels = 3 if sh_mode else colors.shape[1]
    if antialias:
        flags |= _lib.ANTIALIAS
    cfg = _Cfg(cam=camera.to_gsx(), width=int(camera.width), height=int(camera.height),
               flags=flags, blur=float(blur), degree=int(degree), K=int(K), sh_mode=sh_mode,
               return_depth=bool(return_depth), refine=bool(refine_tiles),
               screen_stats=_stats(screen_stats, n, dev), adam=adam)
    if adam is not None and sh_mode != "split":
        raise ValueError("a fused Adam update needs the split SH layout")
    c = _lib.f32c
    (image, final_T, alpha, n_contrib, means2d, depths, radii, comp, depth, ids,
     ranges) = _RenderFn.apply(c(means), c(quats), c(scales), c(opacities),
                               None if sh_a is None else c(sh_a),
                               None if sh_b is None else c(sh_b),
                               None if colors is None else c(colors),
                               background_tensor(background, channels, dev), cfg)
    out = {"image": image, "alpha": alpha, "final_T": final_T, "n_contrib": n_contrib,
           "means2d": means2d, "depths": depths, "radii": radii, "compensation": comp,
           "sorted_ids": ids, "tile_ranges": ranges}
    if return_depth:
        out["depth"] = depth
    return out


def render_gaussians(camera: Camera, means, quats, scales, opacities, colors=None, sh=None,
                     sh_degree: int = 3, background=None, refine_tiles: bool = False,
                     antialias: bool = False, projection: str = "ewa",
                     return_depth: bool = False) -> dict:
    """Render 3D Gaussians; differentiable end to end (render.py:29-112).

    ``scales`` are activated standard deviations and ``opacities`` in [0, 1].
    Exactly one of ``colors`` (N, 3) or ``sh`` (N, K, 3) is given.  Returns
    ``image``, ``alpha``, ``final_T``, ``n_contrib``, ``means2d``, ``depths``
    (per-Gaussian z), ``radii``, ``compensation``; with ``return_depth`` also
    the per-pixel expected ``depth`` (forward-only, as rasterize_depth).
    """
    if (colors is None) == (sh is None):
        raise ValueError("Provide exactly one of `colors` or `sh`.")
    pflags = _check_common(projection)
    if sh is not None:
        if sh.ndim != 3 or sh.shape[2] != 3 or sh.shape[1] < num_sh_bases(sh_degree):
            raise ValueError(f"sh must have shape (N, K>={num_sh_bases(sh_degree)}, 3).")
        if not 0 <= sh_degree <= 3:
            raise ValueError("sh_degree must be in [0, 3].")
        return _run(camera, means, quats, scales, opacities, sh_a=sh, sh_mode="packed",
                    K=sh.shape[1], degree=sh_degree, background=background, antialias=antialias,
                    return_depth=return_depth, refine_tiles=refine_tiles, flags=pflags)
    if colors.ndim != 2 or colors.shape != (means.shape[0], 3):
        raise ValueError("colors must have shape (N, 3).")
    return _run(camera, means, quats, scales, opacities, colors=colors, background=background,
                antialias=antialias, return_depth=return_depth, refine_tiles=refine_tiles,
                flags=pflags)


def render_gaussian_depth(camera: Camera, means, quats, scales, opacities,
                          refine_tiles: bool = False, antialias: bool = False,
                          projection: str = "ewa") -> dict:
    """Expected depth and alpha, forward only (render.py:115-161)."""
    pflags = _check_common(projection)
    with torch.no_grad():
        dev = _lib.require_device(means)
        ones = torch.zeros((means.shape[0], 1), dtype=torch.float32, device=dev)
        out = _run(camera, means, quats, scales, opacities, colors=ones, antialias=antialias,
                   return_depth=True, refine_tiles=refine_tiles, flags=pflags)
    return {"depth": out["depth"], "alpha": out["alpha"], "final_T": out["final_T"],
            "means2d": out["means2d"], "depths": out["depths"], "radii": out["radii"],
            "compensation": out["compensation"]}


def render_gaussian_features(camera: Camera, means, quats, scales, opacities, features,
                             background=None, normalize: bool = False,
                             refine_tiles: bool = False, antialias: bool = False,
                             projection: str = "ewa", return_depth: bool = False) -> dict:
    """Render (N, C) per-Gaussian features (render.py:164-220).

    ``normalize=True`` divides by alpha (zero where alpha <= 1e-6) and ignores
    the background (rasterize.py:493-500, 537-538).
    """
    if features.ndim != 2:
        raise ValueError("features must have shape (N, C).")
    if features.shape[0] != means.shape[0]:
        raise ValueError("features and means2d must have the same first dimension.")
    channels = int(features.shape[1])
    if channels <= 0:
        raise ValueError("features must contain at least one channel.")
    pflags = _check_common(projection)
    bg = None if normalize else background
    out = _run(camera, means, quats, scales, opacities, colors=features, background=bg,
               antialias=antialias, return_depth=return_depth, refine_tiles=refine_tiles,
               flags=pflags)
    feat = out.pop("image")
    if normalize:
        a = out["alpha"][..., None]
        feat = torch.where(a > 1e-6, feat / torch.clamp(a, min=1e-6), torch.zeros_like(feat))
    out["features"] = feat
    return out
