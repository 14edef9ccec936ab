"""Tile-based alpha compositing (``src/mlx3d/splatting/rasterize.py:406-578``).

``rasterize`` / ``rasterize_features`` are differentiable through a
``torch.autograd.Function`` (the stand-in for the reference's
``mx.custom_function`` + ``.vjp``, rasterize.py:345-403) whose forward and
backward are the HIP kernels ``gsx_raster_fwd`` / ``gsx_raster_bwd``.
Features of any channel count composite in one pass (the reference runs
one RGB kernel per 3 channels, rasterize.py:502-532; the per-channel
arithmetic is identical).  ``rasterize_depth`` is forward-only, as in the
reference.
"""

from __future__ import annotations

import torch

from .. import _lib
from .tiles import TILE_SIZE

__all__ = ["rasterize", "rasterize_depth", "rasterize_features"]


def _empty(shape, dev, dtype=torch.float32):
    return torch.empty(shape, dtype=dtype, device=dev)


def tile_order_buffer(width, height, dev):
    """The rasterizers' tile-order buffer for a width x height image
    (gsx_tile_order_words int32 words): each call writes its tile order
    (heaviest tiles first within each XCD's band of tiles), the forward
    also the per-tile contributor bounds that the backward of the same frame
    orders by."""
    return _empty((int(_lib.load().gsx_tile_order_words(width, height)),), dev, torch.int32)


def raster_forward(means2d, conic_opac, feats, sorted_ids, tile_ranges, background, width,
                   height, depths=None, tile_order=None, order_ready=False):
    """gsx_raster_fwd on prepared float32 contiguous tensors (no autograd):
    (out, final_T, n_contrib, depth_map or None, alpha = 1 - final_T).
    With ``tile_order`` (tile_order_buffer) the workgroups take the tiles
    with the longest lists first, and the kernel records each tile's
    contributor bound there, which raster_backward orders its tiles by;
    ``order_ready``: the binning already wrote this frame's order there."""
    dev = means2d.device
    n, C = feats.shape
    out = _empty((height, width, C), dev)
    final_T = _empty((height, width), dev)
    alpha = _empty((height, width), dev)
    n_contrib = _empty((height, width), dev, torch.int32)
    depth_map = _empty((height, width), dev) if depths is not None else None
    L = _lib.load()
    _lib.check(L.gsx_raster_fwd(n, C, _lib.ptr(means2d), _lib.ptr(conic_opac), _lib.ptr(feats),
                                _lib.ptr(depths), _lib.ptr(sorted_ids), sorted_ids.numel(),
                                _lib.ptr(tile_ranges),
                                _lib.ptr(background), width, height, _lib.ptr(out),
                                _lib.ptr(final_T), _lib.ptr(n_contrib), _lib.ptr(depth_map),
                                _lib.ptr(alpha), _lib.ptr(tile_order),
                                1 if (order_ready and tile_order is not None) else 0,
                                _lib.stream_handle(dev)),
               "gsx_raster_fwd")
    return out, final_T, n_contrib, depth_map, alpha


def t_cotangent(g_final_T, g_alpha):
    """Cotangent of final_T when alpha = 1 - final_T is an output too."""
    if g_alpha is None:
        return g_final_T
    return -g_alpha if g_final_T is None else g_final_T - g_alpha


def grad_record_stride(C: int) -> int:
    """Floats per Gaussian of the rasterizer's gradient record: means2d (2),
    conic (3), opacity (1), C features, padded to whole 16-byte groups (at
    least 12, which the preprocess VJP reads)."""
    return max(12, 4 * ((6 + C + 3) // 4))


def raster_backward(means2d, conic_opac, feats, sorted_ids, tile_ranges, background, width,
                    height, final_T, n_contrib, g_out, g_final_T, record: bool = False,
                    tile_order=None):
    """gsx_raster_bwd: gradients w.r.t. means2d, conics, features, opacity.
    ``tile_order``: the buffer the frame's raster_forward filled, or None.

    With ``record`` the kernel accumulates into one (N, stride) record per
    Gaussian (its atomics for a Gaussian then share a cache line or two);
    the four gradients are returned as strided views of it, and the record
    and its stride as two more values."""
    dev = means2d.device
    n, C = feats.shape
    if record:
        stride = grad_record_stride(C)
        rec = _empty((n, stride), dev)
        g_m, g_c, g_o, g_f = rec[:, 0:2], rec[:, 2:5], rec[:, 5], rec[:, 6:6 + C]
        outs = (rec, None, None, None)
    else:
        stride = 0
        g_m = _empty((n, 2), dev)
        g_c = _empty((n, 3), dev)
        g_f = _empty((n, C), dev)
        g_o = _empty((n,), dev)
        outs = (g_m, g_c, g_f, g_o)
    if g_out is None:
        g_out = torch.zeros((height, width, C), dtype=torch.float32, device=dev)
    g_out = _lib.f32c(g_out)
    g_final_T = None if g_final_T is None else _lib.f32c(g_final_T)
    L = _lib.load()
    _lib.check(L.gsx_raster_bwd(n, C, _lib.ptr(means2d), _lib.ptr(conic_opac), _lib.ptr(feats),
                                _lib.ptr(sorted_ids), sorted_ids.numel(), _lib.ptr(tile_ranges),
                                _lib.ptr(background),
                                width, height, _lib.ptr(final_T), _lib.ptr(n_contrib),
                                _lib.ptr(g_out), _lib.ptr(g_final_T), *[_lib.ptr(t) for t in outs],
                                stride, _lib.ptr(tile_order), _lib.stream_handle(dev)),
               "gsx_raster_bwd")
    if record:
        return g_m, g_c, g_f, g_o, rec, stride
    return g_m, g_c, g_f, g_o


def pack_conic_opacity(conics, opacities):
    dev = conics.device
    n = conics.shape[0]
    co = _empty((n, 4), dev)
    L = _lib.load()
    _lib.check(L.gsx_pack_conic_opacity(n, _lib.ptr(conics), _lib.ptr(opacities), _lib.ptr(co),
                                        _lib.stream_handle(dev)), "gsx_pack_conic_opacity")
    return co


class _Rasterize(torch.autograd.Function):
    @staticmethod
    def forward(ctx, means2d, conics, feats, opacities, sorted_ids, tile_ranges, background,
                width, height):
        _lib.require_device(means2d, conics, feats, opacities, sorted_ids, tile_ranges, background)
        co = pack_conic_opacity(conics, opacities)
        order = tile_order_buffer(width, height, means2d.device)
        out, final_T, n_contrib, _, alpha = raster_forward(means2d, co, feats, sorted_ids,
                                                           tile_ranges, background, width, height,
                                                           tile_order=order)
        ctx.save_for_backward(means2d, co, feats, sorted_ids, tile_ranges, background, final_T,
                              n_contrib, order)
        ctx.size = (width, height)
        ctx.mark_non_differentiable(n_contrib)
        ctx.set_materialize_grads(False)  # unused outputs: no zero-filled cotangents
        return out, final_T, alpha, n_contrib

    @staticmethod
    def backward(ctx, g_out, g_final_T, g_alpha, _g_nc):
        means2d, co, feats, ids, ranges, bg, final_T, n_contrib, order = ctx.saved_tensors
        width, height = ctx.size
        g_m, g_c, g_f, g_o = raster_backward(means2d, co, feats, ids, ranges, bg, width, height,
                                             final_T, n_contrib, g_out,
                                             t_cotangent(g_final_T, g_alpha), tile_order=order)
        return g_m, g_c, g_f, g_o, None, None, None, None, None


def _check_grid(width, height, tiles_x, tiles_y):
    if tiles_x != (width + TILE_SIZE - 1) // TILE_SIZE or tiles_y != (height + TILE_SIZE - 1) // TILE_SIZE:
        raise ValueError("tiles_x/tiles_y do not match the image size.")


def _ids(t):
    return t.to(torch.int32).contiguous()


def background_tensor(background, channels: int, dev):
    """None (a zero background: the kernels read NULL) or a contiguous float32
    (channels,) tensor; a scalar is broadcast to every channel.  The kernels
    read one background value per channel, so any other shape is refused
    (rasterize.py:428-429, 493-500)."""
    if background is None:
        return None
    bg = torch.as_tensor(background, dtype=torch.float32, device=dev)
    if bg.ndim == 0:
        bg = bg.expand(channels)
    if bg.shape != (channels,):
        raise ValueError(f"background must have shape ({channels},).")
    return bg.contiguous()


def rasterize(means2d, conics, colors, opacities, sorted_ids, tile_ranges, width: int,
              height: int, tiles_x: int, tiles_y: int, background=None) -> dict:
    """Alpha-composite binned 2D Gaussians into an image (rasterize.py:406-446).

    Returns ``image`` (H, W, 3), ``alpha`` (H, W) = 1 - final_T, and the
    saved ``final_T`` / ``n_contrib`` buffers.
    """
    _check_grid(width, height, tiles_x, tiles_y)
    dev = means2d.device
    if colors.ndim != 2:
        raise ValueError("colors must have shape (N, C).")
    bg = background_tensor(background, int(colors.shape[1]), dev)
    image, final_T, alpha, n_contrib = _Rasterize.apply(
        _lib.f32c(means2d), _lib.f32c(conics), _lib.f32c(colors), _lib.f32c(opacities),
        _ids(sorted_ids), _ids(tile_ranges), bg, int(width), int(height))
    return {"image": image, "alpha": alpha, "final_T": final_T, "n_contrib": n_contrib}


def rasterize_features(means2d, conics, features, opacities, sorted_ids, tile_ranges,
                       width: int, height: int, tiles_x: int, tiles_y: int, background=None,
                       normalize: bool = False) -> dict:
    """Alpha-composite arbitrary (N, C) feature channels (rasterize.py:449-545).

    ``normalize=True`` returns ``sum_i alpha_i T_i f_i / alpha`` (zero where
    alpha <= 1e-6) and ignores ``background``.
    """
    if features.ndim != 2:
        raise ValueError("features must have shape (N, C).")
    if features.shape[0] != means2d.shape[0]:
        raise ValueError("features and means2d must have the same first dimension.")
    channels = int(features.shape[1])
    if channels <= 0:
        raise ValueError("features must contain at least one channel.")
    _check_grid(width, height, tiles_x, tiles_y)
    dev = means2d.device
    bg = None if normalize else background_tensor(background, channels, dev)
    feat, final_T, alpha, n_contrib = _Rasterize.apply(
        _lib.f32c(means2d), _lib.f32c(conics), _lib.f32c(features), _lib.f32c(opacities),
        _ids(sorted_ids), _ids(tile_ranges), bg, int(width), int(height))
    if normalize:
        a = alpha[..., None]
        feat = torch.where(a > 1e-6, feat / torch.clamp(a, min=1e-6), torch.zeros_like(feat))
    return {"features": feat, "alpha": alpha, "final_T": final_T, "n_contrib": n_contrib}


def rasterize_depth(means2d, conics, opacities, depths, sorted_ids, tile_ranges, width: int,
                    height: int, tiles_x: int, tiles_y: int) -> dict:
    """Forward-only expected depth (rasterize.py:548-578): ``depth`` (H, W),
    ``alpha``, ``final_T``.  Same termination rule as the colour kernel."""
    _check_grid(width, height, tiles_x, tiles_y)
    with torch.no_grad():
        _lib.require_device(means2d, conics, opacities, depths, sorted_ids, tile_ranges)
        d = _lib.f32c(depths)
        co = pack_conic_opacity(_lib.f32c(conics), _lib.f32c(opacities))
        _, final_T, _, depth, alpha = raster_forward(_lib.f32c(means2d), co,
                                                     d[:, None].contiguous(), _ids(sorted_ids),
                                                     _ids(tile_ranges), None, width, height,
                                                     depths=d,
                                                     tile_order=tile_order_buffer(
                                                         width, height, means2d.device))
    return {"depth": depth, "alpha": alpha, "final_T": final_T}
