"""Dense all-pairs renderer, the reference's correctness oracle
(``src/mlx3d/splatting/reference.py:16-74``), exported for API completeness.

Every Gaussian is evaluated at every pixel in one global depth order, so the
cost is O(N H W): tiny scenes only.  The projection is the HIP
``project_gaussians``; the compositing is differentiable torch arithmetic on
the same device, evaluated in bands of pixel rows.  Its rules differ from
the tile rasterizer's in the two places the reference's oracle differs:
the splat that takes the transmittance below 1e-4 is still composited (the
product of the earlier ``1 - alpha`` factors decides), and the 0.99 alpha
clamp passes no gradient while it is active.  It is not on the render
path: ``render_gaussians`` never calls it.
"""

from __future__ import annotations

import torch

from ..cameras import Camera
from .projection import project_gaussians

__all__ = ["render_gaussians_reference"]

# pixels per band: bounds the (N, band) intermediates to about 2^24 floats
_BAND_ELEMS = 1 << 24


def _composite_band(m2, con, opac, colors, live, xs, ys):
    """Front-to-back composite of depth-ordered Gaussians over the pixels
    (xs, ys) (flattened band).  Returns (colour (P, C), transmittance (P,))."""
    dx = m2[:, 0:1] - xs[None, :]
    dy = m2[:, 1:2] - ys[None, :]
    q = con[:, 0:1] * dx * dx + con[:, 2:3] * dy * dy
    power = -0.5 * q - con[:, 1:2] * dx * dy
    a = torch.minimum(opac[:, None] * torch.exp(power), torch.full_like(power, 0.99))
    zero = torch.zeros_like(a)
    a = torch.where(power > 0.0, zero, a)
    a = torch.where(a < 1.0 / 255.0, zero, a)
    a = a * live[:, None]
    one_minus = 1.0 - a
    # transmittance in front of each splat: exclusive cumulative product
    t_front = torch.cumprod(torch.cat([torch.ones_like(one_minus[:1]), one_minus[:-1]], 0), 0)
    reached = (t_front > 1e-4).to(a.dtype)
    w = a * t_front * reached
    colour = w.transpose(0, 1) @ colors
    t_final = torch.prod(torch.where(reached > 0, one_minus, torch.ones_like(one_minus)), 0)
    return colour, t_final


def render_gaussians_reference(camera: Camera, means: torch.Tensor, quats: torch.Tensor,
                               scales: torch.Tensor, opacities: torch.Tensor,
                               colors: torch.Tensor, background=None,
                               antialias: bool = False) -> dict:
    """Dense reference render matching ``render_gaussians`` (reference.py:16-74).

    ``scales`` are standard deviations, ``opacities`` in [0, 1], ``colors``
    (N, C).  Returns ``image`` (H, W, C), ``alpha`` and ``final_T`` (H, W);
    differentiable through torch autograd.
    """
    H, W = int(camera.height), int(camera.width)
    dev = means.device
    C = colors.shape[1]
    bg = (torch.zeros((C,), dtype=torch.float32, device=dev) if background is None
          else torch.as_tensor(background, dtype=torch.float32, device=dev).expand(C))
    proj = project_gaussians(camera, means, quats, scales, antialias=antialias)
    order = torch.argsort(proj["depths"].detach(), stable=True)
    m2 = proj["means2d"][order]
    con = proj["conics"][order]
    opac = (opacities * proj["compensation"])[order]
    cols = colors.to(torch.float32)[order]
    live = (proj["radii"][order] > 0).to(torch.float32)
    n = max(int(means.shape[0]), 1)
    rows = max(1, min(H, _BAND_ELEMS // (n * W)))
    xs_row = torch.arange(W, dtype=torch.float32, device=dev) + 0.5
    images, trans = [], []
    for y0 in range(0, H, rows):
        y1 = min(H, y0 + rows)
        ys = (torch.arange(y0, y1, dtype=torch.float32, device=dev) + 0.5)
        xs = xs_row.repeat(y1 - y0)
        yy = ys.repeat_interleave(W)
        colour, t_final = _composite_band(m2, con, opac, cols, live, xs, yy)
        images.append(colour + t_final[:, None] * bg[None, :])
        trans.append(t_final)
    image = torch.cat(images, 0).reshape(H, W, C)
    final_T = torch.cat(trans, 0).reshape(H, W)
    return {"image": image, "alpha": 1.0 - final_T, "final_T": final_T}
