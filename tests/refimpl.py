"""Independent float64 restatements used to pin the CPU oracle.

None of these reuse the oracle's code path: projection is the explicit
matrix form J R Sigma R^T J^T of the reference's own test
(tests/test_splatting.py:114-165), SH basis values come from
scipy.special.sph_harm, binning is a brute-force enumerate-and-sort, and
compositing is the dense all-Gaussians-at-all-pixels form of
src/mlx3d/splatting/reference.py:16-74 (optionally restricted to the tiles
each Gaussian is binned to and to the kernel's termination rule).  Torch
float64 autograd through these gives reference gradients.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from mlx3d_amd.cameras import Camera

TILE = 16


# ------------------------------------------------------------------ scenes
def random_scene(seed=0, n=300, width=96, height=64, fov=50.0, eye=(0.0, 0.0, -4.0)):
    """The reference's random_scene fixture (test_splatting.py:30-40), with
    numpy's PCG64 in place of MLX's RNG."""
    rng = np.random.default_rng(seed)
    means = (rng.standard_normal((n, 3)) * 0.5).astype(np.float32)
    quats = rng.standard_normal((n, 4)).astype(np.float32)
    scales = np.exp(rng.standard_normal((n, 3)) * 0.3 - 2.5).astype(np.float32)
    opac = (1.0 / (1.0 + np.exp(-rng.standard_normal(n)))).astype(np.float32)
    colors = rng.uniform(size=(n, 3)).astype(np.float32)
    cam = Camera.look_at(eye=eye, at=(0, 0, 0), width=width, height=height, fov=fov)
    return cam, means, quats, scales, opac, colors


def oracle_camera(cam: Camera):
    from oracle import oracle as O

    f = cam.gsx_fields()
    return O.make_camera(f["R"], f["t"], f["center"], f["fx"], f["fy"], f["cx"], f["cy"],
                         f["lim_x"], f["lim_y"], f["znear"], f["width"], f["height"],
                         f["orthographic"], f["lens"], f["dist"])


# -------------------------------------------------------------- projection
def quat_to_rot_f64(q: torch.Tensor) -> torch.Tensor:
    q = q / torch.linalg.norm(q, dim=-1, keepdim=True)
    w, x, y, z = q.unbind(-1)
    return torch.stack([
        torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], -1),
        torch.stack([2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)], -1),
        torch.stack([2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1),
    ], -2)


def project_matrix_f64(cam: Camera, means, quats, scales, blur=0.3, antialias=False):
    """EWA projection in explicit matrix form, float64, differentiable."""
    f = cam.gsx_fields()
    R = torch.tensor(f["R"], dtype=torch.float64).reshape(3, 3)
    t = torch.tensor(f["t"], dtype=torch.float64)
    fx, fy, cx, cy = cam.fx, cam.fy, cam.cx, cam.cy
    p = means @ R.T + t
    x, y, z = p.unbind(-1)
    zs = torch.clamp(z, min=1e-6)
    u = fx * x / zs + cx
    v = fy * y / zs + cy
    limx = 1.3 * 0.5 * cam.width / fx
    limy = 1.3 * 0.5 * cam.height / fy
    tx = torch.clamp(x / zs, -limx, limx) * zs
    ty = torch.clamp(y / zs, -limy, limy) * zs
    zero = torch.zeros_like(zs)
    J = torch.stack([torch.stack([fx / zs, zero, -fx * tx / zs ** 2], -1),
                     torch.stack([zero, fy / zs, -fy * ty / zs ** 2], -1)], -2)
    Rq = quat_to_rot_f64(quats)
    M = Rq * scales[:, None, :]
    cov3 = M @ M.transpose(-1, -2)
    T = J @ R
    cov2 = T @ cov3 @ T.transpose(-1, -2)
    a0, b, c0 = cov2[:, 0, 0], cov2[:, 0, 1], cov2[:, 1, 1]
    a, c = a0 + blur, c0 + blur
    det = a * c - b * b
    ds = torch.clamp(det, min=1e-12)
    conics = torch.stack([c / ds, -b / ds, a / ds], -1)
    if antialias and blur > 0:
        comp = torch.sqrt(torch.clamp(a0 * c0 - b * b, min=0.0) / ds)
    else:
        comp = torch.ones_like(det)
    mid = 0.5 * (a + c)
    lam1 = mid + torch.sqrt(torch.clamp(mid * mid - det, min=0.01))
    radii = torch.ceil(3.0 * torch.sqrt(torch.clamp(lam1, min=0.0)))
    valid = (z > cam.znear) & (det > 0)
    radii = torch.where(valid, radii, torch.zeros_like(radii))
    comp = torch.where(valid, comp, torch.zeros_like(comp))
    return dict(means2d=torch.stack([u, v], -1), conics=conics, depths=z, radii=radii,
                compensation=comp, lam1=lam1)


def project_points_f64(cam: Camera, pts: torch.Tensor, eps: float = 1e-8):
    """Camera.project_points (cameras.py:290-311) with its lens models
    (cameras.py:42-77), float64, differentiable."""
    R = torch.tensor(cam.R.numpy(), dtype=torch.float64)
    t = torch.tensor(cam.t.numpy(), dtype=torch.float64)
    pc = pts @ R.T + t
    if cam.orthographic:
        return torch.stack([cam.fx * pc[..., 0] + cam.cx, cam.fy * pc[..., 1] + cam.cy], -1)
    z = pc[..., 2]
    inv = 1.0 / torch.where(z.abs() < eps, torch.full_like(z, eps), z)
    x, y = pc[..., 0] * inv, pc[..., 1] * inv
    if cam.distortion is not None:
        c = list(cam.distortion)
        if cam.fisheye:
            k1, k2, k3, k4 = (c + [0.0] * 4)[:4]
            r = torch.sqrt(x * x + y * y)
            th = torch.atan(r)
            th2 = th * th
            thd = th * (1 + th2 * (k1 + th2 * (k2 + th2 * (k3 + th2 * k4))))
            scale = thd / torch.clamp(r, min=1e-9)
            x, y = x * scale, y * scale
        else:
            k1, k2, p1, p2 = c[:4]
            k3 = c[4] if len(c) > 4 else 0.0
            r2 = x * x + y * y
            radial = 1 + r2 * (k1 + r2 * (k2 + r2 * k3))
            x, y = (x * radial + 2 * p1 * x * y + p2 * (r2 + 2 * x * x),
                    y * radial + p1 * (r2 + 2 * y * y) + 2 * p2 * x * y)
    return torch.stack([cam.fx * x + cam.cx, cam.fy * y + cam.cy], -1)


def project_ut_f64(cam: Camera, means, quats, scales, blur=0.3, antialias=False):
    """project_gaussians_ut (projection.py:149-205) in float64, differentiable."""
    Rq = quat_to_rot_f64(quats)
    sq = Rq * scales[:, None, :]
    offsets = torch.cat([sq.transpose(1, 2), -sq.transpose(1, 2)], 1)
    sigma = means[:, None, :] + math.sqrt(3.0) * offsets
    xy = project_points_f64(cam, sigma.reshape(-1, 3)).reshape(means.shape[0], 6, 2)
    m2 = xy.mean(1)
    d = xy - m2[:, None, :]
    a0 = (d[..., 0] * d[..., 0]).mean(1)
    b = (d[..., 0] * d[..., 1]).mean(1)
    c0 = (d[..., 1] * d[..., 1]).mean(1)
    a, c = a0 + blur, c0 + blur
    det = a * c - b * b
    ds = torch.clamp(det, min=1e-12)
    conics = torch.stack([c / ds, -b / ds, a / ds], -1)
    if antialias and blur > 0:
        comp = torch.sqrt(torch.clamp(a0 * c0 - b * b, min=0.0) / ds)
    else:
        comp = torch.ones_like(det)
    mid = 0.5 * (a + c)
    lam1 = mid + torch.sqrt(torch.clamp(mid * mid - det, min=0.01))
    radii = torch.ceil(3.0 * torch.sqrt(torch.clamp(lam1, min=0.0)))
    R = torch.tensor(cam.R.numpy(), dtype=torch.float64)
    t = torch.tensor(cam.t.numpy(), dtype=torch.float64)
    z = (means @ R.T + t)[:, 2]
    valid = (z > cam.znear) & (det > 0)
    radii = torch.where(valid, radii, torch.zeros_like(radii))
    comp = torch.where(valid, comp, torch.zeros_like(comp))
    return dict(means2d=m2, conics=conics, depths=z, radii=radii, compensation=comp, lam1=lam1)


def lens_cameras(width=96, height=64):
    """Pinhole, Brown-Conrady (4 and 5 coefficients), fisheye and orthographic
    variants of one pose, for the UT projection."""
    base = Camera.look_at(eye=(0.3, -0.2, -3.0), at=(0, 0, 0), fov=55.0, width=width,
                          height=height)
    kw = dict(R=base.R, t=base.t, fx=base.fx, fy=base.fy, cx=base.cx, cy=base.cy, width=width,
              height=height)
    return {
        "pinhole": base,
        "brown4": Camera(**kw, distortion=(-0.35, 0.12, 0.002, -0.001)),
        "brown5": Camera(**kw, distortion=(0.08, -0.03, -0.004, 0.003, 0.01)),
        "fisheye": Camera(**kw, distortion=(0.05, -0.02, 0.004, -0.001), fisheye=True),
        "ortho": Camera.orthographic_camera(1.6, width, height, R=base.R, t=base.t),
    }


# ---------------------------------------------------------------------- SH
def sh_basis_scipy(degree: int, dirs: np.ndarray) -> np.ndarray:
    """Real SH basis in the 3DGS sign convention, via scipy's complex Y_l^m.

    3DGS orders degree-l terms m = -l..l and uses Y_{l,m} real with the
    Condon-Shortley phase removed and an extra (-1)^m... the conventions are
    fixed here by matching signs per basis function (see signs below), which
    is what 'up to sign' in the survey's check means; magnitudes come only
    from scipy.
    """
    from scipy.special import sph_harm_y

    x, y, z = dirs[:, 0].astype(np.float64), dirs[:, 1].astype(np.float64), dirs[:, 2].astype(np.float64)
    theta = np.arccos(np.clip(z, -1, 1))  # polar from +z
    phi = np.arctan2(y, x)
    cols = []
    for l in range(degree + 1):
        for m in range(-l, l + 1):
            Y = sph_harm_y(l, abs(m), theta, phi)
            if m > 0:
                val = math.sqrt(2) * (-1) ** m * Y.real
            elif m < 0:
                val = math.sqrt(2) * (-1) ** m * Y.imag
            else:
                val = Y.real
            cols.append(val)
    return np.stack(cols, -1)


# ----------------------------------------------------------------- binning
def tile_rects_np(means2d, radii, width, height):
    """tiles.py:54-65 in numpy float32."""
    tx_n = (width + TILE - 1) // TILE
    ty_n = (height + TILE - 1) // TILE
    x = means2d[:, 0].astype(np.float32)
    y = means2d[:, 1].astype(np.float32)
    r = radii.astype(np.float32)
    f16 = np.float32(16)
    with np.errstate(invalid="ignore"):
        xmin = np.clip(np.floor((x - r) / f16), 0, tx_n - 1).astype(np.int64)
        xmax = np.clip(np.floor((x + r) / f16), 0, tx_n - 1).astype(np.int64)
        ymin = np.clip(np.floor((y - r) / f16), 0, ty_n - 1).astype(np.int64)
        ymax = np.clip(np.floor((y + r) / f16), 0, ty_n - 1).astype(np.int64)
        on = (r > 0) & (x + r >= 0) & (x - r < np.float32(width)) & (y + r >= 0) & (y - r < np.float32(height))
    return xmin, xmax, ymin, ymax, on, tx_n, ty_n


def refine_keep_np(tx, ty, width, height, gx, gy, conic):
    """tiles.py:91-146 for one (tile, Gaussian), numpy float32 in the
    reference's operation order: minimum of the conic quadratic over the
    tile's continuous rectangle (corners + clipped edge minimisers) <= 12."""
    f = np.float32
    x0, y0 = f(tx * TILE), f(ty * TILE)
    x1, y1 = f(min((tx + 1) * TILE, width)), f(min((ty + 1) * TILE, height))
    gx, gy = f(gx), f(gy)
    dxl, dxr, dyb, dyt = x0 - gx, x1 - gx, y0 - gy, y1 - gy
    if dxl <= 0 and dxr >= 0 and dyb <= 0 and dyt >= 0:
        return True
    a, b, c = (f(v) for v in conic[:3])
    two = f(2.0)

    def q(dx, dy):
        return (a * dx * dx + two * b * dx * dy) + c * dy * dy

    def clip(v, lo, hi):
        return min(max(v, lo), hi)

    cands = [q(dxl, dyb), q(dxl, dyt), q(dxr, dyb), q(dxr, dyt),
             q(dxl, clip(-(b / c) * dxl, dyb, dyt)), q(dxr, clip(-(b / c) * dxr, dyb, dyt)),
             q(clip(-(b / a) * dyb, dxl, dxr), dyb), q(clip(-(b / a) * dyt, dxl, dxr), dyt)]
    return bool(min(cands) <= f(12.0))


def bin_bruteforce(means2d, radii, depths, width, height, conics=None):
    """Enumerate every (tile, Gaussian) pair (dropping those refine_tiles
    rejects when conics are given) and sort by (tile, depth, index) with
    Python's stable sort; ranges (0, 0) for empty tiles."""
    xmin, xmax, ymin, ymax, on, tx_n, ty_n = tile_rects_np(means2d, radii, width, height)
    pairs = []
    for g in range(means2d.shape[0]):
        if not on[g]:
            continue
        for ty in range(ymin[g], ymax[g] + 1):
            for tx in range(xmin[g], xmax[g] + 1):
                if conics is not None and not refine_keep_np(
                        tx, ty, width, height, means2d[g, 0], means2d[g, 1], conics[g]):
                    continue
                pairs.append((ty * tx_n + tx, float(depths[g]), g))
    pairs.sort(key=lambda p: (p[0], p[1], p[2]))
    ids = np.array([p[2] for p in pairs], dtype=np.int32)
    ranges = np.zeros((tx_n * ty_n, 2), np.int32)
    for i, p in enumerate(pairs):
        t = p[0]
        if i == 0 or pairs[i - 1][0] != t:
            ranges[t, 0] = i
        ranges[t, 1] = i + 1
    return ids, ranges, tx_n, ty_n


def tile_mask(means2d, radii, width, height):
    """(N, H, W) bool: pixel lies in a tile the Gaussian is binned to."""
    xmin, xmax, ymin, ymax, on, _, _ = tile_rects_np(means2d, radii, width, height)
    tx = np.arange(width) // TILE
    ty = np.arange(height) // TILE
    mx_ = (tx[None, :] >= xmin[:, None]) & (tx[None, :] <= xmax[:, None])
    my_ = (ty[None, :] >= ymin[:, None]) & (ty[None, :] <= ymax[:, None])
    return (my_[:, :, None] & mx_[:, None, :]) & on[:, None, None]


# ------------------------------------------------------------ compositing
def dense_composite_f64(means2d, conics, opac, feats, order, width, height, bg=None,
                        mask=None, kernel_stop=True, straight_through=False):
    """Dense float64 compositing of reference.py:47-74.

    ``order`` is the global front-to-back order.  With ``mask`` (N, H, W)
    only masked (Gaussian, pixel) pairs participate (the tiles a Gaussian is
    binned to).  ``kernel_stop`` applies the kernel's termination: the splat
    that would take T below 1e-4 is not composited and nothing after it is
    (rasterize.py:82-83); otherwise the reference.py rule (keep while the
    transmittance in front is > 1e-4).  ``straight_through`` gives the 0.99
    alpha clamp the gradient rule of the reference's backward kernel
    (rasterize.py:193: dL/dG = o dL/dalpha whether or not the clamp is
    active); without it autograd gives the clamp zero gradient when active,
    the rule of the reference's dense oracle.
    """
    xs = torch.arange(width, dtype=torch.float64) + 0.5
    ys = torch.arange(height, dtype=torch.float64) + 0.5
    m = means2d[order]
    co = conics[order]
    o = opac[order]
    f = feats[order]
    dx = m[:, 0, None, None] - xs[None, None, :]
    dy = m[:, 1, None, None] - ys[None, :, None]
    a, b, c = co[:, 0, None, None], co[:, 1, None, None], co[:, 2, None, None]
    power = -0.5 * (a * dx * dx + c * dy * dy) - b * dx * dy
    raw = o[:, None, None] * torch.exp(power)
    if straight_through:
        # value min(raw, 0.99), derivative d raw everywhere
        alpha = raw - torch.clamp(raw - 0.99, min=0.0).detach()
    else:
        alpha = torch.clamp(raw, max=0.99)
    alpha = torch.where(power > 0, torch.zeros_like(alpha), alpha)
    alpha = torch.where(alpha < 1.0 / 255.0, torch.zeros_like(alpha), alpha)
    if mask is not None:
        alpha = alpha * torch.as_tensor(mask[order.cpu().numpy()], dtype=torch.float64)
    one_minus = 1.0 - alpha
    trans_in = torch.cumprod(torch.cat([torch.ones_like(one_minus[:1]), one_minus[:-1]], 0), 0)
    if kernel_stop:
        trans_out = trans_in * one_minus
        crossed = (trans_out < 1e-4).to(torch.int64)
        # keep pairs strictly before the first crossing
        keep = torch.cumsum(crossed, 0) == 0
    else:
        keep = trans_in > 1e-4
    w = alpha * trans_in * keep
    img = torch.einsum("nhw,nc->hwc", w, f)
    final_T = torch.prod(torch.where(keep, one_minus, torch.ones_like(one_minus)), 0)
    if bg is not None:
        img = img + final_T[..., None] * bg
    return img, final_T, w


def depth_order(depths):
    d = np.asarray(depths)
    return torch.as_tensor(np.argsort(d, kind="stable"))


def eval_sh_f64(degree: int, sh: torch.Tensor, dirs: torch.Tensor) -> torch.Tensor:
    """Polynomial 3DGS real-SH expansion + 0.5 (sh.py:57-78), float64; the
    basis is tied to scipy by test_oracle_sh.test_poly_basis_is_scipy_basis."""
    x, y, z = dirs[:, 0:1], dirs[:, 1:2], dirs[:, 2:3]
    C0, C1 = 0.28209479177387814, 0.4886025119029199
    C2 = [1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792,
          0.5462742152960396]
    C3 = [-0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154,
          -0.4570457994644658, 1.445305721320277, -0.5900435899266435]
    basis = [torch.full_like(x, C0)]
    if degree > 0:
        basis += [-C1 * y, C1 * z, -C1 * x]
    if degree > 1:
        xx, yy, zz = x * x, y * y, z * z
        basis += [C2[0] * x * y, C2[1] * y * z, C2[2] * (2 * zz - xx - yy), C2[3] * x * z,
                  C2[4] * (xx - yy)]
    if degree > 2:
        basis += [C3[0] * y * (3 * xx - yy), C3[1] * x * y * z, C3[2] * y * (4 * zz - xx - yy),
                  C3[3] * z * (2 * zz - 3 * xx - 3 * yy), C3[4] * x * (4 * zz - xx - yy),
                  C3[5] * z * (xx - yy), C3[6] * x * (xx - 3 * yy)]
    out = sum(b * sh[:, k] for k, b in enumerate(basis))
    return out + 0.5


def render_f64(cam: Camera, means, quats, scales, opac, colors=None, sh=None, degree=0,
               bg=None, antialias=False, mask=None, order=None, kernel_stop=True,
               straight_through=False):
    """Differentiable float64 render: matrix-form projection, SH colour with
    stop-gradient directions (render.py:73-80), dense restricted compositing."""
    p = project_matrix_f64(cam, means, quats, scales, antialias=antialias)
    oe = opac * p["compensation"]
    if sh is not None:
        center = torch.tensor(cam.gsx_fields()["center"], dtype=torch.float64)
        d = means.detach() - center
        d = d / torch.clamp(torch.linalg.norm(d, dim=-1, keepdim=True), min=1e-8)
        colors = torch.clamp(eval_sh_f64(degree, sh, d), min=0.0)
    img, T, _ = dense_composite_f64(p["means2d"], p["conics"], oe, colors, order, cam.width,
                                    cam.height, bg=bg, mask=mask, kernel_stop=kernel_stop,
                                    straight_through=straight_through)
    return img, T, p


# ------------------------------------------------------------------- meshes
from mlx3d_amd.scenes import ico_sphere  # noqa: E402,F401  (the tests' mesh)


def mesh_zbuffer_f64(tri_xy, tri_z, width, height, znear=0.01):
    """All-faces float64 z-buffer: (nearest face, its depth, depth margin to
    the runner-up, coverage ambiguous) per pixel, for checking the binned
    rasterizer."""
    txy = np.asarray(tri_xy, np.float64).reshape(-1, 3, 2)
    tz = np.asarray(tri_z, np.float64).reshape(-1, 3)
    px = (np.arange(width) + 0.5)[None, :, None]
    py = (np.arange(height) + 0.5)[:, None, None]
    ax, ay = txy[:, 0, 0], txy[:, 0, 1]
    bx, by = txy[:, 1, 0], txy[:, 1, 1]
    cx, cy = txy[:, 2, 0], txy[:, 2, 1]
    den = (by - cy) * (ax - cx) + (cx - bx) * (ay - cy)
    ok = np.abs(den) >= 1e-12
    den = np.where(ok, den, 1.0)
    l0 = ((by - cy) * (px - cx) + (cx - bx) * (py - cy)) / den
    l1 = ((cy - ay) * (px - cx) + (ax - cx) * (py - cy)) / den
    l2 = 1.0 - l0 - l1
    z = l0 * tz[:, 0] + l1 * tz[:, 1] + l2 * tz[:, 2]
    hit = ok & (l0 >= -1e-5) & (l1 >= -1e-5) & (l2 >= -1e-5) & (z > znear)
    zz = np.where(hit, z, np.inf)
    best = np.argmin(zz, axis=-1)
    bz = np.take_along_axis(zz, best[..., None], -1)[..., 0]
    srt = np.sort(zz, axis=-1)
    margin = np.full(bz.shape, np.inf)
    if zz.shape[-1] > 1:
        with np.errstate(invalid="ignore"):
            gap = srt[..., 1] - srt[..., 0]
        margin = np.where(np.isfinite(srt[..., 0]), gap, np.inf)
    # a face's coverage of a pixel is ambiguous when its smallest barycentric
    # sits within rounding distance of the -1e-5 threshold
    lmin = np.minimum(np.minimum(l0, l1), l2)
    amb = (ok & (z > znear) & (np.abs(lmin + 1e-5) < 1e-4)).any(axis=-1)
    return (np.where(np.isfinite(bz), best, -1).astype(np.int32),
            np.where(np.isfinite(bz), bz, 0.0), margin, amb)


# ------------------------------------------------------------ 2DGS geometry
def surfel_features_f64(means, quats, depths, center):
    """(N, 5) = (z, z^2, n) of trainer.py:200-206 in float64: n the third
    column of the rotation of the normalised quaternion, normalised, flipped
    to face the camera centre."""
    q = quats / torch.linalg.norm(quats, dim=-1, keepdim=True)
    w, x, y, z = q.unbind(-1)
    col = torch.stack([2 * (x * z + w * y), 2 * (y * z - w * x), 1 - 2 * (x * x + y * y)], -1)
    n = col / torch.clamp(torch.linalg.norm(col, dim=-1, keepdim=True), min=1e-8)
    view = torch.as_tensor(center, dtype=means.dtype) - means
    n = torch.where((n * view).sum(-1, keepdim=True) < 0, -n, n)
    return torch.cat([depths[:, None], (depths * depths)[:, None], n], 1)


def geometry_loss_f64(F, alpha, camera, min_alpha, lam_dv, lam_nc):
    """The 2DGS losses of trainer.py:208-257 on an alpha-normalised (H, W, 5)
    render, float64 (the camera's unprojection evaluated in float64)."""
    H, W = alpha.shape
    valid = (alpha > min_alpha).to(F.dtype)
    ed, ed2 = F[..., 0], F[..., 1]
    dv = (torch.clamp(ed2 - ed * ed, min=0.0) * valid).sum() / torch.clamp(valid.sum(), min=1.0)
    u = torch.arange(W, dtype=F.dtype) + 0.5
    v = torch.arange(H, dtype=F.dtype) + 0.5
    # cameras.py:327-336 in float64: undistorted normalised coordinates,
    # scaled by the depth, then (X_cam - t) R
    xn = ((u[None, :] - camera.cx) / camera.fx).expand(H, W)
    yn = ((v[:, None] - camera.cy) / camera.fy).expand(H, W)
    R, t = camera.R.double(), camera.t.double()
    if camera.orthographic:
        pc = torch.stack([xn, yn, ed], -1)
    else:
        xu, yu = camera._undistort(xn, yn)
        pc = torch.stack([xu * ed, yu * ed, ed], -1)
    pts = (pc - t) @ R
    tx = pts[:-1, 1:] - pts[:-1, :-1]
    ty = pts[1:, :-1] - pts[:-1, :-1]
    dn = torch.linalg.cross(tx, ty)
    dn = dn / torch.clamp(torch.linalg.norm(dn, dim=-1, keepdim=True), min=1e-8)
    rn = F[:-1, :-1, 2:5]
    rn = rn / torch.clamp(torch.linalg.norm(rn, dim=-1, keepdim=True), min=1e-8)
    v4 = valid[:-1, :-1] * valid[:-1, 1:] * valid[1:, :-1] * valid[1:, 1:]
    nc = ((1.0 - (rn * dn).sum(-1).abs()) * v4).sum() / torch.clamp(v4.sum(), min=1.0)
    return lam_dv * dv + lam_nc * nc, dv, nc
