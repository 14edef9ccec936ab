"""Writes the golden fixtures in this directory.

The expected values come from the independent float64 restatements in
tests/refimpl.py (matrix-form EWA projection, scipy-tied SH polynomials,
brute-force binning, dense all-pairs compositing and torch float64
autograd through them), never from the CPU oracle or the HIP library, so
the fixtures pin both.  The reference itself (MLX + Metal kernels) cannot
run on this Linux host, so no fixture holds reference-produced numbers.

Scenes are small and seeded.  Gaussians whose tile rectangle or radius
sits within float32 noise of an integer boundary are dropped, so float32
and float64 agree on which tiles each Gaussian is binned to.

Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from mlx3d_amd.cameras import Camera  # noqa: E402
from refimpl import (bin_bruteforce, depth_order, eval_sh_f64, project_matrix_f64,  # noqa: E402
                     render_f64, sh_basis_scipy, tile_mask)

TILE = 16
F64 = torch.float64


def t64(a, grad=False):
    return torch.tensor(np.asarray(a), dtype=F64, requires_grad=grad)


def cam_of(spec):
    eye, at, w, h, fov = spec
    return Camera.look_at(eye=tuple(eye), at=tuple(at), width=int(w), height=int(h), fov=float(fov))


def cam_arrays(spec):
    eye, at, w, h, fov = spec
    return dict(cam_eye=np.array(eye, np.float64), cam_at=np.array(at, np.float64),
                cam_size=np.array([w, h], np.int32), cam_fov=np.array(fov, np.float64))


def safe_mask(p, width, height, margin=1e-3):
    """Gaussians whose radius and tile-rectangle edges are clear of integer
    boundaries by `margin` (so float32 and float64 bin them alike)."""
    r64 = 3.0 * np.sqrt(np.maximum(p["lam1"].detach().numpy(), 0.0))
    ok = np.abs(r64 - np.round(r64)) > margin
    m = p["means2d"].detach().numpy()
    r = p["radii"].detach().numpy()
    for edge in (m[:, 0] - r, m[:, 0] + r, m[:, 1] - r, m[:, 1] + r):
        q = edge / TILE
        ok &= np.abs(q - np.round(q)) > margin / TILE
    # clear of the on-screen test and the depth cull too
    ok &= np.abs(m[:, 0] + r) > margin
    ok &= np.abs(m[:, 0] - r - width) > margin
    ok &= np.abs(m[:, 1] + r) > margin
    ok &= np.abs(m[:, 1] - r - height) > margin
    return ok


def projection():
    spec = ((0.3, -0.2, -3.0), (0.0, 0.0, 0.0), 80, 48, 55.0)
    cam = cam_of(spec)
    rng = np.random.default_rng(21)
    n = 160
    means = (rng.standard_normal((n, 3)) * 0.5).astype(np.float32)
    means[:6, 2] = -5.0  # behind the camera
    means[6:12, 0] = 7.0  # outside the frustum clip
    quats = rng.standard_normal((n, 4)).astype(np.float32)
    scales = np.exp(rng.standard_normal((n, 3)) * 0.3 - 2.3).astype(np.float32)
    out = dict(means=means, quats=quats, scales=scales, **cam_arrays(spec))
    for aa in (0, 1):
        p = project_matrix_f64(cam, t64(means), t64(quats), t64(scales), antialias=bool(aa))
        r64 = 3.0 * np.sqrt(np.maximum(p["lam1"].numpy(), 0.0))
        out[f"aa{aa}_safe"] = np.abs(r64 - np.round(r64)) > 1e-3
        for k in ("means2d", "conics", "depths", "radii", "compensation"):
            out[f"aa{aa}_{k}"] = p[k].numpy()
    return out


def sh():
    rng = np.random.default_rng(22)
    n = 64
    coef = (rng.standard_normal((n, 16, 3)) * 0.3).astype(np.float32)
    d = rng.standard_normal((n, 3))
    dirs = (d / np.linalg.norm(d, axis=1, keepdims=True)).astype(np.float32)
    out = dict(sh=coef, dirs=dirs)
    for deg in range(4):
        k = (deg + 1) ** 2
        # the polynomial form must agree with scipy's basis on exact unit vectors
        unit = dirs.astype(np.float64) / np.linalg.norm(dirs.astype(np.float64), axis=1,
                                                        keepdims=True)
        basis = sh_basis_scipy(deg, unit)
        poly = (eval_sh_f64(deg, torch.eye(k, dtype=F64)[None].expand(n, k, k), t64(unit))
                - 0.5).numpy()
        sign = np.sign(np.sum(poly * basis, 0))  # 3DGS sign convention vs scipy's
        assert np.all(sign != 0) and np.abs(poly - basis * sign).max() < 1e-9, deg
        out[f"deg{deg}"] = eval_sh_f64(deg, t64(coef), t64(dirs)).numpy()
    return out


def binning():
    out = {}
    spec = ((0.0, 0.0, -4.0), (0.0, 0.0, 0.0), 96, 64, 50.0)
    cam = cam_of(spec)
    rng = np.random.default_rng(23)
    n = 400
    means = (rng.standard_normal((n, 3)) * 0.5).astype(np.float32)
    quats = rng.standard_normal((n, 4)).astype(np.float32)
    scales = np.exp(rng.standard_normal((n, 3)) * 0.3 - 2.5).astype(np.float32)
    p = project_matrix_f64(cam, t64(means), t64(quats), t64(scales))
    ok = safe_mask(p, 96, 64)
    cases = {
        "scene": (p["means2d"].numpy()[ok].astype(np.float32),
                  p["radii"].numpy()[ok].astype(np.float32),
                  p["depths"].numpy()[ok].astype(np.float32), 96, 64),
    }
    m = rng.uniform(0, 200, (300, 2)).astype(np.float32)
    cases["ties"] = (m, rng.integers(1, 30, 300).astype(np.float32),
                     rng.choice(np.array([1.0, 2.0, 3.0], np.float32), 300), 200, 120)
    m2 = np.concatenate([[[100.0, 60.0]], m[:20]]).astype(np.float32)
    r2 = np.concatenate([[1e5], np.full(20, 5.0)]).astype(np.float32)
    cases["huge"] = (m2, r2, rng.uniform(1, 2, 21).astype(np.float32), 200, 120)
    for name, (m2d, rad, dep, w, h) in cases.items():
        ids, ranges, _, _ = bin_bruteforce(m2d, rad, dep, w, h)
        out.update({f"{name}_means2d": m2d, f"{name}_radii": rad, f"{name}_depths": dep,
                    f"{name}_size": np.array([w, h], np.int32), f"{name}_ids": ids,
                    f"{name}_ranges": ranges})
    return out


def render_colors():
    """render_gaussians with colours: image/alpha and parameter gradients of
    sum(image * g_img) + sum(alpha * g_alpha)."""
    spec = ((0.2, 0.1, -4.0), (0.0, 0.0, 0.0), 96, 64, 50.0)
    cam = cam_of(spec)
    rng = np.random.default_rng(24)
    n = 300
    means = (rng.standard_normal((n, 3)) * 0.5).astype(np.float32)
    quats = rng.standard_normal((n, 4)).astype(np.float32)
    scales = np.exp(rng.standard_normal((n, 3)) * 0.3 - 2.5).astype(np.float32)
    opac = np.minimum(1.0 / (1.0 + np.exp(-rng.standard_normal(n))), 0.9).astype(np.float32)
    colors = rng.uniform(size=(n, 3)).astype(np.float32)
    p = project_matrix_f64(cam, t64(means), t64(quats), t64(scales), antialias=True)
    ok = safe_mask(p, 96, 64)
    means, quats, scales, opac, colors = (a[ok] for a in (means, quats, scales, opac, colors))
    bg = np.array([0.1, 0.2, 0.3], np.float32)
    g_img = rng.standard_normal((64, 96, 3)).astype(np.float32)
    g_alpha = rng.standard_normal((64, 96)).astype(np.float32)
    t = {k: t64(v, True) for k, v in dict(means=means, quats=quats, scales=scales, opac=opac,
                                           colors=colors).items()}
    p = project_matrix_f64(cam, t["means"].detach(), t["quats"].detach(), t["scales"].detach(),
                           antialias=True)
    m2d = p["means2d"].numpy().astype(np.float32)
    rad = p["radii"].numpy().astype(np.float32)
    mask = tile_mask(m2d, rad, 96, 64)
    img, T, _ = render_f64(cam, t["means"], t["quats"], t["scales"], t["opac"],
                           colors=t["colors"], bg=t64(bg), antialias=True, mask=mask,
                           order=depth_order(p["depths"].numpy()))
    loss = (img * t64(g_img)).sum() + ((1 - T) * t64(g_alpha)).sum()
    loss.backward()
    out = dict(means=means, quats=quats, scales=scales, opacities=opac, colors=colors, bg=bg,
               g_img=g_img, g_alpha=g_alpha, image=img.detach().numpy(),
               alpha=(1 - T).detach().numpy(), **cam_arrays(spec))
    for k, name in [("means", "g_means"), ("quats", "g_quats"), ("scales", "g_scales"),
                    ("opac", "g_opacities"), ("colors", "g_colors")]:
        out[name] = t[k].grad.numpy()
    return out


def render_model():
    """GaussianModel.render: raw parameters (log-scales, logit opacities,
    SH degree 2 stored as degree 3), L = sum(image * g_img)."""
    spec = ((-0.3, 0.2, -3.5), (0.0, 0.0, 0.0), 80, 64, 55.0)
    cam = cam_of(spec)
    rng = np.random.default_rng(25)
    n = 250
    means = (rng.standard_normal((n, 3)) * 0.5).astype(np.float32)
    quats = rng.standard_normal((n, 4)).astype(np.float32)
    log_scales = (rng.standard_normal((n, 3)) * 0.3 - 2.5).astype(np.float32)
    logit = np.clip(rng.standard_normal(n), -4.0, 2.0).astype(np.float32)  # opacity < 0.9
    sh_dc = rng.uniform(-0.5, 0.5, (n, 1, 3)).astype(np.float32)
    sh_rest = (rng.standard_normal((n, 15, 3)) * 0.1).astype(np.float32)
    p = project_matrix_f64(cam, t64(means), t64(quats), torch.exp(t64(log_scales)))
    ok = safe_mask(p, 80, 64)
    means, quats, log_scales, logit, sh_dc, sh_rest = (
        a[ok] for a in (means, quats, log_scales, logit, sh_dc, sh_rest))
    g_img = rng.standard_normal((64, 80, 3)).astype(np.float32)
    t = {k: t64(v, True) for k, v in dict(means=means, quats=quats, scales=log_scales,
                                           opac=logit, sh_dc=sh_dc, sh_rest=sh_rest).items()}
    scales_a = torch.exp(t["scales"])
    opac_a = 1.0 / (1.0 + torch.exp(-t["opac"]))
    p = project_matrix_f64(cam, t["means"].detach(), t["quats"].detach(), scales_a.detach())
    m2d = p["means2d"].numpy().astype(np.float32)
    rad = p["radii"].numpy().astype(np.float32)
    mask = tile_mask(m2d, rad, 80, 64)
    shc = torch.cat([t["sh_dc"], t["sh_rest"]], 1)
    img, T, _ = render_f64(cam, t["means"], t["quats"], scales_a, opac_a, sh=shc, degree=2,
                           mask=mask, order=depth_order(p["depths"].numpy()))
    (img * t64(g_img)).sum().backward()
    out = dict(means=means, quats=quats, log_scales=log_scales, logit_opacities=logit,
               sh_dc=sh_dc, sh_rest=sh_rest, g_img=g_img, image=img.detach().numpy(),
               alpha=(1 - T).detach().numpy(), sh_degree=np.array(2, np.int32),
               **cam_arrays(spec))
    for k, name in [("means", "g_means"), ("quats", "g_quats"), ("scales", "g_scales"),
                    ("opac", "g_opacities"), ("sh_dc", "g_sh_dc"), ("sh_rest", "g_sh_rest")]:
        out[name] = t[k].grad.numpy()
    return out


def main():
    for name, fn in [("projection", projection), ("sh", sh), ("binning", binning),
                     ("render_colors", render_colors), ("render_model", render_model)]:
        data = {k: (v.astype(np.float32) if v.dtype == np.float64 and v.ndim > 0 else v)
                for k, v in fn().items()}  # float32 keeps ~1e-7 relative: ample here
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **data)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
