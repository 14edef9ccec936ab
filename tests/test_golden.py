"""Committed known-answer fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from independent float64 restatements) checked
against the CPU oracle and, marked gpu, against the HIP library through the
drop-in API.  Tolerances are the north star's: image/alpha 1e-5 absolute,
gradients max|d|/max|ref| < 1e-3, sorted ids / ranges / radii exact."""

import os

import numpy as np
import pytest
import torch

from mlx3d_amd.cameras import Camera
from oracle import oracle as O
from refimpl import oracle_camera

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def camera(f):
    w, h = (int(v) for v in f["cam_size"])
    return Camera.look_at(eye=tuple(f["cam_eye"]), at=tuple(f["cam_at"]), width=w, height=h,
                          fov=float(f["cam_fov"]))


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / (np.abs(b).max() + 1e-30))


def check_projection(out, f, aa):
    p = f"aa{aa}_"
    safe = f[p + "safe"]
    # culled Gaussians behind the camera project to ~1e7 px: relative there
    np.testing.assert_allclose(out["means2d"], f[p + "means2d"], rtol=2e-6, atol=1e-4)
    np.testing.assert_allclose(out["depths"], f[p + "depths"], atol=1e-5)
    np.testing.assert_allclose(out["conics"], f[p + "conics"], rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(out["compensation"], f[p + "compensation"], atol=1e-5)
    np.testing.assert_array_equal(out["radii"][safe], f[p + "radii"][safe])
    assert safe.mean() > 0.97


def check_render(img, alpha, grads, f, names):
    np.testing.assert_allclose(img, f["image"], atol=1e-5)
    np.testing.assert_allclose(alpha, f["alpha"], atol=1e-5)
    for name in names:
        e = rel(grads[name], f[name])
        assert e < 1e-3, f"{name}: {e}"


# ------------------------------------------------------------- CPU oracle
@pytest.mark.parametrize("aa", [0, 1])
def test_oracle_projection_golden(aa):
    f = load("projection")
    out = O.project(oracle_camera(camera(f)), f["means"], f["quats"], f["scales"],
                    antialias=bool(aa))
    check_projection(out, f, aa)


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_oracle_sh_golden(deg):
    f = load("sh")
    np.testing.assert_allclose(O.eval_sh(deg, f["sh"], f["dirs"]), f[f"deg{deg}"], atol=2e-6)


@pytest.mark.parametrize("case", ["scene", "ties", "huge"])
def test_oracle_binning_golden(case):
    f = load("binning")
    w, h = (int(v) for v in f[f"{case}_size"])
    ids, ranges, _, _ = O.bin_gaussians(f[f"{case}_means2d"], f[f"{case}_radii"],
                                        f[f"{case}_depths"], w, h)
    np.testing.assert_array_equal(ids, f[f"{case}_ids"])
    np.testing.assert_array_equal(ranges, f[f"{case}_ranges"])


def _oracle_render(cam, means, quats, scales, opac, colors=None, sh=None, degree=0, flags=0,
                   bg=None, g_img=None, g_alpha=None):
    oc = oracle_camera(cam)
    pre = O.preprocess_fwd(oc, means, quats, scales, opac, sh=sh, degree=degree, flags=flags)
    feats = pre["colors"] if sh is not None else colors
    ids, ranges, _, _ = O.bin_gaussians(pre["means2d"], pre["radii"], pre["depths"], cam.width,
                                        cam.height)
    r = O.raster_fwd(pre["means2d"], pre["conics"], pre["opac_eff"], feats, ids, ranges,
                     cam.width, cam.height, bg=bg)
    gr = O.raster_bwd(pre["means2d"], pre["conics"], pre["opac_eff"], feats, ids, ranges,
                      cam.width, cam.height, r["final_T"], r["n_contrib"], g_img,
                      grad_final_T=None if g_alpha is None else -g_alpha, bg=bg)
    K = 0 if sh is None else sh.shape[1]
    g = O.preprocess_bwd(oc, means, quats, scales, opac, pre["colors"] if sh is not None else None,
                         K, degree, flags, gr["means2d"], gr["conics"], gr["opacities"],
                         gr["features"] if sh is not None else None)
    g["colors"] = gr["features"]
    return r, g


def test_oracle_render_colors_golden():
    f = load("render_colors")
    r, g = _oracle_render(camera(f), f["means"], f["quats"], f["scales"], f["opacities"],
                          colors=f["colors"], flags=O.ANTIALIAS, bg=f["bg"], g_img=f["g_img"],
                          g_alpha=f["g_alpha"])
    grads = {"g_means": g["means"], "g_quats": g["quats"], "g_scales": g["scales"],
             "g_opacities": g["opacities"], "g_colors": g["colors"]}
    check_render(r["image"], 1 - r["final_T"], grads, f, list(grads))


def test_oracle_render_model_golden():
    f = load("render_model")
    sh = np.concatenate([f["sh_dc"], f["sh_rest"]], 1)
    r, g = _oracle_render(camera(f), f["means"], f["quats"], f["log_scales"],
                          f["logit_opacities"], sh=sh, degree=int(f["sh_degree"]),
                          flags=O.LOG_SCALES | O.LOGIT_OPACITY, g_img=f["g_img"])
    grads = {"g_means": g["means"], "g_quats": g["quats"], "g_scales": g["scales"],
             "g_opacities": g["opacities"], "g_sh_dc": g["sh"][:, :1], "g_sh_rest": g["sh"][:, 1:]}
    check_render(r["image"], 1 - r["final_T"], grads, f, list(grads))


# -------------------------------------------------------------- HIP path
def cu(a):
    return torch.as_tensor(np.ascontiguousarray(a)).to("cuda")


def host(t):
    return t.detach().cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("aa", [0, 1])
def test_gpu_projection_golden(aa):
    from mlx3d_amd.splatting import project_gaussians

    f = load("projection")
    out = project_gaussians(camera(f), cu(f["means"]), cu(f["quats"]), cu(f["scales"]),
                            antialias=bool(aa))
    check_projection({k: host(v) for k, v in out.items()}, f, aa)


@pytest.mark.gpu
@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_gpu_sh_golden(deg):
    from mlx3d_amd.splatting import eval_sh

    f = load("sh")
    np.testing.assert_allclose(host(eval_sh(deg, cu(f["sh"]), cu(f["dirs"]))), f[f"deg{deg}"],
                               atol=2e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["scene", "ties", "huge"])
def test_gpu_binning_golden(case):
    from mlx3d_amd.splatting import bin_gaussians

    f = load("binning")
    w, h = (int(v) for v in f[f"{case}_size"])
    ids, ranges, _, _ = bin_gaussians(cu(f[f"{case}_means2d"]), cu(f[f"{case}_radii"]),
                                      cu(f[f"{case}_depths"]), w, h)
    np.testing.assert_array_equal(host(ids), f[f"{case}_ids"])
    np.testing.assert_array_equal(host(ranges), f[f"{case}_ranges"])


@pytest.mark.gpu
def test_gpu_render_colors_golden():
    from mlx3d_amd.splatting import render_gaussians

    f = load("render_colors")
    t = {k: cu(f[k]).requires_grad_(True) for k in ("means", "quats", "scales", "opacities",
                                                    "colors")}
    out = render_gaussians(camera(f), t["means"], t["quats"], t["scales"], t["opacities"],
                           colors=t["colors"], background=cu(f["bg"]), antialias=True)
    ((out["image"] * cu(f["g_img"])).sum() + (out["alpha"] * cu(f["g_alpha"])).sum()).backward()
    grads = {"g_" + k: host(v.grad) for k, v in t.items()}
    check_render(host(out["image"]), host(out["alpha"]), grads, f, list(grads))


@pytest.mark.gpu
def test_gpu_render_model_golden():
    from mlx3d_amd.splatting import GaussianModel

    f = load("render_model")
    m = GaussianModel({"means": cu(f["means"]), "quats": cu(f["quats"]),
                       "scales": cu(f["log_scales"]), "opacities": cu(f["logit_opacities"]),
                       "sh_dc": cu(f["sh_dc"]), "sh_rest": cu(f["sh_rest"])}, sh_degree=3)
    m.active_sh_degree = int(f["sh_degree"])
    m.requires_grad_(True)
    out = m.render(camera(f))
    (out["image"] * cu(f["g_img"])).sum().backward()
    p = m.params
    grads = {"g_means": host(p["means"].grad), "g_quats": host(p["quats"].grad),
             "g_scales": host(p["scales"].grad), "g_opacities": host(p["opacities"].grad),
             "g_sh_dc": host(p["sh_dc"].grad), "g_sh_rest": host(p["sh_rest"].grad)}
    check_render(host(out["image"]), host(out["alpha"]), grads, f, list(grads))
