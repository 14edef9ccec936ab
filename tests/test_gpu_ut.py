"""GPU parity of the UT projection (gsx_project_ut_fwd/bwd and the fused
preprocess under GSX_PROJECT_UT) against the CPU oracle, on pinhole,
Brown-Conrady, fisheye and orthographic cameras.

Forward outputs (means2d, conics, depths, radii, compensation) and the
rendered image / contributor counts are bit-identical to the oracle (same
float32 operations); gradients within max|d| / max|ref| < 1e-3.
"""

from __future__ import annotations

import numpy as np
import pytest

from gpu_util import assert_bits, cu, host, oracle_backward, oracle_forward, rel_err, say
from mlx3d_amd.splatting import GaussianModel, project_gaussians_ut, render_gaussians
from mlx3d_amd.splatting.trainer import GaussianTrainer, TrainerConfig
from oracle import oracle as O
from refimpl import lens_cameras, oracle_camera

pytestmark = pytest.mark.gpu

CAMS = ["pinhole", "brown4", "brown5", "fisheye", "ortho"]


def _scene(n, seed, w=160, h=112):
    rng = np.random.default_rng(seed)
    means = (rng.standard_normal((n, 3)) * 0.7).astype(np.float32)
    quats = rng.standard_normal((n, 4)).astype(np.float32)
    scales = np.exp(rng.standard_normal((n, 3)) * 0.4 - 3.2).astype(np.float32)
    opac = (1 / (1 + np.exp(-rng.standard_normal(n)))).astype(np.float32)
    sh = (rng.standard_normal((n, 16, 3)) * 0.2).astype(np.float32)
    return lens_cameras(w, h), means, quats, scales, opac, sh


def test_device_atan_bitexact():
    from mlx3d_amd import _lib

    r = np.concatenate([np.linspace(0, 4, 400001), np.geomspace(1e-20, 1e20, 200001),
                        [0.41421356, 0.41421357, 1.0, 0.99999994, 1.0000001]]).astype(np.float32)
    x = cu(r)
    y = x.new_empty(x.shape)
    _lib.check(_lib.load().gsx_debug_atanf(x.numel(), _lib.ptr(x), _lib.ptr(y),
                                           _lib.stream_handle(x.device)), "atan")
    assert_bits(host(y), O.atanf(r), "device atan")


@pytest.mark.parametrize("name", CAMS)
@pytest.mark.parametrize("antialias", [False, True])
def test_project_ut_bitexact(name, antialias):
    say(f"project_ut {name} aa={antialias}")
    cams, means, quats, scales, _, _ = _scene(5000, 1)
    cam = cams[name]
    t = [cu(a).requires_grad_(True) for a in (means, quats, scales)]
    out = project_gaussians_ut(cam, *t, antialias=antialias)
    ref = O.project_ut(oracle_camera(cam), means, quats, scales, antialias=antialias)
    for k in ("means2d", "conics", "depths", "radii", "compensation"):
        assert_bits(host(out[k]), ref[k], f"{name} {k}")
    rng = np.random.default_rng(2)
    gm2 = rng.standard_normal((5000, 2)).astype(np.float32)
    gco = (rng.standard_normal((5000, 3)) * 1e-3).astype(np.float32)
    gd = rng.standard_normal(5000).astype(np.float32)
    gc = rng.standard_normal(5000).astype(np.float32)
    ((out["means2d"] * cu(gm2)).sum() + (out["conics"] * cu(gco)).sum()
     + (out["depths"] * cu(gd)).sum() + (out["compensation"] * cu(gc)).sum()).backward()
    g = O.project_bwd(oracle_camera(cam), means, quats, scales, gm2, gco, gd, gc,
                      antialias=antialias, ut=True)
    for k, a, b in zip(("means", "quats", "scales"), t, g):
        e = rel_err(host(a.grad), b)
        say(f"  grad {k}: rel {e:.2e}")
        assert e < 1e-5


@pytest.mark.parametrize("name", CAMS)
def test_render_ut_matches_oracle(name):
    say(f"render ut {name}")
    cams, means, quats, scales, opac, sh = _scene(6000, 3)
    cam = cams[name]
    t = [cu(a).requires_grad_(True) for a in (means, quats, scales, opac, sh)]
    out = render_gaussians(cam, t[0], t[1], t[2], t[3], sh=t[4], sh_degree=3, antialias=True,
                           projection="ut")
    flags = O.PROJECT_UT | O.ANTIALIAS
    pre, feats, ids, ranges, r = oracle_forward(cam, means, quats, scales, opac, sh=sh, degree=3,
                                                flags=flags)
    np.testing.assert_array_equal(host(out["sorted_ids"]), ids)
    np.testing.assert_array_equal(host(out["n_contrib"]), r["n_contrib"])
    assert_bits(host(out["image"]), r["image"], "image")
    rng = np.random.default_rng(4)
    g_img = rng.standard_normal(r["image"].shape).astype(np.float32)
    g_a = rng.standard_normal(r["final_T"].shape).astype(np.float32)
    ((out["image"] * cu(g_img)).sum() + (out["alpha"] * cu(g_a)).sum()).backward()
    g = oracle_backward(cam, means, quats, scales, opac, pre, feats, ids, ranges, r, g_img, g_a,
                        sh=sh, degree=3, flags=flags)
    for k, a, key in [("means", t[0], "means"), ("quats", t[1], "quats"),
                      ("scales", t[2], "scales"), ("opacities", t[3], "opacities"),
                      ("sh", t[4], "sh")]:
        e = rel_err(host(a.grad), g[key])
        say(f"  grad {k}: rel {e:.2e}")
        assert e < 1e-3


def test_model_and_trainer_ut():
    cams, means, quats, scales, opac, sh = _scene(3000, 5)
    cam = cams["fisheye"]
    lo = np.log(opac / (1 - opac)).astype(np.float32)
    raw = dict(means=means, quats=quats, scales=np.log(scales).astype(np.float32), opacities=lo,
               sh_dc=sh[:, :1].copy(), sh_rest=sh[:, 1:].copy())
    model = GaussianModel({k: cu(v) for k, v in raw.items()})
    model.active_sh_degree = 3
    out = model.render(cam, projection="ut")
    flags = O.PROJECT_UT | O.LOG_SCALES | O.LOGIT_OPACITY
    _, _, _, _, r = oracle_forward(cam, means, quats, raw["scales"], lo, sh=sh, degree=3,
                                   flags=flags)
    assert_bits(host(out["image"]), r["image"], "model image")
    target = out["image"].detach().flip(1).contiguous()
    tr = GaussianTrainer(model, TrainerConfig(projection="ut", densify_from=2, densify_every=3,
                                              densify_until=10, densify_grad_threshold=1e-6))
    losses = [tr.step(cam, target)["loss"] for _ in range(6)]
    say(f"  ut trainer losses {losses[0]:.4f} -> {losses[-1]:.4f}")
    assert all(np.isfinite(losses)) and losses[-1] < losses[0]
    with pytest.raises(ValueError):
        render_gaussians(cam, *[cu(a) for a in (means, quats, scales, opac)],
                         colors=cu(sh[:, 0]), projection="xyz")
