"""Parity at the benchmark configurations' full sizes (configs 1-5 of
mlx3d_amd.scenes): GPU vs CPU oracle on the same seeded scenes.  Sorted ids, tile ranges
and n_contrib bit-exact; images/depth bit-exact; gradients to 1e-3
relative.  Also size-independent invariants of the binning."""

import numpy as np
import pytest
import torch

from gpu_util import (assert_bits, assert_features, cu, host, oracle_backward, oracle_forward,
                      rel_err, say)
from mlx3d_amd import scenes
from mlx3d_amd.splatting import GaussianModel, render_gaussian_features
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _model(scene):
    m = GaussianModel({"means": cu(scene.means), "quats": cu(scene.quats),
                       "scales": cu(scene.log_scales), "opacities": cu(scene.logit_opacities),
                       "sh_dc": cu(scene.sh_dc), "sh_rest": cu(scene.sh_rest)}, sh_degree=3)
    m.active_sh_degree = scene.sh_degree
    return m


def _sh(scene):
    return np.concatenate([scene.sh_dc, scene.sh_rest], 1)


def _flags(scene):
    f = O.LOG_SCALES | O.LOGIT_OPACITY
    return f | (O.ANTIALIAS if scene.antialias else 0)


def _invariants(ids, ranges, n):
    ids, ranges = host(ids), host(ranges)
    lens = ranges[:, 1] - ranges[:, 0]
    assert (lens >= 0).all()
    assert int(lens.sum()) == ids.shape[0]
    nz = lens > 0
    # non-empty ranges tile [0, D) in tile order
    st = ranges[nz, 0]
    assert st[0] == 0 and (np.diff(st) > 0).all()
    assert (ranges[nz, 1][:-1] == st[1:]).all()
    assert ids.min(initial=0) >= 0 and ids.max(initial=0) < n


def _check_view(scene, view, backward=True, grad_tol=1e-3):
    cam = scene.cameras[view]
    say(f"{scene.name} view {view}: N={scene.n} {cam.width}x{cam.height}")
    model = _model(scene)
    model.requires_grad_(backward)
    out = model.render(cam, antialias=scene.antialias, return_depth=scene.depth)
    _invariants(out["sorted_ids"], out["tile_ranges"], scene.n)
    flags = _flags(scene)
    sh = _sh(scene)
    pre, feats, ids, ranges, r = oracle_forward(cam, scene.means, scene.quats, scene.log_scales,
                                                scene.logit_opacities, sh=sh,
                                                degree=scene.sh_degree, flags=flags,
                                                depth=scene.depth)
    say(f"  D={ids.shape[0]}")
    np.testing.assert_array_equal(host(out["tile_ranges"]), ranges)
    np.testing.assert_array_equal(host(out["sorted_ids"]), ids)
    np.testing.assert_array_equal(host(out["n_contrib"]), r["n_contrib"])
    assert_bits(host(out["image"]), r["image"], "image")
    assert_bits(host(out["final_T"]), r["final_T"], "final_T")
    if scene.depth:
        assert_bits(host(out["depth"]), r["depth"], "depth")
    if not backward:
        return
    target = scene.target(cam)
    loss = (out["image"] - cu(target)).abs().mean()
    loss.backward()
    img = r["image"]
    g_img = (np.sign(img - target) / np.float32(target.size)).astype(np.float32)
    g = oracle_backward(cam, scene.means, scene.quats, scene.log_scales, scene.logit_opacities,
                        pre, feats, ids, ranges, r, g_img, None, sh=sh, degree=scene.sh_degree,
                        flags=flags)
    p = model.params
    shg = np.concatenate([host(p["sh_dc"].grad), host(p["sh_rest"].grad)], 1)
    for name, a, b in [("means", host(p["means"].grad), g["means"]),
                       ("quats", host(p["quats"].grad), g["quats"]),
                       ("scales", host(p["scales"].grad), g["scales"]),
                       ("opacities", host(p["opacities"].grad), g["opacities"]),
                       ("sh", shg, g["sh"])]:
        e = rel_err(a, b)
        say(f"  grad {name}: rel {e:.2e}")
        assert e < grad_tol


def test_config1_forward():
    scene = scenes.make_scene(1)
    _check_view(scene, 0, backward=False)


def test_config2_fwd_bwd():
    _check_view(scenes.make_scene(2), 0)


@pytest.mark.parametrize("view", [0, 5])
def test_config3_fwd_bwd(view):
    _check_view(scenes.make_scene(3), view)


def test_config4_heavy_tail():
    scene = scenes.make_scene(4)
    _check_view(scene, 0)


def test_config5_features_depth():
    scene = scenes.make_scene(5)
    cam = scene.cameras[0]
    say(f"{scene.name}: N={scene.n}")
    t = [cu(a).requires_grad_(True) for a in (scene.means, scene.quats, scene.scales,
                                              scene.opacities, scene.features)]
    out = render_gaussian_features(cam, *t, return_depth=True)
    pre, feats, ids, ranges, r = oracle_forward(cam, scene.means, scene.quats, scene.scales,
                                                scene.opacities, colors=scene.features,
                                                depth=True)
    say(f"  D={ids.shape[0]}")
    np.testing.assert_array_equal(host(out["sorted_ids"]), ids)
    np.testing.assert_array_equal(host(out["n_contrib"]), r["n_contrib"])
    assert_features(host(out["features"]), r["image"], "features")
    assert_bits(host(out["depth"]), r["depth"], "depth")
    target = scene.target(cam)
    (out["features"] - cu(target)).abs().mean().backward()
    g_img = (np.sign(r["image"] - target) / np.float32(target.size)).astype(np.float32)
    g = oracle_backward(cam, scene.means, scene.quats, scene.scales, scene.opacities, pre, feats,
                        ids, ranges, r, g_img, None)
    for name, a, key in [("means", t[0], "means"), ("quats", t[1], "quats"),
                         ("scales", t[2], "scales"), ("opacities", t[3], "opacities"),
                         ("features", t[4], "features")]:
        e = rel_err(host(a.grad), g[key])
        say(f"  grad {name}: rel {e:.2e}")
        assert e < 1e-3


def test_repeat_render_is_deterministic_forward():
    scene = scenes.make_scene(2)
    model = _model(scene)
    with torch.no_grad():
        a = model.render(scene.cameras[0])
        b = model.render(scene.cameras[0])
    np.testing.assert_array_equal(host(a["sorted_ids"]), host(b["sorted_ids"]))
    assert_bits(host(a["image"]), host(b["image"]), "repeat image")
