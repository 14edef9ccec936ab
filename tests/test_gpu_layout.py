"""The spatial row order (GaussianModel.reorder_spatial, TrainerConfig
.spatial_order) changes no rendered value: the image, final_T, alpha and
n_contrib of a reordered table are bit-identical to the original's when no
two drawn Gaussians share a depth (a tied pair may composite in the other
order, since the depth sort breaks ties by row: then within 1e-5), the
per-Gaussian outputs are the same rows permuted, and the gradients are the
original's permuted within float32 summation-order noise (the backward's
atomics add a Gaussian's per-tile contributions in another order)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import assert_bits, cu, host, rel_err, say
from mlx3d_amd import scenes
from mlx3d_amd.losses import l1_loss
from mlx3d_amd.splatting import GaussianModel
from mlx3d_amd.splatting.trainer import GaussianTrainer, TrainerConfig

pytestmark = pytest.mark.gpu


def _model(scene, n=None):
    sl = slice(0, n)
    m = GaussianModel({"means": cu(scene.means[sl]), "quats": cu(scene.quats[sl]),
                       "scales": cu(scene.log_scales[sl]),
                       "opacities": cu(scene.logit_opacities[sl]),
                       "sh_dc": cu(scene.sh_dc[sl]), "sh_rest": cu(scene.sh_rest[sl])},
                      sh_degree=3)
    m.active_sh_degree = scene.sh_degree
    return m


def _render_and_grads(model, cam, target, antialias):
    model.requires_grad_(True)
    out = model.render(cam, antialias=antialias)
    loss = l1_loss(out["image"], target)
    loss.backward()
    grads = {k: host(v.grad) for k, v in model.params.items()}
    return {k: host(v) for k, v in out.items() if torch.is_tensor(v)}, grads


@pytest.mark.parametrize("config,n,view", [(2, 20000, 0), (3, 60000, 3)])
def test_reorder_changes_no_render(config, n, view):
    say(f"spatial order: config {config} n={n} view={view}")
    scene = scenes.make_scene(config)
    cam = scene.cameras[view]
    target = cu(scene.target(cam))
    a = _model(scene, n)
    out_a, g_a = _render_and_grads(a, cam, target, scene.antialias)
    b = _model(scene, n)
    perm = b.reorder_spatial()
    assert not torch.equal(perm, torch.arange(perm.numel(), device=perm.device))
    out_b, g_b = _render_and_grads(b, cam, target, scene.antialias)
    p = host(perm)
    # per-pixel outputs: bit-identical when no two drawn Gaussians share a
    # depth; otherwise such a pair may composite in the other order
    d = out_a["depths"][out_a["radii"] > 0]
    ties = len(d) - len(np.unique(d))
    say(f"  {len(d)} drawn Gaussians, {ties} depth ties")
    if ties == 0:
        for k in ("image", "final_T", "alpha"):
            assert_bits(out_b[k], out_a[k], k)
        assert np.array_equal(out_b["n_contrib"], out_a["n_contrib"])
    else:
        for k in ("image", "final_T", "alpha"):
            assert np.abs(out_b[k] - out_a[k]).max() < 1e-5, k
        assert (out_b["n_contrib"] != out_a["n_contrib"]).mean() < 1e-3
    # per-Gaussian outputs: the same rows, permuted
    for k in ("means2d", "radii"):
        assert_bits(out_b[k], out_a[k][p], k)
    # gradients: permuted, within summation-order noise
    for k in g_a:
        err = rel_err(g_b[k], g_a[k][p])
        assert err < 1e-5, (k, err)


def test_trainer_keeps_moments_with_their_rows():
    scene = scenes.make_scene(2)
    cam = scene.cameras[0]
    target = cu(scene.target(cam))
    model = _model(scene, 5000)
    big = 1 << 30
    cfg = TrainerConfig(densify_from=big, densify_until=big, opacity_reset_every=big,
                        sh_increase_every=big, spatial_order=True)
    tr = GaussianTrainer(model, cfg)
    # the table is in spatial order from the start (sorting it again is the identity)
    from mlx3d_amd.splatting import spatial_order

    n = model.num_gaussians
    ident = torch.arange(n, device=model.params["means"].device)
    assert torch.equal(spatial_order(model.params["means"]), ident)
    tr.step(cam, target)
    # scramble the rows (a stand-in for a density event's appended rows),
    # moments alongside, then reorder: every moment row follows its Gaussian
    g = torch.Generator(device="cpu").manual_seed(5)
    shuf = torch.randperm(n, generator=g).to(ident.device)
    with torch.no_grad():
        model._replace({k: v[shuf] for k, v in model.params.items()})
    for name, opt in tr.optimizers.items():
        st = opt.state[name]
        st["m"], st["v"] = st["m"][shuf].contiguous(), st["v"][shuf].contiguous()
    means_before = model.params["means"].detach().clone()
    m_before = {k: tr.optimizers[k].state[k]["m"].clone() for k in tr.optimizers}
    tr._reorder()
    perm = spatial_order(means_before)
    assert torch.equal(model.params["means"].detach(), means_before[perm])
    for k in tr.optimizers:
        assert torch.equal(tr.optimizers[k].state[k]["m"], m_before[k][perm]), k
    res = tr.step(cam, target)
    assert np.isfinite(res["loss"])
