"""Host-side behaviour of the drop-in API that needs no GPU: argument
validation raises the reference's ValueErrors before any kernel, and CPU
tensors are refused rather than silently computed elsewhere."""

import numpy as np
import pytest
import torch

from mlx3d_amd.cameras import Camera
from mlx3d_amd.renderer import Renderer
from mlx3d_amd.splatting import (GaussianModel, bin_gaussians, num_sh_bases, project_gaussians,
                                 rasterize_features, render_gaussian_features, render_gaussians,
                                 rgb_to_sh, sh_to_rgb)


def _scene(n=10):
    g = torch.Generator().manual_seed(0)
    return (torch.randn(n, 3, generator=g) * 0.3, torch.randn(n, 4, generator=g),
            torch.full((n, 3), 0.05), torch.full((n,), 0.5), torch.rand(n, 3, generator=g))


def test_sh_helpers():
    rgb = torch.rand(10, 3)
    assert torch.allclose(sh_to_rgb(rgb_to_sh(rgb)), rgb, atol=1e-6)
    assert num_sh_bases(3) == 16


def test_exactly_one_of_colors_or_sh():
    cam = Camera.look_at(eye=(0, 0, -3.0), width=32, height=32)
    m, q, s, o, c = _scene()
    with pytest.raises(ValueError, match="exactly one"):
        render_gaussians(cam, m, q, s, o)
    with pytest.raises(ValueError, match="exactly one"):
        render_gaussians(cam, m, q, s, o, colors=c, sh=torch.zeros(10, 16, 3))


def test_projection_name_validated():
    cam = Camera.look_at(eye=(0, 0, -3.0), width=32, height=32)
    m, q, s, o, c = _scene()
    with pytest.raises(ValueError, match="projection"):
        render_gaussians(cam, m, q, s, o, colors=c, projection="bad")


def test_feature_shape_validation():
    cam = Camera.look_at(eye=(0, 0, -3.0), width=32, height=32)
    m, q, s, o, c = _scene()
    with pytest.raises(ValueError, match="features must have shape"):
        render_gaussian_features(cam, m, q, s, o, c[:, 0])
    with pytest.raises(ValueError, match="same first dimension"):
        render_gaussian_features(cam, m, q, s, o, c[:-1])
    with pytest.raises(ValueError, match="at least one channel"):
        rasterize_features(torch.zeros(10, 2), torch.zeros(10, 3), torch.zeros(10, 0),
                           torch.zeros(10), torch.zeros(0, dtype=torch.int32),
                           torch.zeros(4, 2, dtype=torch.int32), 32, 32, 2, 2)


def test_cpu_tensors_are_refused():
    cam = Camera.look_at(eye=(0, 0, -3.0), width=32, height=32)
    m, q, s, o, c = _scene()
    with pytest.raises(ValueError, match="GPU only"):
        render_gaussians(cam, m, q, s, o, colors=c)
    with pytest.raises(ValueError, match="GPU only"):
        project_gaussians(cam, m, q, s)
    with pytest.raises(ValueError, match="GPU only"):
        bin_gaussians(torch.zeros(4, 2), torch.ones(4), torch.ones(4), 32, 32)


def test_missing_library_raises(monkeypatch, tmp_path):
    """Without a built libgsx.so the package raises on first use; there is
    no other compute path to fall back to."""
    from mlx3d_amd import _lib
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libgsx.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(ImportError, match="no fallback compute path"):
        _lib.load()
    with pytest.raises(ImportError, match="is missing"):
        _lib.strerror(0)


@pytest.mark.gpu
def test_model_from_points_scales_and_layout():
    pts = torch.tensor([[0.0, 0, 0], [1.0, 0, 0], [0, 2.0, 0], [0, 0, 3.0], [1.0, 1.0, 0]])
    model = GaussianModel.from_points(pts, sh_degree=2)
    assert model.num_gaussians == 5
    assert model.sh.shape == (5, 9, 3)
    assert model.active_sh_degree == 0
    # point 0: nearest squared distances 1, 2, 4 -> mean 7/3
    np.testing.assert_allclose(float(model.scales_act[0, 0]), np.sqrt(7 / 3), rtol=1e-5)
    np.testing.assert_allclose(float(model.opacities_act[0]), 0.1, rtol=1e-5)
    capped = GaussianModel.from_points(pts * 100, sh_degree=0, scale_init_max_scale=0.25)
    assert float(capped.scales_act.max()) <= 0.250001


def test_render_function_is_a_renderer():
    assert isinstance(render_gaussians, Renderer)


# The public names of the reference's mlx3d.splatting (splatting/__init__.py:10-30).
_REFERENCE_SPLATTING_ALL = {
    "GaussianModel", "GaussianTrainer", "TILE_SIZE", "TrainerConfig", "bin_gaussians",
    "eval_sh", "num_sh_bases", "project_gaussians", "project_gaussians_ut",
    "quat_scale_to_cov3d", "rasterize", "rasterize_depth", "rasterize_features",
    "render_gaussian_depth", "render_gaussian_features", "render_gaussians",
    "render_gaussians_reference", "rgb_to_sh", "sh_to_rgb",
}


def test_splatting_exports_cover_the_reference():
    import mlx3d_amd.splatting as S

    assert _REFERENCE_SPLATTING_ALL <= set(S.__all__)
    for name in _REFERENCE_SPLATTING_ALL:
        assert getattr(S, name) is not None


def test_quat_scale_to_cov3d_closed_form():
    from mlx3d_amd.splatting import quat_scale_to_cov3d

    # 90 degrees about z (unnormalised quaternion): diag(1, 4, 9) -> diag(4, 1, 9)
    q = torch.tensor([[2.0, 0.0, 0.0, 2.0]])
    s = torch.tensor([[1.0, 2.0, 3.0]])
    cov = quat_scale_to_cov3d(q, s)
    np.testing.assert_allclose(cov[0].numpy(), np.diag([4.0, 1.0, 9.0]), atol=1e-5)
    g = torch.Generator().manual_seed(3)
    q = torch.randn(64, 4, generator=g)
    s = torch.rand(64, 3, generator=g) + 0.1
    cov = quat_scale_to_cov3d(q, s).double()
    # symmetric positive definite with determinant prod(s^2)
    np.testing.assert_allclose(cov.numpy(), cov.transpose(1, 2).numpy(), atol=1e-6)
    np.testing.assert_allclose(torch.linalg.det(cov).numpy(),
                               (s.double() ** 2).prod(1).numpy(), rtol=1e-4)


def test_unprojection_cache_follows_camera_content():
    """The 2DGS unprojection maps are cached per camera *content*: a camera
    edited in place (same id()) or a fresh camera gets fresh maps."""
    from types import SimpleNamespace

    from mlx3d_amd.splatting.geometry import unprojection_maps
    from mlx3d_amd.splatting.trainer import GaussianTrainer

    holder = SimpleNamespace(_unproject=None)
    cam = Camera.look_at(eye=(0, 0, -3.0), width=24, height=16)
    base0, dir0 = GaussianTrainer._maps(holder, cam, "cpu")
    other = Camera.look_at(eye=(1.0, 0.5, -3.0), width=24, height=16)
    cam.R, cam.t = other.R.clone(), other.t.clone()  # moved in place: same id()
    base1, dir1 = GaussianTrainer._maps(holder, cam, "cpu")
    want_b, want_d = unprojection_maps(cam, "cpu")
    assert torch.equal(base1, want_b) and torch.equal(dir1, want_d)
    assert not torch.equal(base0, base1)
    cam.fx *= 1.5  # intrinsics edited in place
    base2, dir2 = GaussianTrainer._maps(holder, cam, "cpu")
    assert torch.equal(dir2, unprojection_maps(cam, "cpu")[1]) and not torch.equal(dir1, dir2)
    # an equal camera reuses the cached maps (no rebuild)
    assert GaussianTrainer._maps(holder, cam, "cpu")[0] is base2


def test_adam_schedule_advances_only_after_launch():
    """FusedAdam holds the current rates and advances each optimiser once, on
    commit(); adam_step advances only after its launch, so an update that
    raised before launching leaves the schedule where it was."""
    from mlx3d_amd.optim import Adam, FusedAdam, adam_step, exponential_decay

    opt = Adam(learning_rate=exponential_decay(1e-2, 0.5), eps=1e-15)
    p = torch.zeros(8)
    fused = FusedAdam([(opt, "p", p)])
    assert opt.step == 0 and fused.records[0].lr == np.float32(1e-2)
    fused.commit()
    fused.commit()  # once only
    assert opt.step == 1 and opt.learning_rate == 1e-2
    fused = FusedAdam([(opt, "p", p)])
    assert fused.records[0].lr == np.float32(0.5e-2) and opt.step == 1  # not committed: no advance
    with pytest.raises(ValueError):  # CPU tensors are refused before any launch
        adam_step([(opt, {"p": torch.ones(8)}, {"p": p})])
    assert opt.step == 1 and opt.learning_rate == 1e-2
