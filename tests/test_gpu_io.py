"""GPU side of the PLY checkpoint path: a saved model reloads onto the
device bit for bit (the one-copy table path), renders identically, and the
load / save rates at 1M Gaussians (SH3, 236 MB) are reported."""

from __future__ import annotations

import os
import time

import numpy as np
import pytest
import torch

from gpu_util import cu, host, say
from mlx3d_amd.splatting import GaussianModel
from refimpl import random_scene

pytestmark = pytest.mark.gpu


def test_ply_reload_renders_identically(tmp_path):
    cam, means, quats, scales, opac, _ = random_scene(61, n=3000, width=128, height=96)
    rng = np.random.default_rng(61)
    sh = (rng.standard_normal((3000, 16, 3)) * 0.2).astype(np.float32)
    lo = np.log(opac / (1 - opac)).astype(np.float32)
    model = GaussianModel({"means": cu(means), "quats": cu(quats),
                           "scales": cu(np.log(scales).astype(np.float32)), "opacities": cu(lo),
                           "sh_dc": cu(sh[:, :1].copy()), "sh_rest": cu(sh[:, 1:].copy())})
    model.active_sh_degree = 3
    p = str(tmp_path / "m.ply")
    model.save_ply(p)
    loaded = GaussianModel.load_ply(p)
    assert loaded.params["means"].device.type == "cuda"
    a = host(model.render(cam)["image"])
    b = host(loaded.render(cam)["image"])
    np.testing.assert_array_equal(a, b)


def test_ply_checkpoint_rates_1m(tmp_path):
    n = 1_000_000
    g = torch.Generator(device="cuda").manual_seed(0)
    params = {"means": torch.randn((n, 3), device="cuda", generator=g),
              "scales": torch.randn((n, 3), device="cuda", generator=g) - 4.0,
              "quats": torch.randn((n, 4), device="cuda", generator=g),
              "opacities": torch.randn((n,), device="cuda", generator=g),
              "sh_dc": torch.randn((n, 1, 3), device="cuda", generator=g),
              "sh_rest": torch.randn((n, 15, 3), device="cuda", generator=g)}
    model = GaussianModel(params)
    p = str(tmp_path / "big.ply")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    model.save_ply(p)
    t1 = time.perf_counter()
    loaded = GaussianModel.load_ply(p)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    mb = os.path.getsize(p) / 1e6
    say(f"PLY 1M SH3 ({mb:.0f} MB): save {t1 - t0:.3f} s ({mb / (t1 - t0):.0f} MB/s), "
        f"load to GPU {t2 - t1:.3f} s ({mb / (t2 - t1):.0f} MB/s)")
    for k in params:
        assert torch.equal(loaded.params[k], params[k]), k
