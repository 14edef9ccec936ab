"""GPU parity against the CPU oracle on the same seeded float32 inputs.

Bit-exact: exp, projection outputs, SH colour, fused preprocess, sorted ids,
tile ranges, n_contrib, image/final_T/depth (identical operation order on
both sides).  Gradients: max|d|/max|ref| < 1e-3 (the tolerance the
reference's own gradient test uses, test_splatting.py:390-414); the GPU
sums with float atomics in a different order than the oracle.
"""

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import (assert_bits, assert_features, cu, host, oracle_backward, oracle_forward,
                      rel_err, say)
from mlx3d_amd import _lib
from mlx3d_amd.splatting import (GaussianModel, bin_gaussians, eval_sh, project_gaussians,
                                 rasterize, rasterize_depth, rasterize_features,
                                 render_gaussian_depth, render_gaussian_features,
                                 render_gaussians)
from oracle import oracle as O
from refimpl import oracle_camera, random_scene

pytestmark = pytest.mark.gpu


def test_device_is_gfx950():
    buf = ctypes.create_string_buffer(64)
    rc = _lib.load().gsx_device_check(buf, 64)
    say(f"device arch {buf.value.decode()}")
    assert rc == 1


def test_exp_bitwise():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        np.linspace(-90.0, 90.0, 1_000_001, dtype=np.float32),
        rng.uniform(-10.0, 0.0, 1_000_000).astype(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -86.0, 88.0, 1e-30, -1e-30], np.float32),
    ])
    xt = cu(x)
    y = torch.empty_like(xt)
    _lib.check(_lib.load().gsx_debug_expf(x.size, _lib.ptr(xt), _lib.ptr(y),
                                          _lib.stream_handle(xt.device)), "exp")
    assert_bits(host(y), O.expf(x), "exp")


@pytest.mark.parametrize("antialias", [False, True])
def test_projection_bitexact(antialias):
    cam, means, quats, scales, opac, colors = random_scene(0, n=5000)
    means[:50, 2] = -6.0  # behind the camera
    means[50:100, 0] = 8.0  # off-screen: frustum clip active
    out = project_gaussians(cam, cu(means), cu(quats), cu(scales), antialias=antialias)
    ref = O.project(oracle_camera(cam), means, quats, scales, antialias=antialias)
    for k in ("means2d", "conics", "depths", "radii", "compensation"):
        assert_bits(host(out[k]), ref[k], k)


@pytest.mark.parametrize("antialias", [False, True])
def test_projection_vjp(antialias):
    cam, means, quats, scales, opac, colors = random_scene(1, n=3000)
    rng = np.random.default_rng(1)
    tm, tq, ts = (cu(a).requires_grad_(True) for a in (means, quats, scales))
    out = project_gaussians(cam, tm, tq, ts, antialias=antialias)
    g = {k: rng.standard_normal(out[k].shape).astype(np.float32)
         for k in ("means2d", "conics", "depths", "compensation")}
    loss = sum((out[k] * cu(v)).sum() for k, v in g.items())
    loss.backward()
    rm, rq, rs = O.project_bwd(oracle_camera(cam), means, quats, scales, g["means2d"],
                               g["conics"], g["depths"], g["compensation"], antialias=antialias)
    for name, a, b in [("means", tm.grad, rm), ("quats", tq.grad, rq), ("scales", ts.grad, rs)]:
        e = rel_err(host(a), b)
        say(f"project vjp {name}: rel {e:.2e}")
        assert e < 1e-5


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_eval_sh(degree):
    rng = np.random.default_rng(degree)
    n = 4000
    sh = (rng.standard_normal((n, 16, 3)) * 0.3).astype(np.float32)
    d = rng.standard_normal((n, 3))
    dirs = (d / np.linalg.norm(d, axis=1, keepdims=True)).astype(np.float32)
    tsh, td = cu(sh).requires_grad_(True), cu(dirs).requires_grad_(True)
    out = eval_sh(degree, tsh, td)
    assert_bits(host(out), O.eval_sh(degree, sh, dirs), "eval_sh")
    g = rng.standard_normal((n, 3)).astype(np.float32)
    (out * cu(g)).sum().backward()
    gsh, gd = O.eval_sh_bwd(degree, sh, dirs, g)
    assert rel_err(host(tsh.grad), gsh) < 1e-6
    assert rel_err(host(td.grad), gd) < 1e-5


def _bin_case(means2d, radii, depths, W, H, what):
    ids, ranges, tx, ty = bin_gaussians(cu(means2d), cu(radii), cu(depths), W, H)
    rids, rranges, rtx, rty = O.bin_gaussians(means2d, radii, depths, W, H, threads=8)
    say(f"binning {what}: D={rids.shape[0]}")
    assert (tx, ty) == (rtx, rty)
    np.testing.assert_array_equal(host(ranges), rranges)
    np.testing.assert_array_equal(host(ids), rids)


def test_binning_bitexact_scenes():
    for seed in range(3):
        cam, means, quats, scales, opac, colors = random_scene(seed, n=20000, width=640,
                                                               height=360)
        p = O.project(oracle_camera(cam), means, quats, scales)
        _bin_case(p["means2d"], p["radii"], p["depths"], cam.width, cam.height, f"seed {seed}")


def test_binning_edge_cases():
    W, H = 200, 120
    _bin_case(np.zeros((0, 2), np.float32), np.zeros(0, np.float32), np.zeros(0, np.float32),
              W, H, "empty")
    rng = np.random.default_rng(7)
    m = rng.uniform(0, 200, (500, 2)).astype(np.float32)
    _bin_case(m, np.zeros(500, np.float32), np.ones(500, np.float32), W, H, "all culled")
    # exact depth ties everywhere
    _bin_case(m, rng.integers(1, 30, 500).astype(np.float32),
              rng.choice(np.array([1.0, 2.0, 3.0], np.float32), 500), W, H, "ties")
    # one splat covering every tile plus a few small ones
    m2 = np.concatenate([[[100.0, 60.0]], m[:20]]).astype(np.float32)
    r2 = np.concatenate([[1e5], np.full(20, 5.0)]).astype(np.float32)
    _bin_case(m2, r2, rng.uniform(1, 2, 21).astype(np.float32), W, H, "huge splat")
    # a single tile image
    _bin_case(m[:50] * 0.05, np.full(50, 3.0, np.float32), rng.uniform(1, 2, 50).astype(np.float32),
              8, 8, "one tile")


def test_binning_culled_owners_and_clusters():
    """Long runs of zero-count (off-screen) Gaussians between owners in depth
    order (emission's unstaged owner search), and splats clustered over a few
    tiles (long per-tile runs)."""
    rng = np.random.default_rng(21)
    W, H = 640, 360
    n = 120000
    m = rng.uniform(0, [W, H], (n, 2)).astype(np.float32)
    m[::2, 0] += 5000.0  # every other Gaussian off-screen: count 0, valid depth
    r = rng.integers(1, 60, n).astype(np.float32)
    d = rng.uniform(1, 10, n).astype(np.float32)
    _bin_case(m, r, d, W, H, "culled owners")
    # clustered: most splats over a few tiles (long per-tile runs in a sub-chunk)
    m2 = (rng.normal(0, 6, (60000, 2)) + [320, 180]).astype(np.float32)
    _bin_case(m2, rng.integers(1, 12, 60000).astype(np.float32),
              rng.choice(np.linspace(1, 3, 50), 60000).astype(np.float32), W, H, "cluster")


def test_binning_large_image():
    """Images with more tiles than 14 bits of tile id (three radix passes
    over the tile ids) and just below, against the oracle's order."""
    rng = np.random.default_rng(22)
    W, H = 2112, 2064  # 132 x 129 = 17028 tiles (15 significant bits)
    n = 40000
    m = rng.uniform(-50, [W + 50, H + 50], (n, 2)).astype(np.float32)
    r = rng.integers(0, 80, n).astype(np.float32)
    d = rng.uniform(0.5, 8, n).astype(np.float32)
    _bin_case(m, r, d, W, H, "large image")
    W2, H2 = 2032, 2048  # 127 x 128 = 16256 tiles
    _bin_case(m, r, d, W2, H2, "16256 tiles")


def test_bin_sort_sync_abi_and_capacity():
    """gsx_bin_sort (the synchronous entry point) at exact, short and zero
    capacity: short capacity returns 1 with the true D; exact matches the
    oracle bit for bit."""
    cam, means, quats, scales, opac, colors = random_scene(4, n=30000, width=640, height=360)
    p = O.project(oracle_camera(cam), means, quats, scales)
    rids, rranges, tx, ty = O.bin_gaussians(p["means2d"], p["radii"], p["depths"], 640, 360,
                                            threads=8)
    D = rids.shape[0]
    say(f"sync bin_sort: D={D}")
    n = means.shape[0]
    L = _lib.load()
    dev = torch.device("cuda")
    counts = torch.empty(n, dtype=torch.int32, device=dev)
    dkeys = torch.empty(n, dtype=torch.int32, device=dev)
    rects = torch.empty((n, 2), dtype=torch.int32, device=dev)
    st = _lib.stream_handle(dev)
    m2, rad, dep = cu(p["means2d"]), cu(p["radii"]), cu(p["depths"])  # alive past the launch
    _lib.check(L.gsx_bin_prepare(n, _lib.ptr(m2), _lib.ptr(rad), _lib.ptr(dep), 640, 360,
                                 _lib.ptr(counts), _lib.ptr(dkeys), _lib.ptr(rects), st),
               "prepare")
    ranges = torch.empty((tx * ty, 2), dtype=torch.int32, device=dev)
    for cap, want in [(D - 1, 1), (0, 1), (D, 0), (D + 5000, 0)]:
        ws = torch.empty(L.gsx_bin_workspace_bytes(n, cap, tx * ty), dtype=torch.uint8,
                         device=dev)
        ids = torch.full((max(cap, 1),), -1, dtype=torch.int32, device=dev)
        nd = ctypes.c_int64(0)
        rc = L.gsx_bin_sort(n, _lib.ptr(counts), _lib.ptr(dkeys), _lib.ptr(rects), None, None, 0,
                            640, 360, _lib.ptr(ws), ws.numel(), cap, _lib.ptr(ids),
                            _lib.ptr(ranges), ctypes.byref(nd), st)
        say(f"  capacity {cap}: rc={rc} D={nd.value}")
        assert rc == want and nd.value == D
        if rc == 0:
            np.testing.assert_array_equal(host(ids[:D]), rids)
            np.testing.assert_array_equal(host(ranges), rranges)


def test_bin_two_phase_abi_exact_capacity():
    """gsx_bin_count_async reports the emitted duplicate count in
    bin_status[3] (and the row entries in [4]) before the sorts run;
    gsx_bin_depth_async publishes those words to pinned host memory tagged
    with the caller's sequence number; gsx_bin_tiles_async with that
    capacity matches the oracle bit for bit, plain (row placement) and with
    refine_tiles (general path), and publishes the final words."""
    from mlx3d_amd.splatting.tiles import _HostStatus

    m, r, d, co = _elongated(9, n=4000)
    n = m.shape[0]
    L = _lib.load()
    dev = torch.device("cuda")
    st = _lib.stream_handle(dev)
    m2, rad, dep, con = cu(m), cu(r), cu(d), cu(co)  # alive past the launches
    counts = torch.empty(n, dtype=torch.int32, device=dev)
    dkeys = torch.empty(n, dtype=torch.int32, device=dev)
    rects = torch.empty((n, 2), dtype=torch.int32, device=dev)
    _lib.check(L.gsx_bin_prepare(n, _lib.ptr(m2), _lib.ptr(rad), _lib.ptr(dep), 640, 360,
                                 _lib.ptr(counts), _lib.ptr(dkeys), _lib.ptr(rects), st),
               "prepare")
    hr = host(rects).view(np.uint32)
    heights = int(((hr[:, 1] >> 16) * (host(counts) > 0)).sum())
    full, _, tx, ty = O.bin_gaussians(m, r, d, 640, 360, threads=8)
    hs = _HostStatus()
    for seq, refine in ((7, False), (8, True)):
        rids, rranges, _, _ = O.bin_gaussians(m, r, d, 640, 360, threads=8,
                                              conics=co if refine else None)
        say(f"two-phase binning refine={refine}: emitted {full.shape[0]}, kept {rids.shape[0]}")
        dws = torch.empty(L.gsx_bin_depth_workspace_bytes(n), dtype=torch.uint8, device=dev)
        ranges = torch.empty((tx * ty, 2), dtype=torch.int32, device=dev)
        # words 0 and 2..7 are cleared by the count call, the error word is not
        status = torch.tensor([-1, 0, -1, -1, -1, -1, -1, -1], dtype=torch.int32, device=dev)
        _lib.check(L.gsx_bin_count_async(n, _lib.ptr(counts), _lib.ptr(dkeys), _lib.ptr(rects),
                                         640, 360, _lib.ptr(dws), dws.numel(), _lib.ptr(ranges),
                                         _lib.ptr(status), st), "count")
        words = host(status).view(np.uint32)
        assert words[0] == words[1] == words[2] == 0 and (words[5:] == 0).all()
        assert words[3] == full.shape[0] == int(host(counts).sum())
        assert words[4] == heights
        _lib.check(L.gsx_bin_depth_async(n, _lib.ptr(dkeys), _lib.ptr(dws), dws.numel(),
                                         _lib.ptr(status), hs.slot(0), seq, st), "depth sort")
        pub, tag = hs.wait(0, seq)
        assert tag == seq and pub[3] == words[3] and pub[4] == heights and pub[1] == 0
        cap = int(pub[3])
        tws = torch.empty(L.gsx_bin_tile_workspace_bytes(cap, tx * ty), dtype=torch.uint8,
                          device=dev)
        ids = torch.full((cap,), -1, dtype=torch.int32, device=dev)
        _lib.check(L.gsx_bin_tiles_async(
            n, _lib.ptr(counts), _lib.ptr(rects), _lib.ptr(m2) if refine else None,
            _lib.ptr(con) if refine else None, 3 if refine else 0, 640, 360, _lib.ptr(dws),
            dws.numel(), _lib.ptr(tws), tws.numel(), cap, _lib.ptr(ids), _lib.ptr(ranges),
            _lib.ptr(status), hs.slot(1), seq, None, st), "tile phase")
        final, tag = hs.wait(1, seq)
        assert tag == seq
        words = host(status).view(np.uint32)
        nd = ctypes.c_int64(0)
        hw = np.ascontiguousarray(words)
        assert L.gsx_bin_status_check(hw.ctypes.data_as(ctypes.c_void_p), cap,
                                      ctypes.byref(nd)) == 0
        assert words[0] == cap and nd.value == rids.shape[0]
        if refine:  # the general path publishes after its tile passes: dropped is final
            np.testing.assert_array_equal(final[:3], words[:3])
        else:  # the row path publishes D with its placement kernel
            assert final[0] == cap and final[1] == 0
        np.testing.assert_array_equal(host(ids[:nd.value]), rids)
        np.testing.assert_array_equal(host(ranges), rranges)


def test_binning_error_bits_reported_once():
    """The renderer's binning reads the sticky error word with its count
    readback: an error bit set (here from the host, as a tile phase's
    bounded wait would set it) makes the next render raise, once."""
    from mlx3d_amd.splatting import tiles

    cam, means, quats, scales, opac, colors = random_scene(11, n=3000, width=320, height=240)
    t = [cu(a) for a in (means, quats, scales, opac, colors)]
    a = render_gaussians(cam, *t[:4], colors=t[4])
    dev = t[0].device
    ws = tiles._workspace_for(dev, _lib.stream_handle(dev))
    ws.status[1] = 1  # GSX_BIN_ERR_LOOKBACK
    with pytest.raises(_lib.GsxError, match="device-side check"):
        render_gaussians(cam, *t[:4], colors=t[4])
    b = render_gaussians(cam, *t[:4], colors=t[4])
    assert_bits(host(b["image"]), host(a["image"]), "image after the reported error")


def test_render_alpha_output_and_gradient():
    """alpha comes from the forward kernel (bit-identical to 1 - final_T) and
    its cotangent reaches the rasterizer as -grad_alpha: a loss on alpha
    and final_T gives the gradients of the same loss written on final_T."""
    cam, means, quats, scales, opac, colors = random_scene(12, n=3000, width=320, height=240)
    rng = np.random.default_rng(12)
    w1, w2 = (cu(rng.normal(size=(240, 320)).astype(np.float32)) for _ in range(2))
    grads = []
    for via_alpha in (True, False):
        t = [cu(a).requires_grad_(True) for a in (means, quats, scales, opac, colors)]
        out = render_gaussians(cam, *t[:4], colors=t[4], antialias=True)
        if via_alpha:
            assert_bits(host(out["alpha"]), host(1.0 - out["final_T"]), "alpha")
            a = out["alpha"]
        else:
            a = 1.0 - out["final_T"]
        loss = (a * w1).sum() + (out["final_T"] * w2).sum() + out["image"].sum()
        grads.append(torch.autograd.grad(loss, t))
    for name, ga, gb in zip(("means", "quats", "scales", "opacities", "colors"), *grads):
        err = rel_err(host(ga), host(gb))
        say(f"alpha path {name}: rel err {err:.2e}")
        assert err < 1e-5, name


def _elongated(seed, n=3000, width=640, height=360):
    rng = np.random.default_rng(seed)
    means2d = rng.uniform(-20, [width + 20, height + 20], (n, 2)).astype(np.float32)
    sig_major = rng.uniform(3.0, 40.0, n)
    sig_minor = rng.uniform(0.4, 2.0, n)
    th = rng.uniform(0, np.pi, n)
    c, s = np.cos(th), np.sin(th)
    cov = np.stack([c * c * sig_major**2 + s * s * sig_minor**2,
                    c * s * (sig_major**2 - sig_minor**2),
                    s * s * sig_major**2 + c * c * sig_minor**2], 1)
    det = cov[:, 0] * cov[:, 2] - cov[:, 1] ** 2
    conics = np.stack([cov[:, 2] / det, -cov[:, 1] / det, cov[:, 0] / det], 1).astype(np.float32)
    radii = np.ceil(3.0 * sig_major).astype(np.float32)
    depths = rng.choice(np.linspace(1, 5, 40), n).astype(np.float32)  # some depth ties
    return means2d, radii, depths, conics


def test_binning_refine_tiles_bitexact():
    for seed in range(2):
        m, r, d, co = _elongated(seed)
        ids, ranges, tx, ty = bin_gaussians(cu(m), cu(r), cu(d), 640, 360, conics=cu(co))
        rids, rranges, _, _ = O.bin_gaussians(m, r, d, 640, 360, threads=8, conics=co)
        full, _, _, _ = O.bin_gaussians(m, r, d, 640, 360, threads=8)
        say(f"refine seed {seed}: D={rids.shape[0]} of {full.shape[0]}")
        np.testing.assert_array_equal(host(ranges), rranges)
        np.testing.assert_array_equal(host(ids), rids)


def test_render_refine_tiles_same_image_fewer_pairs():
    cam, means, quats, scales, opac, colors = random_scene(6, n=4000, width=320, height=240)
    scales[:, 0] *= 8.0  # elongated splats: square boxes cover many unreachable tiles
    t = [cu(a) for a in (means, quats, scales, opac, colors)]
    a = render_gaussians(cam, *t[:4], colors=t[4], antialias=True)
    b = render_gaussians(cam, *t[:4], colors=t[4], antialias=True, refine_tiles=True)
    assert_bits(host(a["image"]), host(b["image"]), "image")
    assert_bits(host(a["final_T"]), host(b["final_T"]), "final_T")
    assert b["sorted_ids"].shape[0] < a["sorted_ids"].shape[0]
    p = O.project(oracle_camera(cam), means, quats, scales, antialias=True)
    oe = (opac * p["compensation"]).astype(np.float32)
    ids, ranges, _, _ = O.bin_gaussians(p["means2d"], p["radii"], p["depths"], 320, 240,
                                        conics=p["conics"])
    r = O.raster_fwd(p["means2d"], p["conics"], oe, colors, ids, ranges, 320, 240)
    say(f"refine render: D {a['sorted_ids'].shape[0]} -> {b['sorted_ids'].shape[0]}")
    np.testing.assert_array_equal(host(b["sorted_ids"]), ids)
    np.testing.assert_array_equal(host(b["n_contrib"]), r["n_contrib"])


def test_rasterize_building_block_bitexact():
    cam, means, quats, scales, opac, colors = random_scene(2, n=3000, width=200, height=150)
    p = O.project(oracle_camera(cam), means, quats, scales)
    ids, ranges, tx, ty = O.bin_gaussians(p["means2d"], p["radii"], p["depths"], 200, 150)
    bg = np.array([0.1, 0.2, 0.3], np.float32)
    out = rasterize(cu(p["means2d"]), cu(p["conics"]), cu(colors), cu(opac), cu(ids), cu(ranges),
                    200, 150, tx, ty, background=cu(bg))
    ref = O.raster_fwd(p["means2d"], p["conics"], opac, colors, ids, ranges, 200, 150, bg=bg)
    np.testing.assert_array_equal(host(out["n_contrib"]), ref["n_contrib"])
    assert_bits(host(out["image"]), ref["image"], "image")
    assert_bits(host(out["final_T"]), ref["final_T"], "final_T")
    d = rasterize_depth(cu(p["means2d"]), cu(p["conics"]), cu(opac), cu(p["depths"]), cu(ids),
                        cu(ranges), 200, 150, tx, ty)
    refd = O.raster_fwd(p["means2d"], p["conics"], opac, p["depths"][:, None], ids, ranges,
                        200, 150, depths=p["depths"])
    assert_bits(host(d["depth"]), refd["depth"], "depth")


@pytest.mark.parametrize("channels", [3, 12, 32])
def test_rasterize_non_plain_batches(channels):
    """Batches holding a Gaussian outside the rasterizers' fast-path range
    (a mean 2e6 px away; a 1e21 conic centred on a pixel, which takes G = 1
    there and exp underflow everywhere else) run the kernels' general
    path, with range-checked exp and selects, for every Gaussian of the
    batch: image and n_contrib bit-exact, gradients <= 1e-3 against the
    oracle.  Four tiles list all Gaussians, as a caller of the building
    block may."""
    W = H = 32
    n = 90
    rng = np.random.default_rng(41 + channels)
    m2 = rng.uniform(0.0, 32.0, (n, 2)).astype(np.float32)
    s = rng.uniform(0.5, 4.0, n)
    con = np.stack([1 / s ** 2, rng.uniform(-0.2, 0.2, n) / s ** 2, 1 / s ** 2], 1)
    con = con.astype(np.float32)
    op = rng.uniform(0.05, 0.9, n).astype(np.float32)
    m2[3] = [2.0e6, 8.0]
    m2[1] = [8.5, 8.5]
    con[1] = [1e21, 0.0, 1e21]
    op[1] = 0.6
    feats = rng.uniform(0.0, 1.0, (n, channels)).astype(np.float32)
    ids = np.arange(n, dtype=np.int32)
    ranges = np.tile(np.array([[0, n]], np.int32), (4, 1))
    t = [cu(a).requires_grad_(True) for a in (m2, con, feats, op)]
    if channels == 3:
        out = rasterize(*t, cu(ids), cu(ranges), W, H, 2, 2)
        img = out["image"]
    else:
        out = rasterize_features(*t, cu(ids), cu(ranges), W, H, 2, 2)
        img = out["features"]
    ref = O.raster_fwd(m2, con, op, feats, ids, ranges, W, H)
    np.testing.assert_array_equal(host(out["n_contrib"]), ref["n_contrib"])
    assert_features(host(img), ref["image"], "image")
    assert_bits(host(out["final_T"]), ref["final_T"], "final_T")
    g_img = rng.standard_normal(ref["image"].shape).astype(np.float32)
    g_a = rng.standard_normal(ref["final_T"].shape).astype(np.float32)
    ((img * cu(g_img)).sum() + (out["alpha"] * cu(g_a)).sum()).backward()
    rg = O.raster_bwd(m2, con, op, feats, ids, ranges, W, H, ref["final_T"], ref["n_contrib"],
                      g_img, grad_final_T=-g_a)
    for name, a, key in [("means2d", t[0], "means2d"), ("conics", t[1], "conics"),
                         ("features", t[2], "features"), ("opacities", t[3], "opacities")]:
        g = host(a.grad)
        assert np.isfinite(g).all(), name
        e = rel_err(g, rg[key])
        say(f"non-plain C={channels} grad {name}: rel {e:.2e}")
        assert e < 1e-3
    # the pixel-centred Gaussian composites (at its own pixel only)
    assert float(host(t[3].grad)[1]) != 0.0


def test_rasterize_backward():
    cam, means, quats, scales, opac, colors = random_scene(3, n=3000, width=200, height=150)
    p = O.project(oracle_camera(cam), means, quats, scales)
    ids, ranges, tx, ty = O.bin_gaussians(p["means2d"], p["radii"], p["depths"], 200, 150)
    bg = np.array([0.3, 0.1, 0.2], np.float32)
    rng = np.random.default_rng(3)
    g_img = rng.standard_normal((150, 200, 3)).astype(np.float32)
    g_a = rng.standard_normal((150, 200)).astype(np.float32)
    t = [cu(a).requires_grad_(True) for a in (p["means2d"], p["conics"], colors, opac)]
    out = rasterize(*t, cu(ids), cu(ranges), 200, 150, tx, ty, background=cu(bg))
    ((out["image"] * cu(g_img)).sum() + (out["alpha"] * cu(g_a)).sum()).backward()
    ref = O.raster_fwd(p["means2d"], p["conics"], opac, colors, ids, ranges, 200, 150, bg=bg)
    rg = O.raster_bwd(p["means2d"], p["conics"], opac, colors, ids, ranges, 200, 150,
                      ref["final_T"], ref["n_contrib"], g_img, grad_final_T=-g_a, bg=bg)
    for name, a, key in [("means2d", t[0], "means2d"), ("conics", t[1], "conics"),
                         ("colors", t[2], "features"), ("opacities", t[3], "opacities")]:
        e = rel_err(host(a.grad), rg[key])
        say(f"raster bwd {name}: rel {e:.2e}")
        assert e < 1e-4


@pytest.mark.parametrize("antialias", [False, True])
def test_render_gaussians_colors(antialias):
    cam, means, quats, scales, opac, colors = random_scene(4, n=4000, width=160, height=96)
    bg = np.array([0.1, 0.2, 0.3], np.float32)
    flags = O.ANTIALIAS if antialias else 0
    opac = np.minimum(opac, 0.95).astype(np.float32)
    t = [cu(a).requires_grad_(True) for a in (means, quats, scales, opac, colors)]
    out = render_gaussians(cam, t[0], t[1], t[2], t[3], colors=t[4], background=cu(bg),
                           antialias=antialias, return_depth=True)
    pre, feats, ids, ranges, r = oracle_forward(cam, means, quats, scales, opac, colors=colors,
                                                flags=flags, bg=bg, depth=True)
    np.testing.assert_array_equal(host(out["sorted_ids"]), ids)
    np.testing.assert_array_equal(host(out["n_contrib"]), r["n_contrib"])
    for k, ref in [("image", r["image"]), ("final_T", r["final_T"]), ("depth", r["depth"]),
                   ("means2d", pre["means2d"]), ("depths", pre["depths"]), ("radii", pre["radii"]),
                   ("compensation", pre["compensation"])]:
        assert_bits(host(out[k]), ref, k)
    rng = np.random.default_rng(4)
    g_img = rng.standard_normal(r["image"].shape).astype(np.float32)
    g_a = rng.standard_normal(r["final_T"].shape).astype(np.float32)
    ((out["image"] * cu(g_img)).sum() + (out["alpha"] * cu(g_a)).sum()).backward()
    g = oracle_backward(cam, means, quats, scales, opac, pre, feats, ids, ranges, r, g_img, g_a,
                        flags=flags, bg=bg)
    for name, a, key in [("means", t[0], "means"), ("quats", t[1], "quats"),
                         ("scales", t[2], "scales"), ("opacities", t[3], "opacities"),
                         ("colors", t[4], "features")]:
        e = rel_err(host(a.grad), g[key])
        say(f"render colors aa={antialias} grad {name}: rel {e:.2e}")
        assert e < 1e-3


@pytest.mark.parametrize("degree", [0, 3])
def test_model_render_sh_raw_params(degree):
    cam, means, quats, scales, opac, _ = random_scene(5, n=5000, width=192, height=128)
    rng = np.random.default_rng(50 + degree)
    n = means.shape[0]
    sh = (rng.standard_normal((n, 16, 3)) * 0.2).astype(np.float32)
    ls = np.log(scales).astype(np.float32)
    lo = np.clip(rng.standard_normal(n), -4, 3).astype(np.float32)
    model = GaussianModel({"means": cu(means), "quats": cu(quats), "scales": cu(ls),
                           "opacities": cu(lo), "sh_dc": cu(sh[:, :1]),
                           "sh_rest": cu(sh[:, 1:])}, sh_degree=3)
    model.active_sh_degree = degree
    model.requires_grad_(True)
    out = model.render(cam)
    flags = O.LOG_SCALES | O.LOGIT_OPACITY
    pre, feats, ids, ranges, r = oracle_forward(cam, means, quats, ls, lo, sh=sh, degree=degree,
                                                flags=flags)
    np.testing.assert_array_equal(host(out["n_contrib"]), r["n_contrib"])
    assert_bits(host(out["image"]), r["image"], "image")
    assert_bits(host(out["means2d"]), pre["means2d"], "means2d")
    g_img = rng.standard_normal(r["image"].shape).astype(np.float32)
    g_a = rng.standard_normal(r["final_T"].shape).astype(np.float32)
    ((out["image"] * cu(g_img)).sum() + (out["alpha"] * cu(g_a)).sum()).backward()
    g = oracle_backward(cam, means, quats, ls, lo, pre, feats, ids, ranges, r, g_img, g_a, sh=sh,
                        degree=degree, flags=flags)
    p = model.params
    shg = np.concatenate([host(p["sh_dc"].grad), host(p["sh_rest"].grad)], 1)
    for name, a, b in [("means", host(p["means"].grad), g["means"]),
                       ("quats", host(p["quats"].grad), g["quats"]),
                       ("scales", host(p["scales"].grad), g["scales"]),
                       ("opacities", host(p["opacities"].grad), g["opacities"]),
                       ("sh", shg, g["sh"])]:
        e = rel_err(a, b)
        say(f"model sh{degree} grad {name}: rel {e:.2e}")
        assert e < 1e-3


@pytest.mark.parametrize("channels", [32, 37])
def test_features_non_finite_forward(channels):
    """A batch holding an infinite, a NaN and a huge (1e31) feature adds its
    channel sums on the vector ALU inside the matrix-core forward, only
    where a pixel composites the Gaussian: the non-finite values land
    exactly where the oracle's multiply-adds put them (no 0 * inf at pixels
    that skip the Gaussian), every other value within 1e-5, n_contrib,
    final_T and depth bit-exact."""
    W = H = 32
    n = 90
    rng = np.random.default_rng(7 + channels)
    m2 = rng.uniform(0.0, 32.0, (n, 2)).astype(np.float32)
    s = rng.uniform(0.5, 4.0, n)
    con = np.stack([1 / s ** 2, rng.uniform(-0.2, 0.2, n) / s ** 2, 1 / s ** 2], 1)
    con = con.astype(np.float32)
    op = rng.uniform(0.05, 0.9, n).astype(np.float32)
    feats = rng.standard_normal((n, channels)).astype(np.float32)
    feats[5, 3] = np.inf
    feats[17, 20] = -np.inf
    feats[40, 9] = np.nan
    feats[41, 30] = 1e31
    depths = rng.uniform(1.0, 5.0, n).astype(np.float32)
    ids = np.arange(n, dtype=np.int32)
    ranges = np.tile(np.array([[0, n]], np.int32), (4, 1))
    out = torch.empty((H, W, channels), device="cuda")
    fT = torch.empty((H, W), device="cuda")
    nct = torch.empty((H, W), dtype=torch.int32, device="cuda")
    dout = torch.empty((H, W), device="cuda")
    aout = torch.empty((H, W), device="cuda")
    dm2, dcon, dfe, ddp, dids, drg = (cu(a) for a in (m2, np.concatenate([con, op[:, None]], 1),
                                                      feats, depths, ids, ranges))
    L = _lib.load()
    P = _lib.ptr
    _lib.check(L.gsx_raster_fwd(n, channels, P(dm2), P(dcon), P(dfe), P(ddp), P(dids), n,
                                P(drg), None, W, H, P(out), P(fT), P(nct), P(dout), P(aout),
                                None, 0, _lib.stream_handle(out.device)), "raster_fwd")
    torch.cuda.synchronize()
    ref = O.raster_fwd(m2, con, op, feats, ids, ranges, W, H, depths=depths)
    np.testing.assert_array_equal(host(nct), ref["n_contrib"])
    assert_bits(host(fT), ref["final_T"], "final_T")
    assert_bits(host(dout), ref["depth"], "depth")
    img = host(out)
    assert not np.isfinite(ref["image"]).all()  # the non-finite values reach pixels
    assert_features(img, ref["image"], "features")


@pytest.mark.parametrize("channels", [1, 2, 4, 5, 12, 32, 37])
def test_features(channels):
    cam, means, quats, scales, opac, _ = random_scene(6, n=3000, width=128, height=96)
    opac = np.minimum(opac, 0.95).astype(np.float32)
    rng = np.random.default_rng(channels)
    feats = rng.standard_normal((3000, channels)).astype(np.float32)
    bg = np.linspace(-0.2, 0.2, channels).astype(np.float32)
    t = [cu(a).requires_grad_(True) for a in (means, quats, scales, opac, feats)]
    out = render_gaussian_features(cam, *t, background=cu(bg), return_depth=True)
    pre, f, ids, ranges, r = oracle_forward(cam, means, quats, scales, opac, colors=feats, bg=bg,
                                            depth=True)
    assert out["features"].shape == (96, 128, channels)
    np.testing.assert_array_equal(host(out["n_contrib"]), r["n_contrib"])
    assert_features(host(out["features"]), r["image"], "features")
    assert_bits(host(out["depth"]), r["depth"], "depth")
    g_img = rng.standard_normal(r["image"].shape).astype(np.float32)
    g_a = rng.standard_normal(r["final_T"].shape).astype(np.float32)
    ((out["features"] * cu(g_img)).sum() + (out["alpha"] * cu(g_a)).sum()).backward()
    g = oracle_backward(cam, means, quats, scales, opac, pre, f, ids, ranges, r, g_img, g_a, bg=bg)
    for name, a, key in [("means", t[0], "means"), ("opacities", t[3], "opacities"),
                         ("features", t[4], "features")]:
        e = rel_err(host(a.grad), g[key])
        say(f"features C={channels} grad {name}: rel {e:.2e}")
        assert e < 1e-3


def test_normalized_features_match_depth():
    # test_splatting.py:312-337
    cam, means, quats, scales, opac, _ = random_scene(7, n=3000, width=128, height=96)
    m, q, s, o = (cu(a) for a in (means, quats, scales, opac))
    depth = render_gaussian_depth(cam, m, q, s, o)
    feat = render_gaussian_features(cam, m, q, s, o, depth["depths"][:, None],
                                    background=cu(np.array([10.0], np.float32)), normalize=True)
    valid = host(depth["alpha"]) > 1e-3
    np.testing.assert_allclose(host(feat["alpha"]), host(depth["alpha"]), atol=1e-6)
    np.testing.assert_allclose(host(feat["features"][..., 0])[valid], host(depth["depth"])[valid],
                               rtol=1e-5)
    assert np.abs(host(feat["features"][..., 0])[~valid]).max(initial=0) < 1e-6


def test_render_on_side_streams():
    """Renders and their backward enqueued on two side streams back to back
    (each stream has its own binning workspace and status words) match the
    same renders run one after the other on the default stream: images and
    n_contrib bit for bit, gradients up to the float atomics' order."""
    scenes = [random_scene(seed, n=3000, width=200, height=150) for seed in (31, 32)]
    rng = np.random.default_rng(33)
    cot = [cu(rng.standard_normal((150, 200, 3)).astype(np.float32)) for _ in scenes]

    def run(i):
        cam, means, quats, scales, opac, colors = scenes[i]
        t = [cu(a).requires_grad_(True) for a in (means, quats, scales, opac, colors)]
        out = render_gaussians(cam, t[0], t[1], t[2], t[3], colors=t[4])
        (out["image"] * cot[i]).sum().backward()
        return out, t

    want = [run(i) for i in range(2)]
    torch.cuda.synchronize()
    side = [torch.cuda.Stream(), torch.cuda.Stream()]  # default priority
    got = []
    for i, s in enumerate(side):
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            got.append(run(i))
    torch.cuda.synchronize()
    for i in range(2):
        (wo, wt), (go, gt) = want[i], got[i]
        np.testing.assert_array_equal(host(go["n_contrib"]), host(wo["n_contrib"]))
        assert_bits(host(go["image"]), host(wo["image"]), f"image {i}")
        for name, a, b in zip(("means", "quats", "scales", "opacities", "colors"), gt, wt):
            e = rel_err(host(a.grad), host(b.grad))
            say(f"side stream {i} grad {name}: rel {e:.2e}")
            assert e < 1e-5


def test_empty_and_culled_render():
    cam, means, quats, scales, opac, colors = random_scene(8, n=10, width=64, height=48)
    means[:, 2] = -10.0  # all behind the camera
    out = render_gaussians(cam, cu(means), cu(quats), cu(scales), cu(opac), colors=cu(colors))
    assert host(out["sorted_ids"]).shape == (0,)
    assert (host(out["final_T"]) == 1.0).all() and (host(out["image"]) == 0).all()
    z = np.zeros((0, 3), np.float32)
    out = render_gaussians(cam, cu(z), cu(np.zeros((0, 4), np.float32)), cu(z),
                           cu(np.zeros(0, np.float32)), colors=cu(z))
    assert (host(out["alpha"]) == 0).all()


@pytest.mark.parametrize("offset", [0.0, 0.3])
def test_raster_active_clamp_closed_form(offset):
    """One splat with o G > 0.99 at the centre pixel (the 0.99 clamp is
    active there), loss = image[8, 8, 0]: the reference's backward passes the
    gradient through the clamp (rasterize.py:193), so dL/dopacity = G c0,
    dL/dc0 = 0.99 and dL/dmean_x = o c0 G (-a dx) in closed form."""
    W = H = 16
    sigma = 3.0
    m2 = np.array([[8.5 + offset, 8.5]], np.float32)
    con = np.array([[1.0 / sigma ** 2, 0.0, 1.0 / sigma ** 2]], np.float32)
    op = np.array([1.0], np.float32)
    col = np.array([[0.7, 0.2, 0.4]], np.float32)
    ids = np.zeros(1, np.int32)
    ranges = np.array([[0, 1]], np.int32)
    t = [cu(a).requires_grad_(True) for a in (m2, con, col, op)]
    out = rasterize(*t, cu(ids), cu(ranges), W, H, 1, 1)
    out["image"][8, 8, 0].backward()
    a = np.float64(con[0, 0])
    dx = np.float64(m2[0, 0]) - 8.5
    G = np.exp(-0.5 * a * dx * dx)
    c0 = np.float64(col[0, 0])
    assert op[0] * G > 0.99
    say(f"clamp closed form offset={offset}: g_opac {float(t[3].grad[0]):.7f} vs {G * c0:.7f}")
    np.testing.assert_allclose(host(out["image"])[8, 8, 0], 0.99 * c0, rtol=1e-6)
    np.testing.assert_allclose(host(t[3].grad)[0], G * c0, rtol=1e-5)
    np.testing.assert_allclose(host(t[2].grad)[0], [0.99, 0.0, 0.0], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(host(t[0].grad)[0, 0], op[0] * c0 * G * (-a * dx), rtol=1e-4,
                               atol=1e-7)
    np.testing.assert_allclose(host(t[1].grad)[0], [-0.5 * G * dx * dx * op[0] * c0, 0, 0],
                               rtol=1e-4, atol=1e-7)


@pytest.mark.parametrize("antialias", [False, True])
def test_render_active_clamp_gradients(antialias):
    """Opacities up to 1 (the clamp active at many pixels): the full render
    backward against the oracle, whose clamp branch the CPU suite pins by a
    closed form and a straight-through float64 autograd check."""
    cam, means, quats, scales, opac, colors = random_scene(9, n=4000, width=160, height=96)
    rng = np.random.default_rng(90)
    opac = rng.uniform(0.6, 1.0, opac.shape).astype(np.float32)
    opac[::2] = 1.0
    scales = (scales * 3.0).astype(np.float32)
    flags = O.ANTIALIAS if antialias else 0
    t = [cu(a).requires_grad_(True) for a in (means, quats, scales, opac, colors)]
    out = render_gaussians(cam, t[0], t[1], t[2], t[3], colors=t[4], antialias=antialias)
    pre, feats, ids, ranges, r = oracle_forward(cam, means, quats, scales, opac, colors=colors,
                                                flags=flags)
    np.testing.assert_array_equal(host(out["n_contrib"]), r["n_contrib"])
    assert_bits(host(out["image"]), r["image"], "image")
    g_img = rng.standard_normal(r["image"].shape).astype(np.float32)
    g_a = rng.standard_normal(r["final_T"].shape).astype(np.float32)
    ((out["image"] * cu(g_img)).sum() + (out["alpha"] * cu(g_a)).sum()).backward()
    g = oracle_backward(cam, means, quats, scales, opac, pre, feats, ids, ranges, r, g_img, g_a,
                        flags=flags)
    for name, a, key in [("means", t[0], "means"), ("quats", t[1], "quats"),
                         ("scales", t[2], "scales"), ("opacities", t[3], "opacities"),
                         ("colors", t[4], "features")]:
        e = rel_err(host(a.grad), g[key])
        say(f"render clamp aa={antialias} grad {name}: rel {e:.2e}")
        assert e < 1e-3


def test_render_direct_output_cotangents():
    """Cotangents on means2d, depths and compensation arrive as stride-0
    expands (from .sum()), which the backward copies before the preprocess
    VJP reads them; they must reach the kernel intact."""
    cam, means, quats, scales, opac, colors = random_scene(11, n=3000, width=128, height=96)
    opac = np.minimum(opac, 0.95).astype(np.float32)
    flags = O.ANTIALIAS
    t = [cu(a).requires_grad_(True) for a in (means, quats, scales, opac, colors)]
    out = render_gaussians(cam, t[0], t[1], t[2], t[3], colors=t[4], antialias=True)
    pre, feats, ids, ranges, r = oracle_forward(cam, means, quats, scales, opac, colors=colors,
                                                flags=flags)
    rng = np.random.default_rng(11)
    g_img = rng.standard_normal(r["image"].shape).astype(np.float32)
    loss = ((out["image"] * cu(g_img)).sum() + out["means2d"].sum() + 2.0 * out["depths"].sum()
            + 3.0 * out["compensation"].sum())
    loss.backward()
    oc = oracle_camera(cam)
    gr = O.raster_bwd(pre["means2d"], pre["conics"], pre["opac_eff"], feats, ids, ranges,
                      cam.width, cam.height, r["final_T"], r["n_contrib"], g_img)
    n = means.shape[0]
    g = O.preprocess_bwd(oc, means, quats, scales, opac, None, 0, 0, flags,
                         gr["means2d"] + np.ones((n, 2), np.float32), gr["conics"],
                         gr["opacities"], None, g_depths=np.full(n, 2.0, np.float32),
                         g_comp=np.full(n, 3.0, np.float32))
    for name, a, key in [("means", t[0], "means"), ("quats", t[1], "quats"),
                         ("scales", t[2], "scales"), ("opacities", t[3], "opacities")]:
        e = rel_err(host(a.grad), g[key])
        say(f"direct cotangents grad {name}: rel {e:.2e}")
        assert e < 1e-3


@pytest.mark.parametrize("C", [3, 5, 32])
def test_raster_backward_gradient_record(C):
    """gsx_raster_bwd into one gradient record per Gaussian (grad_stride > 0)
    against the four separate arrays: the same sums (float atomics add in
    run-dependent order, so to 1e-6 of the largest entry), padding zero."""
    from mlx3d_amd.splatting.rasterize import raster_backward, raster_forward

    say(f"gradient record C={C}")
    cam, means, quats, scales, opac, _ = random_scene(31 + C, n=4000, width=320, height=200)
    rng = np.random.default_rng(C)
    feats = cu(rng.random((means.shape[0], C), dtype=np.float32))
    proj = project_gaussians(cam, cu(means), cu(quats), cu(scales))
    ids, ranges, _, _ = bin_gaussians(proj["means2d"], proj["radii"], proj["depths"], 320, 200)
    co = torch.cat([proj["conics"], (cu(opac) * proj["compensation"])[:, None]], 1).contiguous()
    m2 = proj["means2d"].contiguous()
    bg = torch.zeros(C, device=m2.device)
    _, final_T, n_contrib, _, _ = raster_forward(m2, co, feats, ids, ranges, bg, 320, 200)
    g_out = cu(rng.normal(size=(200, 320, C)).astype(np.float32))
    g_T = cu(rng.normal(size=(200, 320)).astype(np.float32))
    sep = raster_backward(m2, co, feats, ids, ranges, bg, 320, 200, final_T, n_contrib, g_out,
                          g_T)
    rec = raster_backward(m2, co, feats, ids, ranges, bg, 320, 200, final_T, n_contrib, g_out,
                          g_T, record=True)
    for name, a, b in zip(("means2d", "conics", "features", "opacities"), sep, rec[:4]):
        e = float((a - b).abs().max() / a.abs().max().clamp_min(1e-30))
        say(f"  {name}: rel {e:.2e}")
        assert e < 1e-6, name
    stride = rec[5]
    assert stride % 4 == 0 and stride >= 6 + C
    assert float(rec[4][:, 6 + C:].abs().max() if stride > 6 + C else 0.0) == 0.0


@pytest.mark.parametrize("C", [3, 32])
def test_tile_order(C):
    """The rasterizers' tile order: the forward's outputs are bit-identical
    with and without the order buffer; the forward records each tile's
    largest n_contrib and orders each XCD's contiguous band of tiles
    (xcd_remap's equal-count bands) by non-increasing list length
    (quarter-octave buckets, raster order within a bucket); the backward
    cuts the tiles into 8 contiguous
    bands of equal work (at most 2 ceil(T / 8) tiles each), lists each band
    heaviest first at entries 8 i + band, -1 past a band's end, and gives
    the same gradients as in launch order, also when the bound words hold
    arbitrary values (float atomics: to 1e-6 of the largest entry)."""
    from mlx3d_amd.splatting.rasterize import (raster_backward, raster_forward,
                                               tile_order_buffer)

    W, H = 328, 200  # 21 x 13 tiles, the last column and row partial
    T = 21 * 13
    cam, means, quats, scales, opac, _ = random_scene(57 + C, n=5000, width=W, height=H)
    rng = np.random.default_rng(C)
    feats = cu(rng.standard_normal((means.shape[0], C)).astype(np.float32))
    proj = project_gaussians(cam, cu(means), cu(quats), cu(scales))
    ids, ranges, _, _ = bin_gaussians(proj["means2d"], proj["radii"], proj["depths"], W, H)
    co = torch.cat([proj["conics"], (cu(opac) * proj["compensation"])[:, None]], 1).contiguous()
    m2 = proj["means2d"].contiguous()
    bg = torch.linspace(-0.1, 0.1, C, device=m2.device)
    base = raster_forward(m2, co, feats, ids, ranges, bg, W, H)
    order = tile_order_buffer(W, H, m2.device)
    cap = 2 * ((T + 7) // 8)
    assert order.numel() == T + 8 * cap
    ordered = raster_forward(m2, co, feats, ids, ranges, bg, W, H, tile_order=order)
    for name, a, b in zip(("out", "final_T", "n_contrib", "alpha"),
                          (base[0], base[1], base[2], base[4]),
                          (ordered[0], ordered[1], ordered[2], ordered[4])):
        assert torch.equal(a, b), name

    def buckets(w):  # the kernel's key: the exponent and two bits below the leading one
        v = np.maximum(w.astype(np.int64), 0) + 1
        e = np.array([int(x).bit_length() - 1 for x in v])
        frac = np.where(e >= 2, v >> np.maximum(e - 2, 0), v << np.maximum(2 - e, 0)) & 3
        return np.minimum(4 * e + frac, 63)

    def sorted_band(seq, key):  # heaviest bucket first, raster order within a bucket
        return np.array_equal(seq, seq[np.lexsort((seq, -key[seq]))])

    o = host(order)
    nc = np.zeros((13 * 16, 21 * 16), np.int32)
    nc[:H, :W] = host(base[2])
    np.testing.assert_array_equal(o[:T], nc.reshape(13, 16, 21, 16).max(axis=(1, 3)).ravel())
    fwd = o[T:2 * T]
    rg = host(ranges)
    lens = buckets(rg[:, 1] - rg[:, 0])
    q, r = divmod(T, 8)
    lo = 0
    for x in range(8):  # each XCD's band holds its own tiles, longest lists first
        hi = lo + q + (1 if x < r else 0)
        assert np.array_equal(np.sort(fwd[lo:hi]), np.arange(lo, hi))
        assert sorted_band(fwd[lo:hi], lens)
        lo = hi
    g_out = cu(rng.normal(size=(H, W, C)).astype(np.float32))
    g_T = cu(rng.normal(size=(H, W)).astype(np.float32))
    ref = raster_backward(m2, co, feats, ids, ranges, bg, W, H, base[1], base[2], g_out, g_T)
    scrambled = order.clone()
    scrambled[:T] = cu(rng.integers(-2**31, 2**31 - 1, T, dtype=np.int64).astype(np.int32))
    for buf in (order, scrambled):
        got = raster_backward(m2, co, feats, ids, ranges, bg, W, H, base[1], base[2], g_out,
                              g_T, tile_order=buf)
        o = host(buf)
        work, slots = o[:T], o[T:].reshape(cap, 8)  # slots[i, x]: band x's i-th tile
        placed = slots[slots >= 0]
        assert np.array_equal(np.sort(placed), np.arange(T))
        start = 0
        for x in range(8):
            col = slots[:, x]
            size = int((col >= 0).sum())
            assert (col[:size] >= 0).all() and (col[size:] < 0).all()
            assert np.array_equal(np.sort(col[:size]), np.arange(start, start + size))
            assert sorted_band(col[:size], buckets(work))
            start += size
        for name, a, b in zip(("means2d", "conics", "features", "opacities"), ref, got):
            e = float((a - b).abs().max() / a.abs().max().clamp_min(1e-30))
            assert e < 1e-6, name


@pytest.mark.parametrize("case", ["fast", "refine", "culled", "empty"])
def test_binning_writes_the_forward_order(case):
    """gsx_bin_tiles_async with a tile-order buffer writes the forward
    rasterizer's order for the ranges it produces (the placement launch's
    first workgroups, or a launch of its own on the refine_tiles path and
    without duplicates): the same words gsx_raster_fwd computes itself, and
    a forward run with order_ready gives bit-identical outputs."""
    from mlx3d_amd.splatting.rasterize import raster_forward, tile_order_buffer
    from mlx3d_amd.splatting.tiles import BinJob

    say(f"binning-written tile order: {case}")
    W, H = 328, 200
    T = 21 * 13
    n = 0 if case == "empty" else 6000
    cam, means, quats, scales, opac, _ = random_scene(91, n=max(n, 1), width=W, height=H)
    means, quats, scales, opac = means[:n], quats[:n], scales[:n], opac[:n]
    if case == "culled":
        means = means + np.float32(50.0)  # every Gaussian off screen: no duplicates
    proj = project_gaussians(cam, cu(means), cu(quats), cu(scales))
    m2 = proj["means2d"].contiguous()
    co = torch.cat([proj["conics"], (cu(opac) * proj["compensation"])[:, None]], 1).contiguous()
    L = _lib.load()
    dev = m2.device
    counts = torch.empty((n,), dtype=torch.int32, device=dev)
    dkeys = torch.empty((n,), dtype=torch.int32, device=dev)
    rects = torch.empty((n, 2), dtype=torch.int32, device=dev)
    _lib.check(L.gsx_bin_prepare(n, _lib.ptr(m2), _lib.ptr(proj["radii"].contiguous()),
                                 _lib.ptr(proj["depths"].contiguous()), W, H, _lib.ptr(counts),
                                 _lib.ptr(dkeys), _lib.ptr(rects), _lib.stream_handle(dev)),
               "gsx_bin_prepare")
    order = tile_order_buffer(W, H, dev)
    order.fill_(-7)
    job = BinJob(counts, dkeys, rects, W, H, final=True, tile_order=order,
                 refine=(m2, co[:, :3].contiguous()) if case == "refine" else None)
    ids, ranges = job.result()
    ids_full = job.ids
    feats = cu(np.random.default_rng(5).random((n, 3), dtype=np.float32))
    own = tile_order_buffer(W, H, dev)
    base = raster_forward(m2, co, feats, ids_full, ranges, None, W, H, tile_order=own)
    ready = raster_forward(m2, co, feats, ids_full, ranges, None, W, H, tile_order=order,
                           order_ready=True)
    torch.cuda.synchronize()
    assert np.array_equal(host(order)[T:2 * T], host(own)[T:2 * T])
    assert np.array_equal(np.sort(host(order)[T:2 * T]), np.arange(T))
    for name, k in (("out", 0), ("final_T", 1), ("n_contrib", 2), ("alpha", 4)):
        assert torch.equal(base[k], ready[k]), name
    if case != "empty":
        assert (int(ids.numel()) == 0) == (case == "culled")
