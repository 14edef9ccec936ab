"""GPU parity of the training step: photometric loss kernels, multi-group
Adam, screen-gradient statistics, density control and GaussianTrainer.step,
each against the CPU oracle (oracle/train_oracle.c, oracle/density.py,
oracle/gsx_oracle.c).

Tolerances: Adam and the screen-gradient statistics are float32 in the
reference's operation order and must match bit for bit; the loss values
(float32 on the GPU vs float64 in the oracle) within 2e-6 absolute; loss
and parameter gradients within max|d| / max|ref| < 1e-4 (loss) and 1e-3
(parameters, the rasterizer's bar).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gpu_util import assert_bits, cu, host, oracle_backward, oracle_forward, rel_err, say
from mlx3d_amd import _lib
from mlx3d_amd.losses import l1_loss, photometric, photometric_loss, ssim
from mlx3d_amd.optim import Adam, adam_step, exponential_decay
from mlx3d_amd.splatting import GaussianModel
from mlx3d_amd.splatting.trainer import GaussianTrainer, TrainerConfig
from oracle import density as DN
from oracle import oracle as O
from refimpl import random_scene

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H,W,C,ws,sigma", [(64, 80, 3, 11, 1.5), (37, 53, 3, 11, 1.5),
                                            (5, 7, 3, 11, 1.5), (48, 40, 1, 3, 0.7),
                                            (33, 29, 2, 15, 2.5), (20, 24, 3, 1, 1.0),
                                            (24, 20, 5, 11, 1.5), (17, 35, 8, 7, 1.0)])
def test_photometric_matches_oracle(H, W, C, ws, sigma):
    say(f"photometric H={H} W={W} C={C} ws={ws}")
    rng = np.random.default_rng(H + W + ws)
    p = rng.random((H, W, C), dtype=np.float32)
    t = rng.random((H, W, C), dtype=np.float32)
    pt = cu(p).requires_grad_(True)
    l1, s = photometric(pt, cu(t), ws, sigma)
    (0.8 * l1 - 0.2 * s).backward()
    rl1, rs, rg = O.photometric(p, t, ws, sigma, g_l1=0.8, g_ssim=-0.2, grad=True)
    say(f"  l1 {float(l1):.8f} vs {rl1:.8f}; ssim {float(s):.8f} vs {rs:.8f}")
    assert abs(float(l1) - rl1) < 2e-6 and abs(float(s) - rs) < 2e-6
    e = rel_err(host(pt.grad), rg)
    say(f"  grad rel {e:.2e}")
    assert e < 1e-4


@pytest.mark.parametrize("H,W,C,lam,ws", [(64, 80, 3, 0.2, 11), (37, 53, 3, 0.0, 11),
                                          (24, 20, 5, 1.0, 7), (1080, 1920, 3, 0.2, 11),
                                          (48, 40, 1, 0.35, 3)])
def test_photometric_loss_matches_expression(H, W, C, lam, ws):
    """photometric_loss (gsx_photometric_loss_fwd/_bwd) against the
    expression (1 - lam) l1 + lam (1 - ssim) over photometric()'s outputs
    with torch autograd: loss value and gradient bit for bit."""
    say(f"photometric_loss H={H} W={W} C={C} lam={lam}")
    rng = np.random.default_rng(H * W + C)
    p = rng.random((H, W, C), dtype=np.float32)
    t = rng.random((H, W, C), dtype=np.float32)
    a = cu(p).requires_grad_(True)
    b = cu(p).requires_grad_(True)
    fused = photometric_loss(a, cu(t), lam, window_size=ws)
    l1, s = photometric(b, cu(t), window_size=ws)
    expr = (1.0 - lam) * l1 + lam * (1.0 - s)
    assert_bits(host(fused).reshape(1), host(expr).reshape(1), "loss")
    (2.5 * fused).backward()
    (2.5 * expr).backward()
    assert_bits(host(a.grad), host(b.grad), "grad")
    with pytest.raises(ValueError):
        photometric_loss(a, cu(t), 1.5)


def test_l1_writes_one_float():
    """gsx_l1_fwd and gsx_l1_fwd_noalloc write exactly their one output
    float (the neighbours of `out` inside a larger buffer stay untouched)."""
    rng = np.random.default_rng(3)
    n = 100003
    p, t = cu(rng.random(n, dtype=np.float32)), cu(rng.random(n, dtype=np.float32))
    L, st = _lib.load(), _lib.stream_handle(p.device)
    want = float(np.abs(host(p).astype(np.float64) - host(t)).mean())
    ws = torch.empty((int(L.gsx_l1_workspace_bytes(n)),), dtype=torch.uint8, device=p.device)
    for call in ("gsx_l1_fwd", "gsx_l1_fwd_noalloc"):
        buf = torch.full((8,), -7.0, device=p.device)
        out = buf[3:4]
        if call == "gsx_l1_fwd":
            rc = L.gsx_l1_fwd(n, _lib.ptr(p), _lib.ptr(t), _lib.ptr(ws), ws.numel(),
                              _lib.ptr(out), st)
        else:
            rc = L.gsx_l1_fwd_noalloc(n, _lib.ptr(p), _lib.ptr(t), _lib.ptr(out), st)
        _lib.check(rc, call)
        got = host(buf)
        assert abs(float(got[3]) - want) < 1e-6, call
        assert (np.delete(got, 3) == -7.0).all(), (call, got)


def test_photometric_full_size_properties():
    """1920x1080x3: SSIM(x, x) = 1 with zero SSIM gradient; L1 against torch."""
    say("photometric 1080p properties")
    rng = np.random.default_rng(9)
    p = cu(rng.random((1080, 1920, 3), dtype=np.float32)).requires_grad_(True)
    t = cu(rng.random((1080, 1920, 3), dtype=np.float32))
    l1, s = photometric(p, p.detach().clone())
    assert float(l1) == 0.0 and abs(float(s) - 1.0) < 1e-6
    s.backward()
    assert float(p.grad.abs().max()) < 1e-9
    p.grad = None
    l1, s = photometric(p, t)
    ref = (p.detach().double() - t.double()).abs().mean()
    assert abs(float(l1) - float(ref)) < 1e-6
    l1.backward()
    np.testing.assert_array_equal(host(p.grad), host(torch.sign(p.detach() - t) / p.numel()))


def test_ssim_batched_and_errors():
    rng = np.random.default_rng(2)
    a = rng.random((2, 24, 30, 3), dtype=np.float32)
    b = rng.random((2, 24, 30, 3), dtype=np.float32)
    s = float(ssim(cu(a), cu(b)))
    ref = 0.5 * (O.photometric(a[0], b[0])[1] + O.photometric(a[1], b[1])[1])
    assert abs(s - ref) < 2e-6
    with pytest.raises(ValueError):
        ssim(cu(a[0]), cu(b[0]), window_size=10)
    with pytest.raises(ValueError):
        photometric(cu(a[0]), cu(b[1, :20]))


@pytest.mark.parametrize("n,offset", [(1, 0), (7, 0), (4101, 0), (4101, 1),
                                      (1080 * 1920 * 3, 0), (65537, 3)])
def test_l1_loss_matches_closed_form(n, offset):
    """mean |p - t| against float64, and the gradient bit for bit against
    sign(p - t) * (g / n) in float32; offset views take the unvectorised
    path."""
    say(f"l1 n={n} offset={offset}")
    rng = np.random.default_rng(n + offset)
    p = rng.random(n + offset, dtype=np.float32)
    t = rng.random(n + offset, dtype=np.float32)
    t[offset::5] = p[offset::5]  # equal entries: sign 0
    base = cu(p).requires_grad_(True)
    loss = l1_loss(base[offset:], cu(t)[offset:])  # offset > 0: unaligned contiguous view
    ref = np.abs(p[offset:].astype(np.float64) - t[offset:].astype(np.float64)).mean()
    assert abs(float(loss) - ref) <= 2e-7 * max(ref, 1e-30) + 1e-12
    (2.5 * loss).backward()
    g = base.grad[offset:]
    sc = np.float32(2.5) / np.float32(n)
    want = (np.sign(p[offset:] - t[offset:]).astype(np.float32) * sc).astype(np.float32)
    assert_bits(host(g), want, "l1 grad")


@pytest.mark.parametrize("n,soff", [(4101, 0), (65537, 1), (1080 * 1920 * 3, 0)])
def test_l1_sign_pair_matches_plain_pair(n, soff):
    """gsx_l1_fwd_signs / gsx_l1_bwd_signs against gsx_l1_fwd / gsx_l1_bwd
    through the C ABI: loss and gradient bit for bit, with NaN, +-inf and
    equal entries; the codes against numpy's comparisons.  soff = 1 puts the
    sign bytes at an odd address (the byte-wise path)."""
    say(f"l1 signs n={n} soff={soff}")
    rng = np.random.default_rng(n)
    p = rng.standard_normal(n).astype(np.float32)
    t = rng.standard_normal(n).astype(np.float32)
    t[::7] = p[::7]
    p[3::101] = np.nan
    t[5::211] = np.inf
    pc, tc = cu(p), cu(t)
    L, st = _lib.load(), _lib.stream_handle(pc.device)
    ws = torch.empty((int(L.gsx_l1_workspace_bytes(n)),), dtype=torch.uint8, device=pc.device)
    sbuf = torch.full((n + 8,), 0xAB, dtype=torch.uint8, device=pc.device)
    signs = sbuf[soff:soff + n]
    g = cu(np.array([1.75], np.float32))
    outs, grads = [], []
    for pair in ("plain", "signs"):
        out = torch.empty((1,), dtype=torch.float32, device=pc.device)
        grad = torch.empty_like(pc)
        if pair == "plain":
            _lib.check(L.gsx_l1_fwd(n, _lib.ptr(pc), _lib.ptr(tc), _lib.ptr(ws), ws.numel(),
                                    _lib.ptr(out), st), "gsx_l1_fwd")
            _lib.check(L.gsx_l1_bwd(n, _lib.ptr(pc), _lib.ptr(tc), _lib.ptr(g), _lib.ptr(grad),
                                    st), "gsx_l1_bwd")
        else:
            _lib.check(L.gsx_l1_fwd_signs(n, _lib.ptr(pc), _lib.ptr(tc), _lib.ptr(ws),
                                          ws.numel(), _lib.ptr(signs), _lib.ptr(out), st),
                       "gsx_l1_fwd_signs")
            _lib.check(L.gsx_l1_bwd_signs(n, _lib.ptr(signs), _lib.ptr(pc), _lib.ptr(tc),
                                          _lib.ptr(g), _lib.ptr(grad), st), "gsx_l1_bwd_signs")
        outs.append(host(out))
        grads.append(host(grad))
    assert_bits(outs[1], outs[0], "l1 loss")
    assert_bits(grads[1], grads[0], "l1 grad")
    d = p - t
    want = np.where(d > 0, 0, np.where(d < 0, 1, np.where(d == 0, 2, 3))).astype(np.uint8)
    got = host(sbuf)
    assert (got[soff:soff + n] == want).all()
    assert (np.delete(got, np.arange(soff, soff + n)) == 0xAB).all()  # nothing outside


def test_l1_loss_errors():
    with pytest.raises(ValueError):
        l1_loss(torch.zeros(3), torch.zeros(3))  # host tensors
    with pytest.raises(ValueError):
        l1_loss(cu(np.zeros(3, np.float32)), cu(np.zeros(4, np.float32)))


def test_adam_bitexact_multi_group():
    say("adam groups")
    rng = np.random.default_rng(4)
    sizes = [5, 1024, 4099, 3, 0, 100_003, 7, 64, 12, 999]  # > 8 groups: two launches
    ps = [rng.normal(size=n).astype(np.float32) for n in sizes]
    opts, params, ref = [], [], []
    for i, n in enumerate(sizes):
        base = cu(np.concatenate([[0.0], ps[i]]).astype(np.float32))
        # odd groups start one float into their buffer: the scalar path
        p = base[1:] if i % 2 else cu(ps[i])
        params.append(p)
        lr = exponential_decay(1e-2 * (i + 1), 0.97) if i == 0 else 1e-3 * (i + 1)
        opts.append(Adam(learning_rate=lr, eps=1e-15))
        ref.append([ps[i].copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)])
    for step in range(3):
        grads = [rng.normal(size=n).astype(np.float32) for n in sizes]
        adam_step([(opts[i], {"w": cu(grads[i])}, {"w": params[i]}) for i in range(len(sizes))])
        for i in range(len(sizes)):
            lr = 1e-2 * 0.97 ** step if i == 0 else 1e-3 * (i + 1)
            ref[i] = list(O.adam(ref[i][0], grads[i], ref[i][1], ref[i][2], lr, eps=1e-15))
    for i in range(len(sizes)):
        assert_bits(host(params[i]), ref[i][0], f"adam param {i}")
        assert_bits(host(opts[i].state["w"]["m"]), ref[i][1], f"adam m {i}")
        assert_bits(host(opts[i].state["w"]["v"]), ref[i][2], f"adam v {i}")
    assert abs(opts[0].learning_rate - 1e-2 * 0.97 ** 2) < 1e-12


def test_accum_screen_grads_bitexact():
    rng = np.random.default_rng(8)
    n = 100_001
    g = (rng.normal(size=(n, 2)) * 1e-4).astype(np.float32)
    radii = np.where(rng.random(n) < 0.3, 0.0, rng.integers(1, 50, n)).astype(np.float32)
    acc0 = rng.random(n).astype(np.float32)
    cnt0 = rng.integers(0, 5, n).astype(np.float32)
    acc, cnt = cu(acc0), cu(cnt0)
    gd, rd = cu(g), cu(radii)  # alive until the kernel has run
    _lib.check(_lib.load().gsx_accum_screen_grads(
        n, _lib.ptr(gd), _lib.ptr(rd), 1279, 720, _lib.ptr(acc), _lib.ptr(cnt), 0,
        _lib.stream_handle(acc.device)), "accum")
    ra, rc = O.accum_screen_grads(g, radii, 1279, 720, acc0, cnt0)
    assert_bits(host(acc), ra, "grad_accum")
    assert_bits(host(cnt), rc, "grad_count")


def _model(seed, n, degree=3):
    cam, means, quats, scales, opac, _ = random_scene(seed, n=n, width=160, height=112)
    rng = np.random.default_rng(100 + seed)
    sh = (rng.standard_normal((n, 16, 3)) * 0.2).astype(np.float32)
    ls = np.log(scales).astype(np.float32)
    lo = np.clip(rng.standard_normal(n), -4, 3).astype(np.float32)
    raw = dict(means=means, quats=quats, scales=ls, opacities=lo, sh_dc=sh[:, :1].copy(),
               sh_rest=sh[:, 1:].copy())
    model = GaussianModel({k: cu(v) for k, v in raw.items()}, sh_degree=3)
    model.active_sh_degree = degree
    return cam, model, raw, sh


@pytest.mark.parametrize("degree", [0, 3])
def test_trainer_step_matches_oracle(degree):
    say(f"trainer step degree {degree}")
    cam, model, raw, sh = _model(21 + degree, 4000, degree)
    rng = np.random.default_rng(7)
    target = rng.random((cam.height, cam.width, 3), dtype=np.float32)
    cfg = TrainerConfig(densify_from=1, densify_until=100, densify_every=50)
    tr = GaussianTrainer(model, cfg)
    p0 = {k: v.copy() for k, v in raw.items()}
    info = tr.step(cam, cu(target))

    flags = O.LOG_SCALES | O.LOGIT_OPACITY
    pre, feats, ids, ranges, r = oracle_forward(cam, raw["means"], raw["quats"], raw["scales"],
                                                raw["opacities"], sh=sh, degree=degree,
                                                flags=flags)
    lam = cfg.lambda_dssim
    l1, s, g_img = O.photometric(r["image"], target, g_l1=1 - lam, g_ssim=-lam, grad=True)
    loss = (1 - lam) * l1 + lam * (1 - s)
    say(f"  loss {info['loss']:.8f} vs oracle {loss:.8f}")
    assert abs(info["loss"] - loss) < 2e-6
    g = oracle_backward(cam, raw["means"], raw["quats"], raw["scales"], raw["opacities"], pre,
                        feats, ids, ranges, r, g_img.astype(np.float32), None, sh=sh,
                        degree=degree, flags=flags)
    g["sh_dc"], g["sh_rest"] = g["sh"][:, :1], g["sh"][:, 1:]
    for k in ("means", "quats", "scales", "opacities", "sh_dc", "sh_rest"):
        st = tr.optimizers[k].state[k]
        m1, v1 = host(st["m"]), host(st["v"])
        # first step from zero moments: m = 0.1 g
        e = rel_err(m1 / np.float32(0.1), g[k])
        say(f"  grad {k}: rel {e:.2e}")
        assert e < 1e-3
        # the update the kernel applied, recomputed in float32 from its moments
        lr = np.float32(tr.optimizers[k].learning_rate)
        expect = p0[k] - (lr * m1) / (np.sqrt(v1) + np.float32(1e-15))
        assert_bits(host(model.params[k]), expect.astype(np.float32), f"update {k}")
    # screen-space statistics of the rasterizer's dL/dmeans2d
    ra, rc = O.accum_screen_grads(g["raster"]["means2d"], pre["radii"], cam.width, cam.height,
                                  np.zeros(4000), np.zeros(4000))
    np.testing.assert_array_equal(host(tr.grad_count), rc)
    e = rel_err(host(tr.grad_accum), ra)
    say(f"  grad_accum rel {e:.2e}")
    assert e < 1e-3


def _bwd_inputs(seed, n, K, with_extra):
    """Parameters, forward colours and output cotangents for the preprocess
    backward, plus nonzero Adam moments, as device tensors."""
    cam, _, raw, sh = _model(seed, n)
    rng = np.random.default_rng(seed + 1)
    f = lambda *s, sc=1.0: cu((rng.standard_normal(s) * sc).astype(np.float32))  # noqa: E731
    params = {k: cu(raw[k]) for k in ("means", "quats", "scales", "opacities")}
    params["sh_dc"] = cu(sh[:, 0].copy())
    params["sh_rest"] = cu(sh[:, 1:K].reshape(n, 3 * (K - 1)).copy())
    cot = dict(colors=cu(rng.uniform(-0.2, 1.0, (n, 3)).astype(np.float32)),
               g_m2=f(n, 2, sc=1e-2), g_con=f(n, 3, sc=1e-3), g_op=f(n, sc=1e-2),
               g_col=f(n, 3, sc=1e-2), extra=f(n, 2, sc=1e-2) if with_extra else None,
               g_dep=f(n, sc=1e-2) if with_extra else None,
               g_comp=f(n, sc=1e-2) if with_extra else None)
    moments = {k: (f(*v.shape, sc=1e-3),
                   cu(rng.uniform(1e-8, 1e-6, v.shape).astype(np.float32)))
               for k, v in params.items()}
    return cam, params, cot, moments


_ORDER = ("means", "quats", "scales", "opacities", "sh_dc", "sh_rest")
_LRS = dict(means=1.6e-4, quats=1e-3, scales=5e-3, opacities=5e-2, sh_dc=2.5e-3,
            sh_rest=1.25e-4)


def _offset_copy(t):
    """A copy of t that starts 4 bytes past a 16-byte boundary."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    buf[1:].copy_(t.reshape(-1))
    return buf[1:].view(t.shape)


@pytest.mark.parametrize("n,K,degree,flags,extra,misalign", [
    (3001, 16, 3, 0, True, False), (3001, 16, 1, _lib.ANTIALIAS, False, False),
    (2500, 9, 2, _lib.PROJECT_UT, True, False),
    (777, 1, 0, _lib.PROJECT_UT | _lib.ANTIALIAS, True, False), (1, 4, 1, 0, False, False),
    (3001, 16, 3, 0, True, True), (1500, 9, 2, 0, False, True)])
def test_preprocess_bwd_adam_matches_bwd_then_adam(n, K, degree, flags, extra, misalign):
    """gsx_preprocess_bwd_adam against gsx_preprocess_bwd + gsx_adam_step on
    the same cotangents: parameters and both moments bit for bit (ragged last
    block, degrees below the stored K, UT, antialiasing, optional inputs, SH
    rest rows of odd and even width, and SH rest tensors off 16-byte
    alignment, which take the element-wise path)."""
    say(f"preprocess_bwd_adam n={n} K={K} degree={degree} flags={flags} extra={extra} "
        f"misalign={misalign}")
    cam, params, cot, moments = _bwd_inputs(50 + K, n, K, extra)
    flags |= _lib.LOG_SCALES | _lib.LOGIT_OPACITY
    L, ptr, st = _lib.load(), _lib.ptr, _lib.stream_handle(params["means"].device)
    gcam = cam.to_gsx()
    groups = [k for k in _ORDER if k != "sh_rest" or K > 1]
    # separate: gradients written out, then one multi-group Adam launch
    sep = {k: (params[k].clone(), moments[k][0].clone(), moments[k][1].clone()) for k in groups}
    g = {k: torch.empty_like(params[k]) for k in _ORDER}
    _lib.check(L.gsx_preprocess_bwd(
        gcam, n, ptr(sep["means"][0]), ptr(sep["quats"][0]), ptr(sep["scales"][0]),
        ptr(sep["opacities"][0]), ptr(cot["colors"]), K, degree, flags, 0.3, ptr(cot["g_m2"]),
        ptr(cot["g_con"]), ptr(cot["g_op"]), ptr(cot["g_col"]), ptr(cot["extra"]),
        ptr(cot["g_dep"]), ptr(cot["g_comp"]), ptr(g["means"]), ptr(g["quats"]),
        ptr(g["scales"]), ptr(g["opacities"]), ptr(g["sh_dc"]), 3,
        ptr(g["sh_rest"]) if K > 1 else None, 3 * (K - 1), 0, st), "gsx_preprocess_bwd")
    # the same VJP from the rasterizer's gradient record (12 floats per
    # Gaussian: means2d, conic, opacity, colour): bit-identical gradients
    rec = torch.zeros((n, 12), dtype=torch.float32, device=cot["g_m2"].device)
    rec[:, 0:2] = cot["g_m2"]
    rec[:, 2:5] = cot["g_con"]
    rec[:, 5] = cot["g_op"]
    rec[:, 6:9] = cot["g_col"]
    g2 = {k: torch.empty_like(params[k]) for k in _ORDER}
    _lib.check(L.gsx_preprocess_bwd(
        gcam, n, ptr(sep["means"][0]), ptr(sep["quats"][0]), ptr(sep["scales"][0]),
        ptr(sep["opacities"][0]), ptr(cot["colors"]), K, degree, flags, 0.3, ptr(rec), None,
        None, None, ptr(cot["extra"]), ptr(cot["g_dep"]), ptr(cot["g_comp"]), ptr(g2["means"]),
        ptr(g2["quats"]), ptr(g2["scales"]), ptr(g2["opacities"]), ptr(g2["sh_dc"]), 3,
        ptr(g2["sh_rest"]) if K > 1 else None, 3 * (K - 1), 12, st), "gsx_preprocess_bwd rec")
    for k in groups:
        assert_bits(host(g2[k]), host(g[k]), f"record-layout gradient {k}")
    arr = (_lib.GsxAdamGroup * len(groups))()
    for j, k in enumerate(groups):
        p, m, v = sep[k]
        arr[j] = _lib.GsxAdamGroup(p.data_ptr(), g[k].data_ptr(), m.data_ptr(), v.data_ptr(),
                                   p.numel(), _LRS[k])
    _lib.check(L.gsx_adam_step(len(groups), ctypes.cast(arr, ctypes.c_void_p), 0.9, 0.999,
                               1e-15, st), "gsx_adam_step")
    # fused
    fus = {k: (params[k].clone(), moments[k][0].clone(), moments[k][1].clone()) for k in groups}
    if misalign:
        fus["sh_rest"] = tuple(_offset_copy(t) for t in fus["sh_rest"])
    arr = (_lib.GsxAdamGroup * 6)()
    for j, k in enumerate(groups):
        p, m, v = fus[k]
        arr[j] = _lib.GsxAdamGroup(p.data_ptr(), None, m.data_ptr(), v.data_ptr(), p.numel(),
                                   _LRS[k])
    _lib.check(L.gsx_preprocess_bwd_adam(
        gcam, n, ptr(fus["means"][0]), ptr(fus["quats"][0]), ptr(fus["scales"][0]),
        ptr(fus["opacities"][0]), ptr(fus["sh_dc"][0]),
        ptr(fus["sh_rest"][0]) if K > 1 else None, ptr(cot["colors"]), K, degree, flags, 0.3,
        ptr(cot["g_m2"]), ptr(cot["g_con"]), ptr(cot["g_op"]), ptr(cot["g_col"]),
        ptr(cot["extra"]), ptr(cot["g_dep"]), ptr(cot["g_comp"]),
        ctypes.cast(arr, ctypes.c_void_p), 0.9, 0.999, 1e-15, 0, st), "gsx_preprocess_bwd_adam")
    for k in groups:
        for slot, a, b in zip(("param", "m", "v"), fus[k], sep[k]):
            assert_bits(host(a), host(b), f"{slot} {k}")
        assert not torch.equal(fus[k][0], params[k]), k  # the update ran


def test_preprocess_bwd_adam_rejects_mismatched_groups():
    cam, params, cot, moments = _bwd_inputs(60, 64, 4, False)
    L, ptr, st = _lib.load(), _lib.ptr, _lib.stream_handle(params["means"].device)
    arr = (_lib.GsxAdamGroup * 6)()
    for j, k in enumerate(_ORDER):
        arr[j] = _lib.GsxAdamGroup(params[k].data_ptr(), None, moments[k][0].data_ptr(),
                                   moments[k][1].data_ptr(), params[k].numel(), 1e-3)
    arr[2] = _lib.GsxAdamGroup(params["quats"].data_ptr(), None, moments["scales"][0].data_ptr(),
                               moments["scales"][1].data_ptr(), params["scales"].numel(), 1e-3)

    def call():
        return L.gsx_preprocess_bwd_adam(
            cam.to_gsx(), 64, ptr(params["means"]), ptr(params["quats"]),
            ptr(params["scales"]), ptr(params["opacities"]), ptr(params["sh_dc"]),
            ptr(params["sh_rest"]), ptr(cot["colors"]), 4, 1, _lib.LOG_SCALES, 0.3,
            ptr(cot["g_m2"]), ptr(cot["g_con"]), ptr(cot["g_op"]), ptr(cot["g_col"]), None,
            None, None, ctypes.cast(arr, ctypes.c_void_p), 0.9, 0.999, 1e-15, 0, st)
    before = host(params["means"])
    assert call() != _lib.GSX_OK  # group 2 names the quaternions, not the scales
    torch.cuda.synchronize()
    assert_bits(host(params["means"]), before, "untouched means")


def test_trainer_fused_adam_sh_degree_zero_model():
    """A model stored with SH degree 0 (K = 1: an empty sh_rest group): the
    fused update leaves the empty group alone and matches the separate one."""
    say("fused adam, SH degree 0 model")
    cam, means, quats, scales, opac, _ = random_scene(61, n=2000, width=160, height=112)
    rng = np.random.default_rng(62)
    raw = dict(means=means, quats=quats, scales=np.log(scales).astype(np.float32),
               opacities=np.clip(rng.standard_normal(2000), -4, 3).astype(np.float32),
               sh_dc=(rng.standard_normal((2000, 1, 3)) * 0.2).astype(np.float32),
               sh_rest=np.zeros((2000, 0, 3), np.float32))
    models = [GaussianModel({k: cu(v) for k, v in raw.items()}, sh_degree=0) for _ in range(2)]
    cfg = TrainerConfig(densify_from=1 << 30, densify_until=1 << 30, opacity_reset_every=1 << 30,
                        sh_increase_every=1 << 30)
    trs = [GaussianTrainer(m, cfg, fuse_adam=f) for m, f in zip(models, (True, False))]
    target = cu(rng.random((cam.height, cam.width, 3), dtype=np.float32))
    for _ in range(3):
        infos = [tr.step(cam, target) for tr in trs]
        assert abs(infos[0]["loss"] - infos[1]["loss"]) <= 1e-6 * abs(infos[1]["loss"])
    for k in ("means", "quats", "scales", "opacities", "sh_dc"):
        a, b = host(models[0].params[k]), host(models[1].params[k])
        lr = float(trs[0].optimizers[k].learning_rate)
        assert (np.abs(a.astype(np.float64) - b) <= 24 * lr + 1e-6 * np.abs(b)).all(), k
    assert models[0].params["sh_rest"].shape == (2000, 0, 3)


@pytest.mark.parametrize("method,projection,degree", [("vanilla", "ewa", 3), ("vanilla", "ut", 1),
                                                       ("mcmc", "ewa", 0)])
def test_trainer_fused_adam_close_to_separate_update(method, projection, degree):
    """GaussianTrainer with the update inside the backward against the
    separate Adam launch over several steps.  The rasterizer backward adds
    per-Gaussian cotangents with float atomics, so the two runs see gradients
    that differ in the last bits; with eps 1e-15 a near-zero gradient whose
    sign differs moves a parameter by about 3 lr the other way.  Bar: the
    learning rates agree exactly, every parameter within 32 lr of its group
    (four steps, plus 1e-6 relative), 99% of them within 1e-5 relative."""
    say(f"fused adam trainer {method} {projection} degree {degree}")
    models = [_model(41, 3000, degree)[1] for _ in range(2)]
    cam = _model(41, 10, degree)[0]
    cfg = TrainerConfig(method=method, projection=projection, densify_from=1 << 30,
                        densify_until=1 << 30, opacity_reset_every=1 << 30,
                        sh_increase_every=1 << 30, mcmc_noise_scale=0.0)
    trs = [GaussianTrainer(m, cfg, fuse_adam=f) for m, f in zip(models, (True, False))]
    rng = np.random.default_rng(5)
    for step in range(4):
        target = cu(rng.random((cam.height, cam.width, 3), dtype=np.float32))
        infos = [tr.step(cam, target) for tr in trs]
        assert abs(infos[0]["loss"] - infos[1]["loss"]) <= 1e-6 * abs(infos[1]["loss"]), step
    for k in ("means", "quats", "scales", "opacities", "sh_dc", "sh_rest"):
        assert trs[0].optimizers[k].learning_rate == trs[1].optimizers[k].learning_rate
        lr = max(float(trs[0].optimizers[k].learning_rate), 1e-12)
        a, b = host(models[0].params[k]), host(models[1].params[k])
        d = np.abs(a.astype(np.float64) - b)
        say(f"  {k}: max |d| {d.max():.3e} (lr {lr:.2e}), "
            f"{int((d > 1e-5 * np.abs(b) + 1e-12).sum())} of {d.size} beyond 1e-5 rel")
        assert (d <= 8 * 4 * lr + 1e-6 * np.abs(b)).all(), k
        assert (d > 1e-5 * np.abs(b) + 1e-12).mean() < 0.01, k


def test_densify_and_prune_matches_oracle():
    say("densify_and_prune")
    _, model, raw, _ = _model(31, 3000)
    # scales are about 0.08: extent 8 puts percent_dense * extent mid-range
    # (clones and splits); 50 rows below the opacity floor
    raw["opacities"][:50] = -7.0
    model.params["opacities"][:50] = -7.0
    rng = np.random.default_rng(3)
    acc = (rng.random(3000) * 4e-3).astype(np.float32)
    cnt = rng.integers(0, 10, 3000).astype(np.float32)
    np.random.seed(11)
    stats = model.densify_and_prune(cu(acc), cu(cnt), scene_extent=8.0,
                                    return_optimizer_state=True)
    np.random.seed(11)
    ref, rstats, keep = DN.densify_and_prune(raw, acc, cnt, scene_extent=8.0)
    say(f"  {stats['cloned']} cloned, {stats['split']} split, {stats['pruned']} pruned")
    assert {k: stats[k] for k in ("cloned", "split", "pruned")} == rstats
    assert stats["cloned"] > 0 and stats["split"] > 0 and stats["pruned"] > 0
    np.testing.assert_array_equal(stats["_keep_idx"], keep)
    assert stats["_new_count"] == rstats["cloned"] + 2 * rstats["split"]
    for k, v in ref.items():
        a = host(model.params[k])
        assert a.shape == v.shape, k
        np.testing.assert_allclose(a, v, rtol=2e-6, atol=2e-6, err_msg=k)


def test_relocate_mcmc_moves_rows():
    say("relocate_mcmc")
    _, model, raw, _ = _model(32, 2000)
    rng = np.random.default_rng(5)
    acc = rng.random(2000).astype(np.float32)
    cnt = rng.integers(0, 4, 2000).astype(np.float32)
    k, dst, src = DN.relocate_select(raw, acc, cnt, relocate_frac=0.05, min_opacity=0.1)
    out = model.relocate_mcmc(cu(acc), cu(cnt), relocate_frac=0.05, min_opacity=0.1,
                              generator=torch.Generator(device="cuda").manual_seed(0))
    assert out["relocated"] == k == 100
    np.testing.assert_array_equal(np.sort(host(out["_moved_idx"])), dst)
    p = {kk: host(v) for kk, v in model.params.items()}
    moved = np.zeros(2000, bool)
    moved[dst] = True
    for kk in raw:
        np.testing.assert_array_equal(p[kk][~moved], raw[kk][~moved], err_msg=kk)
    np.testing.assert_allclose(p["opacities"][dst], np.log(0.05 / 0.95), rtol=1e-6)
    # every moved row is a copy of a source row, up to the rounding of the
    # reference's scatter-add a + (v - a); log-scales shrink by log 1.6
    srcv = raw["sh_rest"][src].reshape(len(src), -1)
    srcs = raw["scales"][src] - np.float32(np.log(1.6))
    for i in dst:
        d = np.abs(srcv - p["sh_rest"][i].ravel()).max(axis=1)
        j = int(np.argmin(d))
        assert d[j] < 1e-6
        np.testing.assert_allclose(p["scales"][i], srcs[j], rtol=0, atol=1e-6)


def test_densify_carries_moments():
    """Moments passed to densify_and_prune follow their rows: a kept row's
    moments move with it, clones and split rows start at zero."""
    say("densify moments")
    _, model, raw, _ = _model(33, 2500)
    raw["opacities"][:40] = -7.0
    model.params["opacities"][:40] = -7.0
    rng = np.random.default_rng(4)
    acc = (rng.random(2500) * 4e-3).astype(np.float32)
    cnt = rng.integers(0, 10, 2500).astype(np.float32)
    moments = {k: {"m": cu(rng.normal(size=raw[k].shape).astype(np.float32)),
                   "v": cu(rng.random(raw[k].shape).astype(np.float32))}
               for k in ("means", "sh_rest", "opacities")}
    old = {k: {s: host(t) for s, t in v.items()} for k, v in moments.items()}
    np.random.seed(5)
    stats = model.densify_and_prune(cu(acc), cu(cnt), scene_extent=8.0, moments=moments,
                                    return_optimizer_state=True)
    new = stats["_moments"]
    keep = stats["_keep_idx"]
    nk = keep.shape[0]
    assert nk == 2500 - stats["pruned"] and stats["cloned"] > 0 and stats["split"] > 0
    for k, slots in new.items():
        for s, t in slots.items():
            a = host(t)
            assert a.shape[0] == model.num_gaussians
            np.testing.assert_array_equal(a[:nk], old[k][s][keep], err_msg=f"{k}.{s}")
            assert not a[nk:].any(), f"{k}.{s}: new rows must start at zero"


def test_relocate_clears_moved_moments():
    say("relocate moments")
    _, model, raw, _ = _model(34, 1500)
    rng = np.random.default_rng(6)
    acc = rng.random(1500).astype(np.float32)
    cnt = rng.integers(0, 4, 1500).astype(np.float32)
    m = cu(rng.normal(size=(1500, 3)).astype(np.float32))
    v = cu(rng.random((1500, 3)).astype(np.float32))
    before = host(m)
    out = model.relocate_mcmc(cu(acc), cu(cnt), relocate_frac=0.05, min_opacity=0.1,
                              jitter_scale=0.0, moments={"means": {"m": m, "v": v}})
    moved = np.zeros(1500, bool)
    moved[host(out["_moved_idx"])] = True
    assert out["relocated"] == moved.sum() > 0
    assert not host(m)[moved].any() and not host(v)[moved].any()
    np.testing.assert_array_equal(host(m)[~moved], before[~moved])


def _knn_reference(pts, ref, k):
    """Brute force of the rule gsx_knn_log_scale restates: float32 squared
    distances summed over x, y, z, stable order by (distance, index)."""
    out = np.empty(len(pts), np.float32)
    for i, q in enumerate(pts):
        d = ((q[None, :] - ref) ** 2).astype(np.float32)
        d = (d[:, 0] + d[:, 1]) + d[:, 2]
        order = np.argsort(d, kind="stable")[:k]
        dk = d[order]
        near = dk[1:k] if dk[0] <= np.float32(1e-12) else dk[:k - 1]
        s = np.float32(0.0)
        for x in near:
            s = np.float32(s + x)
        mean = max(np.float32(s / np.float32(k - 1)), np.float32(1e-8))
        out[i] = np.log(np.sqrt(mean, dtype=np.float32), dtype=np.float32)
    return out


def test_knn_log_scale_matches_bruteforce():
    """from_points' nearest-neighbour scale (model.py:72-92): self hits
    skipped, ties to the lower index, duplicates, a capped variant."""
    say("knn log scale")
    from mlx3d_amd.splatting.density import knn_log_scales

    rng = np.random.default_rng(8)
    pts = rng.normal(0, 1, (3000, 3)).astype(np.float32)
    pts[100:110] = pts[99]  # exact duplicates: zero distances
    pts[200:400] = np.round(pts[200:400] * 4) / 4  # a lattice: many equal distances
    ref = pts[rng.permutation(3000)[:1200]]  # a subset: some queries have no self hit
    for r, k in [(pts, 4), (ref, 4), (pts, 2), (ref, 8)]:
        got = host(knn_log_scales(cu(pts), cu(r), k))
        want = _knn_reference(pts, r, k)
        e = np.abs(got - want).max()
        say(f"  n_ref={len(r)} k={k}: max |d| {e:.2e}")
        assert e <= 2e-6
    capped = host(knn_log_scales(cu(pts), cu(pts), 4, max_scale=0.05))
    assert capped.max() <= np.log(0.05) + 1e-6
    np.testing.assert_array_equal(capped, np.minimum(host(knn_log_scales(cu(pts), cu(pts), 4)),
                                                     np.float32(np.log(0.05))))


@pytest.mark.parametrize("method", ["vanilla", "mcmc", "2dgs"])
def test_trainer_loop(method):
    """Fits a random scene to the render of another for 40 steps: the loss
    falls, density control fires, Adam state follows the table size."""
    say(f"trainer loop {method}")
    cam, gt, _, _ = _model(41, 3000)
    with torch.no_grad():
        target = gt.render(cam)["image"].detach()
    _, model, _, _ = _model(42, 2000, degree=0)
    cfg = TrainerConfig(method=method, densify_from=5, densify_until=30, densify_every=10,
                        densify_grad_threshold=1e-5, opacity_reset_every=1000,
                        sh_increase_every=15,
                        lambda_2d_depth_variance=0.1 if method == "2dgs" else 0.0,
                        lambda_2d_normal_consistency=0.05 if method == "2dgs" else 0.0)
    tr = GaussianTrainer(model, cfg, scene_extent=2.0,
                         generator=torch.Generator(device="cuda").manual_seed(1))
    losses, events = [], 0
    for _ in range(40):
        info = tr.step(cam, target)
        losses.append(info["loss"])
        events += info["densify"] is not None
        n = model.num_gaussians
        for k, opt in tr.optimizers.items():
            assert opt.state[k]["m"].shape[0] == n
        assert np.isfinite(info["loss"])
    say(f"  loss {losses[0]:.4f} -> {losses[-1]:.4f}, N {model.num_gaussians}, events {events}")
    assert losses[-1] < 0.9 * losses[0]
    assert events == 3 and model.active_sh_degree == 2
    if method == "mcmc":
        assert model.num_gaussians == 2000
    else:
        assert model.num_gaussians != 2000
    if method == "2dgs":
        assert float(model.params["scales"][:, 2].max()) <= np.log(1e-4 * 2.0) + 1e-6


def test_2dgs_geometry_terms_leave_screen_stats_alone():
    """The 2DGS geometry render reads the projection's means2d, not the
    probed ones (trainer.py:212-213): from identical state, one step with the
    geometry regularisers on gives the same density statistics as one with
    them off.  The raster backward's float atomics add in run-dependent
    order, so the comparison is relative (1e-5 of the largest entry), far
    below the geometry gradient the probe would otherwise collect."""
    say("2dgs screen statistics with and without geometry terms")
    cam, gt, _, _ = _model(51, 3000)
    with torch.no_grad():
        target = gt.render(cam)["image"].detach()
    stats = []
    for lam_dv, lam_nc in ((0.0, 0.0), (0.5, 0.5)):
        _, model, _, _ = _model(52, 2000, degree=0)
        cfg = TrainerConfig(method="2dgs", densify_from=1, densify_until=100,
                            densify_every=1000, opacity_reset_every=1000,
                            lambda_2d_depth_variance=lam_dv,
                            lambda_2d_normal_consistency=lam_nc)
        tr = GaussianTrainer(model, cfg, scene_extent=2.0)
        info = tr.step(cam, target)
        assert np.isfinite(info["loss"])
        torch.cuda.synchronize()
        stats.append((host(tr.grad_accum), host(tr.grad_count)))
    (a0, c0), (a1, c1) = stats
    np.testing.assert_array_equal(c0, c1)
    assert float(a0.max()) > 0
    e = float(np.abs(a1 - a0).max() / np.abs(a0).max())
    say(f"  grad_accum rel diff {e:.2e}")
    assert e < 1e-5


def test_2dgs_unprojection_maps_follow_the_camera():
    """The 2DGS trainer caches the unprojection maps by camera content: two
    differently posed cameras created one after another (a new object may
    reuse a freed one's id) and a camera moved in place each get their own
    maps, equal to a fresh unprojection_maps call."""
    from mlx3d_amd.cameras import Camera
    from mlx3d_amd.splatting.geometry import unprojection_maps

    say("2dgs unprojection-map cache keyed by camera content")
    _, model, _, _ = _model(61, 1500, degree=0)
    cfg = TrainerConfig(method="2dgs", densify_from=1 << 30, densify_until=1 << 30,
                        opacity_reset_every=1 << 30, lambda_2d_depth_variance=0.2,
                        lambda_2d_normal_consistency=0.2)
    tr = GaussianTrainer(model, cfg, scene_extent=2.0)
    dev = model.params["means"].device
    target = torch.zeros((112, 160, 3), dtype=torch.float32, device=dev)
    for i in range(4):
        eye = (0.0, 0.3 * (i % 2), -4.0 + 0.5 * (i % 2))
        cam = Camera.look_at(eye=eye, at=(0, 0, 0), width=160, height=112, fov=50.0)
        info = tr.step(cam, target)
        assert np.isfinite(info["loss"])
        base, dirs = tr._maps(cam, dev)
        rb, rd = unprojection_maps(cam, dev)
        assert torch.equal(base, rb) and torch.equal(dirs, rd), i
        del cam
    # the same object moved in place
    cam = Camera.look_at(eye=(0.0, 0.0, -4.0), at=(0, 0, 0), width=160, height=112, fov=50.0)
    tr.step(cam, target)
    cam.t = torch.as_tensor(cam.t, dtype=torch.float32) + 0.25
    base, dirs = tr._maps(cam, dev)
    rb, rd = unprojection_maps(cam, dev)
    assert torch.equal(base, rb) and torch.equal(dirs, rd)
