"""How far the shipped compositing arithmetic lies from the reference's
literal expressions.

The kernels and the oracle evaluate the power as the factored
(A dx + B dy) dx + (C dy) dy, exp as the fitted splat_exp, and accumulate
colours with one multiply-add.  rasterize.py:75-76 writes the power as
-0.5 (a dx dx + c dy dy) - b dx dy, :80 calls metal::exp and :84 writes
`acc += rgb * (alpha * T)`; Metal's fast-math may or may not contract and
reassociate them, so no single arithmetic is "the reference's".  The oracle's
ORC_ARITH_* modes evaluate those expressions literally (op by op, the float32
rounding of the double exp) so the number of n_contrib and image decisions
the choice changes can be counted.

CPU tests: the literal modes are pinned (literal power against numpy's
op-by-op float32, one tile against a pure-Python compositing loop), and the
counts at C1 stay small.  Run as a script for the full-size counts at the
benchmark configurations:

    python tests/test_oracle_literal.py [configs...]
"""

from __future__ import annotations

import os
import sys

import numpy as np

if __name__ == "__main__":  # as a script: the repository root and tests/ on the path
    _here = os.path.dirname(os.path.abspath(__file__))
    sys.path[:0] = [os.path.dirname(_here), _here]

from oracle import oracle as O  # noqa: E402
from refimpl import oracle_camera  # noqa: E402

MODES = {
    "power": O.ARITH_LITERAL_POWER,
    "acc": O.ARITH_SEPARATE_ACC,
    "exp": O.ARITH_ROUNDED_EXP,
    "all": O.ARITH_LITERAL_POWER | O.ARITH_SEPARATE_ACC | O.ARITH_ROUNDED_EXP,
}


def test_literal_power_is_op_by_op_float32():
    rng = np.random.default_rng(0)
    n = 20000
    a, c = (rng.uniform(0.01, 3.0, n).astype(np.float32) for _ in range(2))
    b = (rng.uniform(-0.9, 0.9, n) * np.sqrt(a * c)).astype(np.float32)
    dx, dy = (rng.uniform(-6, 6, n).astype(np.float32) for _ in range(2))
    h = np.float32(-0.5)
    want = h * ((a * dx) * dx + (c * dy) * dy) - (b * dx) * dy  # float32 throughout
    got = np.array([O.literal_power(*map(float, v)) for v in zip(a, b, c, dx, dy)], np.float32)
    np.testing.assert_array_equal(got.view(np.int32), want.view(np.int32))
    # the factored form differs from the literal one in some last bits
    fac = np.array([O.splat_power(*map(float, v)) for v in zip(a[:2000], b[:2000], c[:2000],
                                                               dx[:2000], dy[:2000])], np.float32)
    assert (fac != want[:2000]).any()


def _tile_literal(xy, co, op, rgb, ids, W, H):
    """rasterize.py:40-96 for one 16x16 tile in pure Python, every float32
    operation rounded separately, exp the rounding of the double exp."""
    f = np.float32
    img = np.zeros((H, W, 3), np.float32)
    nct = np.zeros((H, W), np.int32)
    for py in range(H):
        for px in range(W):
            T, acc, last = f(1.0), np.zeros(3, np.float32), 0
            pxf, pyf = f(px) + f(0.5), f(py) + f(0.5)
            for j, g in enumerate(ids):
                dx, dy = xy[g, 0] - pxf, xy[g, 1] - pyf
                a, b, c = co[g]
                power = f(-0.5) * ((a * dx) * dx + (c * dy) * dy) - (b * dx) * dy
                if power > 0:
                    continue
                alpha = min(f(0.99), op[g] * f(np.exp(np.float64(power))))
                if alpha < f(1.0) / f(255.0):
                    continue
                nT = T * (f(1.0) - alpha)
                if nT < f(1e-4):
                    break
                acc = acc + rgb[g] * (alpha * T)
                T, last = nT, j + 1
            img[py, px] = acc
            nct[py, px] = last
    return img, nct


def test_all_literal_matches_python_loop_on_one_tile():
    rng = np.random.default_rng(1)
    n, W, H = 40, 16, 16
    xy = rng.uniform(-2, 18, (n, 2)).astype(np.float32)
    s = rng.uniform(1.0, 6.0, (n, 2))
    rho = rng.uniform(-0.6, 0.6, n)
    cov = np.stack([s[:, 0] ** 2, rho * s[:, 0] * s[:, 1], s[:, 1] ** 2], 1)
    det = cov[:, 0] * cov[:, 2] - cov[:, 1] ** 2
    co = np.stack([cov[:, 2] / det, -cov[:, 1] / det, cov[:, 0] / det], 1).astype(np.float32)
    op = rng.uniform(0.05, 0.999, n).astype(np.float32)
    rgb = rng.uniform(size=(n, 3)).astype(np.float32)
    ids = np.arange(n, dtype=np.int32)
    ranges = np.array([[0, n]], np.int32)
    r = O.raster_fwd(xy, co, op, rgb, ids, ranges, W, H, arith=MODES["all"])
    img, nct = _tile_literal(xy, co, op, rgb, ids, W, H)
    np.testing.assert_array_equal(r["n_contrib"], nct)
    np.testing.assert_array_equal(r["image"].view(np.int32), img.view(np.int32))
    # and the shipped arithmetic is a different one on the same tile
    r0 = O.raster_fwd(xy, co, op, rgb, ids, ranges, W, H)
    assert (r0["image"] != r["image"]).any()


def flip_counts(config: int, view: int = 0, threads: int | None = None) -> dict:
    """Shipped vs literal arithmetic on one view of a benchmark
    configuration: pixels whose n_contrib differs, pixels with any image
    channel differing, and the largest image difference."""
    from mlx3d_amd import scenes

    threads = threads or O.default_threads()
    sc = scenes.make_scene(config)
    cam = sc.cameras[view]
    flags = O.LOG_SCALES | O.LOGIT_OPACITY | (O.ANTIALIAS if sc.antialias else 0)
    sh = None if sc.sh_dc is None else np.concatenate([sc.sh_dc, sc.sh_rest], 1)
    pre = O.preprocess_fwd(oracle_camera(cam), sc.means, sc.quats, sc.log_scales,
                           sc.logit_opacities, sh=sh, degree=sc.sh_degree, flags=flags,
                           threads=threads)
    feats = pre["colors"] if sh is not None else sc.features
    ids, ranges, _, _ = O.bin_gaussians(pre["means2d"], pre["radii"], pre["depths"], cam.width,
                                        cam.height, threads=threads)

    def run(arith):
        return O.raster_fwd(pre["means2d"], pre["conics"], pre["opac_eff"], feats, ids, ranges,
                            cam.width, cam.height, threads=threads, arith=arith)

    base = run(0)
    out = {"config": sc.name, "pixels": cam.width * cam.height, "pairs_D": int(ids.shape[0])}
    for name, mode in MODES.items():
        r = run(mode)
        dn = r["n_contrib"] != base["n_contrib"]
        di = (r["image"] != base["image"]).any(-1)
        out[name] = {"n_contrib": int(dn.sum()), "image": int(di.sum()),
                     "max_abs": float(np.abs(r["image"] - base["image"]).max())}
    return out


def test_flip_counts_c1_are_small():
    res = flip_counts(1)
    for name in MODES:
        m = res[name]
        # a handful of threshold decisions move; images stay within 1e-3
        assert m["n_contrib"] <= 0.01 * res["pixels"], (name, m)
        assert m["max_abs"] < 1e-3, (name, m)
    assert res["acc"]["n_contrib"] == 0  # accumulation order never moves a decision


if __name__ == "__main__":
    cfgs = [int(a) for a in sys.argv[1:]] or [1, 2, 3, 4, 5]
    print("| config | pixels | D | mode | n_contrib flips | image pixels changed | max abs |")
    print("|---|---|---|---|---|---|---|")
    for c in cfgs:
        res = flip_counts(c)
        for name in MODES:
            m = res[name]
            print(f"| {res['config']} | {res['pixels']} | {res['pairs_D']} | {name} | "
                  f"{m['n_contrib']} | {m['image']} | {m['max_abs']:.3g} |", flush=True)
