"""Helpers shared by the GPU parity tests: host<->device conversion and the
oracle's forward/backward chain on the same float32 inputs."""

from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import oracle as O
from refimpl import oracle_camera

DEV = "cuda"


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def cu(a, dtype=None) -> torch.Tensor:
    t = torch.as_tensor(np.ascontiguousarray(np.asarray(a)))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(DEV)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def assert_bits(a, b, what=""):
    a = np.ascontiguousarray(np.asarray(a, np.float32))
    b = np.ascontiguousarray(np.asarray(b, np.float32))
    assert a.shape == b.shape, f"{what}: shape {a.shape} vs {b.shape}"
    ai, bi = a.view(np.int32), b.view(np.int32)
    bad = ai != bi
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} differ; first {idx.tolist()} "
                             f"gpu={a[bad][:5]} oracle={b[bad][:5]}")


def matrix_core_channels(C: int) -> np.ndarray:
    """Channels that the rasterizers sum on the matrix cores: those of the
    32-channel blocks that hold 17 to 32 channels."""
    mask = np.zeros(C, bool)
    for c0 in range(0, C, 32):
        nc = min(32, C - c0)
        if nc > 16:
            mask[c0:c0 + nc] = True
    return mask


def assert_features(a, b, what="features", atol=1e-5):
    """Rendered channels against the oracle: bitwise where the channel sums
    run on the vector ALU (the oracle's order of multiply-adds), within
    `atol` absolute (the north star's image tolerance) where a 32-channel
    block sums on the matrix cores in another order.  Non-finite values
    must sit at the same places with the same value."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    assert a.shape == b.shape, f"{what}: shape {a.shape} vs {b.shape}"
    mask = matrix_core_channels(a.shape[-1])
    assert_bits(a[..., ~mask], b[..., ~mask], what)
    am, bm = a[..., mask], b[..., mask]
    fin = np.isfinite(bm)
    np.testing.assert_array_equal(np.isfinite(am), fin, err_msg=what)
    np.testing.assert_array_equal(np.isnan(am), np.isnan(bm), err_msg=what)
    np.testing.assert_array_equal(am[np.isinf(bm)], bm[np.isinf(bm)], err_msg=what)
    if fin.any():
        err = float(np.abs(am[fin].astype(np.float64) - bm[fin]).max())
        assert err <= atol, f"{what}: max abs error {err:.3e} > {atol}"


def rel_err(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / (np.abs(b).max() + 1e-30))


def oracle_forward(cam, means, quats, scales, opac, sh=None, degree=0, colors=None, flags=0,
                   bg=None, depth=False, threads=None, tiles=None):
    threads = threads or O.default_threads()
    oc = oracle_camera(cam)
    pre = O.preprocess_fwd(oc, means, quats, scales, opac, sh=sh, degree=degree, flags=flags,
                           threads=threads)
    feats = pre["colors"] if sh is not None else colors
    ids, ranges, _, _ = O.bin_gaussians(pre["means2d"], pre["radii"], pre["depths"], cam.width,
                                        cam.height, threads=threads)
    r = O.raster_fwd(pre["means2d"], pre["conics"], pre["opac_eff"], feats, ids, ranges,
                     cam.width, cam.height, bg=bg, depths=pre["depths"] if depth else None,
                     tiles=tiles, threads=threads)
    return pre, feats, ids, ranges, r


def oracle_backward(cam, means, quats, scales, opac, pre, feats, ids, ranges, r, g_img, g_alpha,
                    sh=None, degree=0, flags=0, bg=None, threads=None):
    threads = threads or O.default_threads()
    oc = oracle_camera(cam)
    gr = O.raster_bwd(pre["means2d"], pre["conics"], pre["opac_eff"], feats, ids, ranges,
                      cam.width, cam.height, r["final_T"], r["n_contrib"], g_img,
                      grad_final_T=None if g_alpha is None else -g_alpha, bg=bg,
                      threads=threads)
    K = 0 if sh is None else sh.shape[1]
    g = O.preprocess_bwd(oc, means, quats, scales, opac, pre["colors"] if sh is not None else None,
                         K, degree, flags, gr["means2d"], gr["conics"], gr["opacities"],
                         gr["features"] if sh is not None else None, threads=threads)
    g["features"] = gr["features"]
    g["raster"] = gr
    return g
