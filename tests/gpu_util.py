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
