"""Seeded synthetic scenes for the five benchmark configurations.

Each generator draws with numpy PCG64 ``default_rng(seed)`` in float64 and
returns float32 host arrays, so the GPU path and the CPU oracle see
identical bytes.  Parameters are returned raw in GaussianModel form
(``scales`` log-sigma, ``opacities`` logits, ``sh_dc`` / ``sh_rest``) and
the activated values are their exp / sigmoid.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from .cameras import Camera

__all__ = ["Scene", "make_scene", "CONFIGS"]


@dataclass
class Scene:
    name: str
    means: np.ndarray
    quats: np.ndarray
    log_scales: np.ndarray
    logit_opacities: np.ndarray
    sh_dc: np.ndarray | None          # (N, 1, 3)
    sh_rest: np.ndarray | None        # (N, K-1, 3)
    features: np.ndarray | None       # (N, C) for the feature config
    sh_degree: int
    cameras: list = field(default_factory=list)
    antialias: bool = False
    depth: bool = False
    backward: bool = True
    target_seed: int = 0

    @property
    def n(self) -> int:
        return self.means.shape[0]

    @property
    def scales(self) -> np.ndarray:
        return np.exp(self.log_scales.astype(np.float64)).astype(np.float32)

    @property
    def opacities(self) -> np.ndarray:
        return (1.0 / (1.0 + np.exp(-self.logit_opacities.astype(np.float64)))).astype(np.float32)

    @property
    def channels(self) -> int:
        return self.features.shape[1] if self.features is not None else 3

    def target(self, cam: Camera) -> np.ndarray:
        rng = np.random.default_rng(self.target_seed)
        return rng.uniform(size=(cam.height, cam.width, self.channels)).astype(np.float32)


def _unit_quats(rng, n):
    q = rng.standard_normal((n, 4))
    return (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)


def _logit(p):
    p = np.clip(p, 1e-7, 1 - 1e-7)
    return np.log(p / (1 - p))


def _sh3(rng, n):
    dc = rng.uniform(-0.5, 0.5, (n, 1, 3)).astype(np.float32)
    rest = (rng.standard_normal((n, 15, 3)) * 0.05).astype(np.float32)
    return dc, rest


def _knn_log_scale(points: np.ndarray) -> np.ndarray:
    """log sqrt(mean of the 3 nearest squared distances), as
    GaussianModel.from_points (model.py:81-89); brute force in chunks."""
    p = points.astype(np.float64)
    out = np.empty(p.shape[0])
    sq = (p * p).sum(1)
    for s in range(0, p.shape[0], 1024):
        q = p[s:s + 1024]
        d = np.maximum((q * q).sum(1)[:, None] - 2 * q @ p.T + sq[None], 0.0)
        part = np.partition(d, 3, axis=1)[:, :4]
        part.sort(axis=1)
        nearest = np.where(part[:, :1] <= 1e-12, part[:, 1:4], part[:, 0:3])
        out[s:s + 1024] = np.maximum(nearest.mean(1), 1e-8)
    return np.log(np.sqrt(out))


def config1(seed: int = 1) -> Scene:
    """10k Gaussians, DC colour only (16 coefficients stored, degree 0),
    isotropic kNN scales, identity rotations, opacity 0.1, 256x256, fwd."""
    rng = np.random.default_rng(seed)
    n = 10_000
    means = (rng.standard_normal((n, 3)) * 0.5).astype(np.float32)
    rgb = rng.uniform(size=(n, 3)).astype(np.float32)
    ls = np.repeat(_knn_log_scale(means)[:, None], 3, 1).astype(np.float32)
    quats = np.zeros((n, 4), np.float32)
    quats[:, 0] = 1.0
    C0 = 0.28209479177387814
    dc = ((rgb - 0.5) / C0)[:, None, :].astype(np.float32)
    rest = np.zeros((n, 15, 3), np.float32)
    logit = np.full(n, math.log(0.1 / 0.9), np.float32)
    cam = Camera.look_at(eye=(0, 0, -4.0), width=256, height=256, fov=60.0)
    return Scene("c1_10k_sh0_256", means, quats, ls, logit, dc, rest, None, 0, [cam],
                 depth=True, backward=False)


def config2(seed: int = 2) -> Scene:
    """100k Gaussians in [-1.5,1.5]^3, SH3, 1280x720, fwd + L1 + bwd."""
    rng = np.random.default_rng(seed)
    n = 100_000
    means = rng.uniform(-1.5, 1.5, (n, 3)).astype(np.float32)
    ls = rng.normal(-4.0, 0.5, (n, 3)).astype(np.float32)
    quats = _unit_quats(rng, n)
    logit = rng.standard_normal(n).astype(np.float32)
    dc, rest = _sh3(rng, n)
    cam = Camera.look_at(eye=(0, 0, -4.0), width=1280, height=720, fov=60.0)
    return Scene("c2_100k_sh3_720p", means, quats, ls, logit, dc, rest, None, 3, [cam],
                 target_seed=102)


def orbit_cameras(seed: int, count: int, radius: float, width: int, height: int):
    rng = np.random.default_rng(seed)
    cams = []
    for _ in range(count):
        th = rng.uniform(0, 2 * math.pi)
        ph = math.radians(rng.uniform(-30.0, 30.0))
        eye = (radius * math.cos(ph) * math.sin(th), radius * math.sin(ph),
               -radius * math.cos(ph) * math.cos(th))
        cams.append(Camera.look_at(eye=eye, width=width, height=height, fov=60.0))
    return cams


def config3(seed: int = 3, n: int = 1_000_000) -> Scene:
    """1M Gaussians, 70% on sphere shells r~U(1,3) (+N(0,0.02) jitter), 30%
    uniform in [-4,4]^3; SH3; antialias; 8 orbit views at radius 5, 1080p."""
    rng = np.random.default_rng(seed)
    n_shell = int(round(0.7 * n))
    d = rng.standard_normal((n_shell, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    r = rng.uniform(1.0, 3.0, (n_shell, 1))
    shell = d * r + rng.normal(0.0, 0.02, (n_shell, 3))
    box = rng.uniform(-4.0, 4.0, (n - n_shell, 3))
    means = np.concatenate([shell, box]).astype(np.float32)
    ls = rng.normal(-4.5, 0.7, (n, 3)).astype(np.float32)
    quats = _unit_quats(rng, n)
    logit = rng.normal(0.0, 1.5, n).astype(np.float32)
    dc, rest = _sh3(rng, n)
    cams = orbit_cameras(1003, 8, 5.0, 1920, 1080)
    return Scene("c3_1m_sh3_aa_1080p_8views", means, quats, ls, logit, dc, rest, None, 3, cams,
                 antialias=True, target_seed=103)


def config4(seed: int = 4, n: int = 3_000_000) -> Scene:
    """3M Gaussians in [-3,3]^3 with heavy-tailed scales (97% exp(N(-5,0.5)),
    3% exp(N(-1.5,0.3))); SH3; 1080p; camera at (0,0,-5) (unspecified in the
    config; recorded here)."""
    rng = np.random.default_rng(seed)
    means = rng.uniform(-3.0, 3.0, (n, 3)).astype(np.float32)
    big = rng.uniform(size=n) < 0.03
    ls = np.where(big[:, None], rng.normal(-1.5, 0.3, (n, 3)), rng.normal(-5.0, 0.5, (n, 3)))
    quats = _unit_quats(rng, n)
    logit = rng.standard_normal(n).astype(np.float32)
    dc, rest = _sh3(rng, n)
    cam = Camera.look_at(eye=(0, 0, -5.0), width=1920, height=1080, fov=60.0)
    return Scene("c4_3m_heavytail_1080p", means, quats, ls.astype(np.float32), logit, dc, rest,
                 None, 3, [cam], target_seed=104)


def config5(seed: int = 5, n: int = 500_000) -> Scene:
    """500k Gaussians in [-2,2]^3 carrying 32 N(0,1) features; 1280x720 with
    depth; camera at (0,0,-4) (unspecified in the config; recorded here)."""
    rng = np.random.default_rng(seed)
    means = rng.uniform(-2.0, 2.0, (n, 3)).astype(np.float32)
    ls = rng.normal(-4.0, 0.5, (n, 3)).astype(np.float32)
    quats = _unit_quats(rng, n)
    logit = rng.standard_normal(n).astype(np.float32)
    feats = rng.standard_normal((n, 32)).astype(np.float32)
    cam = Camera.look_at(eye=(0, 0, -4.0), width=1280, height=720, fov=60.0)
    return Scene("c5_500k_feat32_720p_depth", means, quats, ls, logit, None, None, feats, 0,
                 [cam], depth=True, target_seed=105)


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


def make_scene(config: int, **kw) -> Scene:
    return CONFIGS[config](**kw)


def ico_sphere(level: int = 1, radius: float = 1.0):
    """(verts (V, 3) float32, faces (F, 3) int32): a unit icosahedron whose
    triangles are split into four, `level` times, new vertices pushed onto
    the sphere (20 * 4^level faces; the reference benchmarks its rasterizer
    on level 5, 20 480 faces, examples/benchmark.py:44)."""
    t = (1.0 + 5 ** 0.5) / 2.0
    v = [(-1, t, 0), (1, t, 0), (-1, -t, 0), (1, -t, 0), (0, -1, t), (0, 1, t), (0, -1, -t),
         (0, 1, -t), (t, 0, -1), (t, 0, 1), (-t, 0, -1), (-t, 0, 1)]
    verts = [np.array(p, np.float64) / np.linalg.norm(p) for p in v]
    faces = [(0, 11, 5), (0, 5, 1), (0, 1, 7), (0, 7, 10), (0, 10, 11), (1, 5, 9), (5, 11, 4),
             (11, 10, 2), (10, 7, 6), (7, 1, 8), (3, 9, 4), (3, 4, 2), (3, 2, 6), (3, 6, 8),
             (3, 8, 9), (4, 9, 5), (2, 4, 11), (6, 2, 10), (8, 6, 7), (9, 8, 1)]
    for _ in range(level):
        cache, nf = {}, []

        def mid(a, b):
            key = (min(a, b), max(a, b))
            if key not in cache:
                m = verts[a] + verts[b]
                verts.append(m / np.linalg.norm(m))
                cache[key] = len(verts) - 1
            return cache[key]

        for a, b, c in faces:
            ab, bc, ca = mid(a, b), mid(b, c), mid(c, a)
            nf += [(a, ab, ca), (b, bc, ab), (c, ca, bc), (ab, bc, ca)]
        faces = nf
    return (np.array(verts) * radius).astype(np.float32), np.array(faces, np.int32)

