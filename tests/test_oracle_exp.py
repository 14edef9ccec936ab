"""Pins the oracle's exp (the stand-in for metal::exp, rasterize.py:80,171,274)
against float64 exp: <= 1 ulp everywhere it is used, exact special cases."""

import numpy as np

from oracle import oracle as O


def _ulps(x):
    y = O.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    return np.abs(y - ref) / ulp


def test_exp_accuracy_raster_range():
    # every power the rasterizer can exponentiate after its alpha test
    x = np.linspace(-10.0, 0.0, 400_001, dtype=np.float32)
    assert _ulps(x).max() <= 1.0


def test_exp_accuracy_full_range():
    x = np.linspace(-86.0, 88.0, 400_001, dtype=np.float32)
    assert _ulps(x).max() <= 1.0
    # dense float32 sweep around 0 (every representable value in [-2^-10, 2^-10])
    u = np.arange(0, 2**23, 97, dtype=np.uint32) | np.uint32(0x3A000000)
    small = u.view(np.float32)
    assert _ulps(np.concatenate([small, -small])).max() <= 1.0


def test_exp_special_values():
    x = np.array([0.0, -0.0, -86.5, -1000.0, 88.5, np.inf, -np.inf, np.nan], np.float32)
    y = O.expf(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert y[2] == 0.0 and y[3] == 0.0 and y[6] == 0.0
    assert np.isinf(y[4]) and np.isinf(y[5])
    assert np.isnan(y[7])


def test_exp_monotone():
    x = np.linspace(-20.0, 0.0, 200_001, dtype=np.float32)
    y = O.expf(x)
    assert np.all(np.diff(y) >= 0)
