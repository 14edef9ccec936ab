"""Pins the oracle's two exps against float64 exp -- orc_expf (the
activations, <= 1 ulp) and orc_splat_expf (metal::exp of the compositing
loops, rasterize.py:80,171,274) -- and the compositing power
(rasterize.py:77-78) against float64 and closed forms."""
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


# --- the compositing loops' exp and power (orc_splat_expf / orc_splat_power)

def _splat_ulps(x):
    y = O.splat_expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    return np.abs(y - ref) / ulp


def test_splat_exp_accuracy():
    # every power that can pass the alpha test lies in [-ln 255, 0]; exhaustive
    # float32 sweeps give 2.02 ulp on [-6, 0], 2.19 on [-12, 0], 4.75 on [-87, 0]
    x = np.linspace(-6.0, 0.0, 1_000_001, dtype=np.float32)
    assert _splat_ulps(x).max() <= 2.05
    x = np.linspace(-12.0, 0.0, 1_000_001, dtype=np.float32)
    assert _splat_ulps(x).max() <= 2.2
    x = np.linspace(-86.0, 0.0, 1_000_001, dtype=np.float32)
    assert _splat_ulps(x).max() <= 4.8
    rng = np.random.default_rng(7)
    x = (-rng.exponential(2.0, 1_000_000)).astype(np.float32)
    assert _splat_ulps(x[x > -86]).max() <= 4.8


def test_splat_exp_special_values():
    x = np.array([0.0, -0.0, -86.5, -1000.0, 88.5, np.inf, -np.inf, np.nan, -np.log(2.0)],
                 np.float32)
    y = O.splat_expf(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert y[2] == 0.0 and y[3] == 0.0 and y[6] == 0.0
    assert np.isinf(y[4]) and np.isinf(y[5])
    assert np.isnan(y[7])
    assert abs(float(y[8]) - 0.5) <= 2 * np.spacing(np.float32(0.5))


def test_splat_power_against_float64():
    rng = np.random.default_rng(11)
    worst = 0.0
    for _ in range(20000):
        s1, s2 = np.exp(rng.normal(0, 1.5, 2))
        rho = rng.uniform(-0.95, 0.95)
        a, c = 1 / s1**2, 1 / s2**2
        b = -rho / (s1 * s2)
        a, b, c = (float(np.float32(v)) for v in (a, b, c))
        dx, dy = (float(np.float32(v)) for v in rng.normal(0, 3 * max(s1, s2), 2))
        p = O.splat_power(a, b, c, dx, dy)
        exact = -0.5 * (a * dx * dx + c * dy * dy) - b * dx * dy
        scale = 0.5 * (a * dx * dx + c * dy * dy) + abs(b * dx * dy)
        worst = max(worst, abs(p - exact) / scale)
    # (A dx + B dy) dx + (C dy) dy with five roundings: the error is at most
    # 2 eps scale + eps |power| <= 3 eps scale (eps = 2^-24)
    assert worst <= 3 * 2.0**-24


def test_splat_power_relative_bound_for_culling():
    # the quadrant culling assumes the float32 power is within 4.8e-4 of the
    # exact value, relative, when b^2 < 0.999 a c (nearly degenerate conics)
    rng = np.random.default_rng(12)
    worst = 0.0
    for _ in range(20000):
        s1, s2 = np.exp(rng.normal(0, 1.5, 2))
        rho = rng.uniform(-1, 1) * 0.9994
        a, c = 1 / s1**2, 1 / s2**2
        b = rho * np.sqrt(a * c)
        a, b, c = (float(np.float32(v)) for v in (a, b, c))
        if not b * b < 0.999 * a * c:
            continue
        dx, dy = (float(np.float32(v)) for v in rng.normal(0, 3 * max(s1, s2), 2))
        exact = -0.5 * (a * dx * dx + c * dy * dy) - b * dx * dy
        if exact == 0.0:
            continue
        worst = max(worst, abs(O.splat_power(a, b, c, dx, dy) - exact) / abs(exact))
    assert worst <= 4.8e-4


def test_splat_power_never_positive_for_plain_conics():
    # The forward's plain batches skip the power > 0 test: a conic with
    # a + c in [1e-12, 1e19) and det > 1e-6 (a + c)^2 (float32, as
    # plain_gaussian computes them) never yields a positive float32 power.
    # Worst cases: condition numbers up to the bound, offsets along the
    # minor axis (where the exact power is smallest), offsets of a few
    # 2^-25 steps (the least nonzero pixel offset) up to 1e3 pixels.
    rng = np.random.default_rng(13)
    f32 = np.float32
    checked = 0
    for _ in range(4000):
        lam = 10.0 ** rng.uniform(-10, 6)
        kappa = 10.0 ** rng.uniform(0, 6.05)
        th = rng.uniform(0, np.pi)
        ct, st = np.cos(th), np.sin(th)
        l1, l2 = lam, lam * kappa
        a = f32(l1 * ct * ct + l2 * st * st)
        c = f32(l1 * st * st + l2 * ct * ct)
        b = f32((l1 - l2) * ct * st)
        tr = f32(a + c)
        det = f32(np.float64(a) * np.float64(c) - np.float64(f32(b * b)))
        if not (1e-12 <= tr < 1e19 and det > f32(1e-6) * f32(tr * tr)):
            continue
        for _ in range(8):
            r = 2.0 ** rng.uniform(-25, 10)
            u = rng.normal(0, 1e-3)  # near the minor axis (eigenvalue l1)
            dx = f32(r * (ct + u * st))
            dy = f32(r * (st - u * ct))
            if rng.random() < 0.3:  # exact multiples of the least offset
                dx = f32(np.round(dx * 2.0**25) * 2.0**-25)
                dy = f32(np.round(dy * 2.0**25) * 2.0**-25)
            p = O.splat_power(float(a), float(b), float(c), float(dx), float(dy))
            assert not p > 0.0, (a, b, c, dx, dy, p)
            checked += 1
    assert checked > 10000
    # the bound is needed: a conic with det / (a + c)^2 = 2e-9 (condition
    # number ~5e8) gives a positive power near its minor axis
    assert O.splat_power(311017312.0, -62711700.0, 12644819.0, 0.0762607529759407,
                         0.3782143294811249) > 0.0


def test_splat_power_closed_forms():
    # isotropic unit conic: -(dx^2 + dy^2)/2, exact for small integers
    for dx, dy in ((0, 0), (1, 0), (0, -2), (3, 4), (-5, 12)):
        assert O.splat_power(1.0, 0.0, 1.0, dx, dy) == -(dx * dx + dy * dy) / 2
    # the sign of the cross term: b > 0 lowers the power where dx dy > 0
    assert O.splat_power(1.0, 0.5, 1.0, 1.0, 1.0) == -1.5
    assert O.splat_power(1.0, 0.5, 1.0, 1.0, -1.0) == -0.5
    # a and c are not swapped
    assert O.splat_power(2.0, 0.0, 8.0, 1.0, 0.0) == -1.0
    assert O.splat_power(2.0, 0.0, 8.0, 0.0, 1.0) == -4.0
