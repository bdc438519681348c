"""The shared elementary functions (include/mdnav_math.h) against float64
numpy: these pin the numerics that both the oracle and the HIP path compile."""
import numpy as np
import pytest

from oracle_lib import math_batch


def ulps(got, want64):
    want = want64.astype(np.float32)
    spacing = np.spacing(np.abs(want).astype(np.float32))
    spacing = np.where(spacing == 0, np.float32(1e-45), spacing)
    return np.abs(got.astype(np.float64) - want64) / spacing.astype(np.float64)


def test_exp_expm1_accuracy():
    x = np.linspace(-30, 30, 200001, dtype=np.float32)
    assert ulps(math_batch("exp", x), np.exp(x.astype(np.float64))).max() <= 2.0
    x = np.linspace(-10, 20, 200001, dtype=np.float32)
    assert ulps(math_batch("expm1", x), np.expm1(x.astype(np.float64))).max() <= 3.0
    assert math_batch("exp", np.array([0.0], np.float32))[0] == 1.0
    assert math_batch("exp", np.array([100.0], np.float32))[0] == np.inf
    assert math_batch("exp", np.array([-200.0], np.float32))[0] == 0.0


def test_log_accuracy():
    x = np.concatenate([np.geomspace(1e-7, 1e4, 200001), np.linspace(0.5, 2.0, 10001)]).astype(np.float32)
    y = math_batch("log", x)
    ref = np.log(x.astype(np.float64))
    err = np.abs(y - ref)
    # relative-to-ulp away from log(1)=0, absolute near it
    assert (np.minimum(ulps(y, ref), err / 1.2e-7)).max() <= 3.0
    assert math_batch("log", np.array([1.0], np.float32))[0] == 0.0
    assert math_batch("log", np.array([0.0], np.float32))[0] == -np.inf


def test_sin_cos_accuracy():
    x = np.linspace(-12, 12, 400001, dtype=np.float32)
    for fn, ref in (("sin", np.sin), ("cos", np.cos)):
        y = math_batch(fn, x)
        assert np.abs(y - ref(x.astype(np.float64))).max() < 2.5e-7, fn
    assert math_batch("sin", np.array([0.0], np.float32))[0] == 0.0
    assert math_batch("cos", np.array([0.0], np.float32))[0] == 1.0
    # the Box-Muller argument range [0, 2pi) stays within a couple of ulp
    x = np.linspace(0, 6.2831853, 100001, dtype=np.float32)
    assert np.abs(math_batch("cos", x) - np.cos(x.astype(np.float64))).max() < 1.8e-7


def test_tanh_sigmoid_accuracy():
    x = np.linspace(-15, 15, 300001, dtype=np.float32)
    y = math_batch("tanh", x)
    ref = np.tanh(x.astype(np.float64))
    assert (np.minimum(ulps(y, ref), np.abs(y - ref) / 6e-8)).max() <= 4.0
    assert np.all(np.abs(y) <= 1.0)
    assert np.array_equal(y[::-1], -y)  # odd symmetry holds exactly
    s = math_batch("sigmoid", x)
    assert np.abs(s - 1 / (1 + np.exp(-x.astype(np.float64)))).max() < 2e-7


@pytest.mark.parametrize("fn", ["exp", "log", "tanh"])
def test_monotone(fn):
    x = np.linspace(0.01 if fn == "log" else -8, 8, 100001, dtype=np.float32)
    y = math_batch(fn, x)
    assert np.all(np.diff(y) >= 0)


def test_native_camera_rays_closed_form():
    """sensor_profile.hpp:81-91 at the native tangents (1, 0.8): the corner
    pixel (row 0, col 0) looks along (1, 0.95, 0.75) normalised, the centre
    rows and columns straddle the optical axis symmetrically, and the legacy
    rays are the tan_v = 0.75 case."""
    from oracle_lib import oracle, ptr
    F = np.float32
    nat = np.zeros((320, 3), F)
    leg = np.zeros((320, 3), F)
    oracle().orc_camera_rays_tan(F(0.8), ptr(nat))
    oracle().orc_camera_rays(ptr(leg))
    d = np.array([1.0, 0.95, 0.75])
    assert np.abs(nat[0] - d / np.linalg.norm(d)).max() < 2e-7
    # pixel (15, 19): the opposite corner
    assert np.abs(nat[15 * 20 + 19] - np.array([1.0, -0.95, -0.75]) / np.linalg.norm(d)).max() < 2e-7
    assert np.allclose(nat[:, 0] ** 2 + nat[:, 1] ** 2 + nat[:, 2] ** 2, 1.0, atol=3e-7)
    # up-down mirror: row r and row 15-r differ only in the sign of z
    assert np.array_equal(nat[0:20, 2], -nat[300:320, 2]) and np.array_equal(nat[0:20, :2], nat[300:320, :2])
    leg2 = np.zeros((320, 3), F)
    oracle().orc_camera_rays_tan(F(0.75), ptr(leg2))
    assert leg.tobytes() == leg2.tobytes()


def atan2_batch(y, x):
    from oracle_lib import oracle, ptr
    y = np.ascontiguousarray(y, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(y)
    oracle().orc_atan2_batch(ptr(y), ptr(x), ptr(out), y.size)
    return out


def test_atan2_accuracy_and_special_values():
    """atan2_f (the guided mode 16's yaw, sim.metal:233) against float64
    arctan2 over all four quadrants, magnitudes 1e-30..1e30 and both axes:
    within 4 ulp of the result (measured 3.1 over 10 M uniform samples in
    [-2, 2]^2; 4e-45 absolute near zero), and the C99 Annex
    F special values exactly: signed zeros, x = -0 as negative, infinities,
    NaN."""
    rng = np.random.default_rng(11)
    mag = lambda n: (10.0 ** rng.uniform(-30, 30, n)) * rng.choice([-1, 1], n)
    y = np.concatenate([mag(200000), rng.uniform(-2, 2, 200000), np.sin(np.linspace(0, 2 * np.pi, 20001)),
                        np.zeros(5)]).astype(np.float32)
    x = np.concatenate([mag(200000), rng.uniform(-2, 2, 200000), np.cos(np.linspace(0, 2 * np.pi, 20001)),
                        np.array([1, -1, 2, -2, 3])]).astype(np.float32)
    got = atan2_batch(y, x)
    want = np.arctan2(y.astype(np.float64), x.astype(np.float64))
    assert (np.minimum(ulps(got, want), np.abs(got - want) / 4e-45)).max() <= 4.0
    pi, hp, qp = np.float32(np.pi), np.float32(np.pi / 2), np.float32(np.pi / 4)
    inf = np.float32(np.inf)
    cases = [((0.0, 0.0), 0.0), ((-0.0, 0.0), -0.0), ((0.0, -0.0), pi), ((-0.0, -0.0), -pi),
             ((0.0, -1.0), pi), ((-0.0, -1.0), -pi), ((0.0, 1.0), 0.0), ((-0.0, 1.0), -0.0),
             ((1.0, 0.0), hp), ((1.0, -0.0), hp), ((-1.0, 0.0), -hp), ((-1.0, -0.0), -hp),
             ((1.0, inf), 0.0), ((-1.0, inf), -0.0), ((1.0, -inf), pi), ((-1.0, -inf), -pi),
             ((inf, 1.0), hp), ((-inf, -1.0), -hp), ((inf, inf), qp), ((-inf, inf), -qp),
             ((inf, -inf), np.float32(3 * np.pi / 4)), ((-inf, -inf), np.float32(-3 * np.pi / 4))]
    ys = np.array([c[0][0] for c in cases], np.float32)
    xs = np.array([c[0][1] for c in cases], np.float32)
    got = atan2_batch(ys, xs)
    for (yx, w), g in zip(cases, got):
        assert g == np.float32(w) and np.signbit(g) == np.signbit(np.float32(w)), (yx, g, w)
        assert g == np.float32(np.arctan2(np.float64(yx[0]), np.float64(yx[1]))), yx
    assert np.isnan(atan2_batch(np.array([np.nan, 1], np.float32), np.array([1, np.nan], np.float32))).all()
