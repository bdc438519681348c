"""Pins for the oracle's restatements of the reference's Metal-only pieces.

- guided evaluation modes (sim.metal:233): the mode-12 scale from the
  nearest pooled range, and mode 16's yaw term
  atanh(clamp(1.5 atan2(y, x), -0.85, 0.85)) from the context's goal
  direction, on hand-placed observation rows; modes 13 and 17 beside them;
- the challenge-bank rehearsal slot (sim.metal:103-110): the env's family
  alternates 12 / 13 by env parity through the reference's own
  wtraining_family, and its world is the reference's wgenerate at 4 m, both
  compiled from world.hpp with clang++ (oracle/_ref).
"""
import math

import numpy as np
import pytest

from mdnav import abi
from oracle_lib import OracleTrainer, oracle, ptr, raptor_fixture, ref, ref_available

needs_ref = pytest.mark.skipif(not ref_available("clang"), reason="oracle/_ref not built (needs the reference tree)")

F = np.float32
PRIOR = np.array([0.3, -0.2, 0.1], F)
MEAN = np.array([0.9, 0.4, -0.5, 0.6], F)


def row(near=None, goal=(1.0, 0.0), far_top=None):
    """A 184-input row: 80 current pooled ranges (/12) of 12 m except one cell
    at `near` m, previous ranges of 12 m, the context's goal direction in
    body axes at inputs 160-161, `far_top` of the top two grid rows' cells
    beyond 2.5 m (the rest at 2 m), and the hint at 181-183."""
    o = np.zeros(184, F)
    o[:160] = 1.0
    if far_top is not None:
        o[:20] = F(2.0 / 12)
        o[:far_top] = 1.0
    if near is not None:
        o[45] = F(near) / F(12)
    o[160], o[161] = goal
    o[181:184] = PRIOR
    return o


def means(mode, o):
    m = MEAN.copy()
    oracle().orc_guided_mode_means(mode, ptr(np.ascontiguousarray(o)), ptr(m))
    return m


def blended(scale):
    out = np.empty(4, np.float64)
    out[:3] = PRIOR.astype(np.float64) + scale * (MEAN[:3].astype(np.float64) - PRIOR)
    out[3] = scale * float(MEAN[3])
    return out


def test_mode12_scale_from_nearest_range():
    """scale = clamp((nearest - 0.3) / 2, 0.2, 1): nearest range 0.3, 1.3,
    2.3 and 4.3 m give 0.2, 0.5, 1.0 and 1.0."""
    for near, scale in ((0.3, 0.2), (1.3, 0.5), (2.3, 1.0), (4.3, 1.0), (0.05, 0.2), (1.7, 0.7)):
        got = means(12, row(near=near))
        assert np.abs(got - blended(scale)).max() < 1e-6, (near, got, blended(scale))


def test_mode16_yaw_term():
    """Mode 16: scale 0.25, and the yaw rate gains
    atanh(clamp(1.5 atan2(goal_y, goal_x), -0.85, 0.85))."""
    cases = [((1.0, 0.0), 0.0), ((0.98, 0.2), math.atanh(1.5 * math.atan2(0.2, 0.98))),
             ((0.95, -0.1), math.atanh(1.5 * math.atan2(-0.1, 0.95))), ((0.8, 0.6), math.atanh(0.85)),
             ((0.6, -0.8), -math.atanh(0.85)), ((-1.0, 0.0), math.atanh(0.85)), ((-1.0, -0.0), -math.atanh(0.85)),
             ((0.0, 1.0), math.atanh(0.85)), ((0.99, 0.05), math.atanh(1.5 * math.atan2(0.05, 0.99)))]
    for goal, term in cases:
        got = means(16, row(goal=goal))
        want = blended(0.25)
        want[3] += term
        assert np.abs(got - want).max() < 2e-6, (goal, got, want)
    # the term depends on the direction only through atan2(y, x): swapping
    # the operands changes it
    a, b = means(16, row(goal=(0.9, 0.3))), means(16, row(goal=(0.3, 0.9)))
    assert abs(float(a[3] - b[3])) > 0.5


def test_modes13_and_17():
    """Mode 13 keeps the hint (scale 0); mode 17 scales by
    0.25 + 0.75 (cells of the top two rows beyond 2.5 m) / 20."""
    assert np.abs(means(13, row(near=3.0)) - blended(0.0)).max() < 1e-7
    for far in (0, 5, 12, 20):
        got = means(17, row(far_top=far))
        assert np.abs(got - blended(0.25 + 0.75 * far / 20)).max() < 1e-6, far


@needs_ref
@pytest.mark.parametrize("family,wind", [(1, 0.5), (13, 0.5), (12, 0.0)])
def test_bank_rehearsal_slot_against_reference(family, wind):
    """Every env's schedule slot is the rehearsal level: after its reset the
    env's stream draws the rehearsal family with the reference's
    wtraining_family(env % 2 == 0 ? 12 : 13) and its world with the
    reference's wgenerate(seed, family, 4.0) (sim.metal:103-110); the wind,
    the stream word, the initial distance and the active level follow
    sim.metal:113-121."""
    n = 32
    cfg = abi.default_config(n=n, family=family, speed=1.5, distance=6.0, wind=wind)
    ora = OracleTrainer(cfg, 4, raptor_fixture()[0])
    dummy = np.zeros(1, abi.WORLD)
    ora.set_bank(dummy, np.full((n, 3), abi.BANK_REHEARSAL, np.uint32))
    ora.reset()
    worlds, runs = ora.get("worlds"), ora.get("runs")
    # clang++ build: family 6 passes three draws in one argument list, which
    # clang (like the reference's Metal compiler) evaluates left to right
    R = ref("clang")
    U32 = np.uint32
    for e in range(n):
        rng = np.array([(int(cfg["seed"]) + e * 747796405 + 2891336453) & 0xFFFFFFFF], U32)
        rp = rng.ctypes.data_as(__import__("ctypes").POINTER(__import__("ctypes").c_uint32))
        R.ref_training_family(family, rp)  # the reset's own draws
        R.ref_xorshift(rp)
        fam = R.ref_training_family(12 if e % 2 == 0 else 13, rp)
        seed = R.ref_xorshift(rp)
        want = np.zeros((), abi.WORLD)
        R.ref_generate_world(ptr(want), seed, fam, F(4.0))
        got = worlds[e].copy()
        clean = family in (12, 13) and e % 2 == 0
        assert float(got["wind"][0]) == (0.0 if clean else F(wind)) and got["wind"][1] == 0 and got["wind"][2] == 0
        got["wind"] = want["wind"]
        # wgenerate leaves the slots past the new count as they were: compare
        # the live obstacles and the header
        c = int(want["count"])
        assert got["obstacles"][:c].tobytes() == want["obstacles"][:c].tobytes(), (e, fam)
        for k in ("count", "seed", "family", "goal", "wind"):
            assert np.array_equal(got[k], want[k]), (e, k)
        assert int(runs[e]["rng"]) == int(rng[0])
        g = want["goal"].astype(F)
        dist = np.sqrt(F(g[0] * g[0] + g[1] * g[1]) + F((g[2] - F(1.5)) * (g[2] - F(1.5))))
        assert abs(float(runs[e]["initial_distance"]) - float(dist)) < 1e-6
    assert set(ora.get("bank_active_ids").tolist()) == {abi.BANK_REHEARSAL}
    fams = worlds["family"]
    assert {4, 5}.issubset(set(fams[0::2].tolist()))  # family 12's rehearsal mixture on even envs
    assert set(fams[1::2].tolist()) & {10, 11}  # threat spheres among family 13's
