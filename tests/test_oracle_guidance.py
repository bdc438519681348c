"""Geometry-prior guidance (guidance.hpp): the oracle's restatement against the
reference's own header compiled into oracle/_ref, plus closed-form cases.

The oracle and the reference share every operation except the final atanh,
which the oracle takes from this project's log_f and the reference from
std::log, so hints agree to a few float ulps and the discrete choices (best
cell, goal cell, direct path) agree exactly.  The memory clearance has no
transcendental and must agree bit for bit."""
import math

import numpy as np
import pytest

from oracle_lib import oracle, ptr, ref, ref_available

needs_ref = pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (needs the reference tree)")
F = np.float32
HINT_TOL = 2e-6   # atanh(x) through two different logs, |x| <= 0.8


def scene(rng, kind):
    """Pooled current/previous ranges, goal direction, distance, velocity, sensor dt."""
    cur = np.full(80, 12.0, F)
    if kind >= 1:
        cur = rng.uniform(0.2, 12.0, 80).astype(F)
        cur[rng.random(80) < 0.4] = 12.0
    if kind >= 2:  # a near wall over a block of cells
        r0, c0 = rng.integers(0, 6), rng.integers(0, 8)
        cur.reshape(8, 10)[r0:r0 + 3, c0:c0 + 3] = rng.uniform(0.2, 1.5)
    prev = (cur + rng.normal(0, 0.05, 80)).astype(F)
    prev[rng.random(80) < 0.2] += F(0.3)          # closing obstacles: temporal risk
    prev = np.clip(prev, 0, 12).astype(F)
    g = rng.normal(0, 1, 3)
    if kind % 2 == 0:
        g[0] = abs(g[0]) + 0.5
    goal = (g / np.linalg.norm(g)).astype(F)
    dist = F(rng.choice([0.01, 0.3, 1.0, 3.0, 8.0]) * rng.uniform(0.5, 1.5))
    vel = rng.normal(0, 0.8, 3).astype(F)
    dt = F(rng.choice([0.05, 0.05, 0.1, 0.0]))
    return cur, prev, goal, dist, vel, dt


def hint(lib, prefix, cur, prev, goal, dist, vel, dt):
    out = np.zeros(3, F)
    getattr(lib, prefix + "_guidance")(ptr(cur), ptr(prev), ptr(goal), F(dist), ptr(vel), F(dt), ptr(out))
    return out


@needs_ref
def test_guidance_matches_reference():
    rng = np.random.default_rng(7)
    worst = 0.0
    for i in range(600):
        args = scene(rng, i % 3)
        a, b = hint(oracle(), "orc", *args), hint(ref(), "ref", *args)
        worst = max(worst, float(np.abs(a.astype(np.float64) - b).max()))
    assert worst <= HINT_TOL, worst


def rings(rng, frames=8):
    ranges = rng.uniform(0.3, 12.0, (frames, 320)).astype(F)
    ranges[rng.random((frames, 320)) < 0.3] = 12.0
    poses = np.zeros((frames, 12), F)
    for f in range(frames):
        yaw = rng.uniform(-0.3, 0.3)
        poses[f, 0:3] = rng.normal(0, 0.3, 3) + [0, 0, 1.5]
        poses[f, 3:12] = [math.cos(yaw), -math.sin(yaw), 0, math.sin(yaw), math.cos(yaw), 0, 0, 0, 1]
    pose = np.array([0.05, -0.02, 1.5, 1, 0, 0, 0, 1, 0, 0, 0, 1], F)
    return ranges, poses, pose


@needs_ref
def test_memory_clearance_matches_reference_exactly():
    rng = np.random.default_rng(11)
    for i in range(200):
        ranges, poses, pose = rings(rng)
        d = rng.normal(0, 1, 3)
        d = (d / np.linalg.norm(d)).astype(F)
        latest, valid = int(rng.integers(0, 20)), int(rng.integers(0, 9))
        a, b = np.zeros(1, F), np.zeros(1, F)
        for lib, pre, out in ((oracle(), "orc", a), (ref(), "ref", b)):
            getattr(lib, pre + "_memory_clearance")(ptr(d), ptr(ranges), ptr(poses), ptr(pose), latest, valid,
                                                    F(0.05), ptr(out))
        assert a.tobytes() == b.tobytes(), (i, a, b)


@needs_ref
def test_guidance_memory_matches_reference():
    rng = np.random.default_rng(13)
    worst = 0.0
    for i in range(60):
        cur, prev, goal, dist, vel, dt = scene(rng, i % 3)
        ranges, poses, pose = rings(rng)
        latest, valid = int(rng.integers(0, 20)), int(rng.integers(0, 9))
        out = []
        for lib, pre in ((oracle(), "orc"), (ref(), "ref")):
            h = np.zeros(3, F)
            getattr(lib, pre + "_guidance_memory")(ptr(cur), ptr(prev), ptr(goal), F(dist), ptr(vel), F(dt),
                                                   ptr(ranges), ptr(poses), ptr(pose), latest, valid, ptr(h))
            out.append(h)
        worst = max(worst, float(np.abs(out[0].astype(np.float64) - out[1]).max()))
    assert worst <= HINT_TOL, worst


def test_guidance_closed_forms():
    lib = oracle()
    clear = np.full(80, 12.0, F)
    zero = np.zeros(3, F)
    # goal reached: no hint (guidance.hpp:47)
    assert not hint(lib, "orc", clear, clear, np.array([1, 0, 0], F), 0.04, zero, 0.05).any()
    # open space, goal straight ahead 5 m, at rest: desired speed 1.6, fraction 0.8, along the goal
    h = hint(lib, "orc", clear, clear, np.array([1, 0, 0], F), 5.0, zero, 0.05)
    assert h[1] == 0 and h[2] == 0 and abs(h[0] - math.atanh(0.8)) < 2e-7, h
    # 1 m to go: desired speed sqrt(4 * 0.72), fraction half of it
    h = hint(lib, "orc", clear, clear, np.array([1, 0, 0], F), 1.0, zero, 0.05)
    frac = min(0.8, math.sqrt(4 * 0.72) * 0.5)
    assert abs(h[0] - math.atanh(frac)) < 1e-6, (h, frac)
    # a wall 0.5 m away everywhere: no direct path (0.5 < 0.28 + 0.25 * 1.6^2),
    # so the best cell leads; the four cells nearest the axis tie on alignment
    # and the first in row-major order (row 3, col 4) wins; 0.07 m is left after
    # the stop margin, giving speed sqrt(4 * 0.07)
    wall = np.full(80, 0.5, F)
    h = hint(lib, "orc", wall, wall, np.array([1, 0, 0], F), 5.0, zero, 0.05)
    frac = min(0.8, math.sqrt(4 * (0.5 - 0.28 - 0.15)) * 0.5)
    y, z = 0.9 - 0.2 * 4, (0.875 - 0.25 * 3) * 0.75
    d = np.array([1.0, y, z]) / math.sqrt(1 + y * y + z * z)
    want = [math.atanh(frac * v) for v in d]
    assert np.abs(h - want).max() < 1e-6, (h, want)


@needs_ref
@pytest.mark.parametrize("kw", [dict(), dict(sensor_period=2, sensor_delay=1, family=13, speed=1.5)])
def test_rollout_rows_carry_reference_hint(kw):
    """Wiring of the hint into a 184-input observation row (sim.metal:226):
    the last three inputs of every row equal the reference's guidance applied
    to that row's own inputs: ranges (first 80 inputs x 12), previous ranges
    (next 80 x 12), goal direction (context 0-2), velocity (context 4-6 x 4),
    sensor period x dt x substeps, and the goal distance (context 3 x 10, the
    distance/10 the row stores, so the comparison has a tolerance)."""
    from oracle_lib import OracleTrainer, crazyflie, raptor_fixture
    from mdnav import abi
    cfg = abi.default_config(n=32, family=kw.get("family", 1), speed=kw.get("speed", 1.0), distance=3.0,
                             max_steps=30, **{k: v for k, v in kw.items() if k not in ("family", "speed")})
    t = OracleTrainer(cfg, 24, raptor_fixture()[0])
    t.set_actor_obs(184)
    t.collect()
    rows = t.get("obs").reshape(-1, 184)
    p = crazyflie()
    sensor_dt = F(cfg["sensor_period"]) * F(p["dt"]) * F(cfg["substeps"])
    checked = 0
    for r in rows:
        c = r[160:181]
        if c[3] >= 1.4:  # distance clipped at 15 m: not recoverable
            continue
        cur, prev = (r[:80] * F(12)).astype(F), (r[80:160] * F(12)).astype(F)
        goal = c[0:3].copy()
        vel = (c[4:7] * F(4)).astype(F)
        want = hint(ref(), "ref", cur, prev, goal, F(c[3] * F(10)), vel, sensor_dt)
        assert np.abs(want - r[181:]).max() < 1e-4, (want, r[181:])
        checked += 1
    assert checked > len(rows) // 2 and np.count_nonzero(rows[:, 181:]) > 0
