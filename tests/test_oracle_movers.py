"""Kind-3 bounded movers (world.hpp:26-41) and the moving-threat mix worlds.

- the reference's own motion known answer (navigation_motion_check.mm:19-31):
  a sphere of radius 0.28 m at (6, 0, 1.5) with amplitude 2.7 m, phase
  -pi/2 and velocity (0, 0.8, 0), sampled at t = 0.02 i for i < 1001; from a
  point 0.28 + 0.18 + 1 m beyond its centre the clearance is 1 m and the
  depth looking back at it 1.18 m, within 1e-5;
- the bounds the motion law fixes: the centre stays within the amplitude of
  its rest point along the velocity direction, its speed never exceeds |v|,
  it reaches +-A at the phases pi/2 and -pi/2, and the 1e-8 guards freeze it;
- the oracle's centre, ray cast and clearance against the reference's wc,
  wray and wclearance compiled from world.hpp (oracle/_ref), at times t != 0,
  on the mix worlds and on guard cases either side of 1e-8;
- the mix generator's contract (families 33-35 and the lane rule of 32).
"""
import math

import numpy as np
import pytest

from mdnav import abi
from oracle_lib import OracleTrainer, oracle, ptr, raptor_fixture, ref, ref_available

needs_ref = pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (needs the reference tree)")

F = np.float32
MOVERS, LONG, COURSE, MIX = abi.FAMILY_MOVERS, abi.FAMILY_MOVERS_LONG, abi.FAMILY_COURSE, abi.FAMILY_C3_MIX


def one_mover(center, radius, amplitude, phase, velocity):
    w = np.zeros((), abi.WORLD)
    w["count"] = 1
    o = w["obstacles"][0]
    o["kind"] = 3
    o["center"] = center
    o["size"] = [radius, amplitude, phase]
    o["velocity"] = velocity
    return w


def centre(lib, fn, w, i, t):
    out = np.zeros(3, F)
    getattr(lib, fn)(ptr(w), i, F(t), ptr(out))
    return out


def world(family, seed, distance=4.0):
    w = np.zeros((), abi.WORLD)
    oracle().orc_generate_world(ptr(w), seed, family, F(distance))
    return w


def test_motion_check_known_answer():
    """navigation_motion_check.mm:19-31, on the oracle."""
    lib = oracle()
    w = one_mover([6, 0, 1.5], 0.28, 2.7, -1.57079632679, [0, 0.8, 0])
    n = 1001
    times = (np.arange(n) * F(0.02)).astype(F)
    pts = np.zeros((n, 3), F)
    rays = np.zeros((n, 6), F)
    for i, t in enumerate(times):
        c = centre(lib, "orc_obstacle_center", w, 0, t)
        pts[i] = [c[0] + F(0.28) + F(0.18) + F(1), c[1], c[2]]
        rays[i] = [*pts[i], -1, 0, 0]
        # x and z stay put; y follows A sin(t |v| / A + phase) within fp32 rounding
        assert c[0] == F(6) and c[2] == F(1.5)
        assert abs(c[1] - 2.7 * math.sin(t * 0.8 / 2.7 - math.pi / 2)) < 2e-6
    worlds = np.repeat(w, n)
    clr = np.zeros(n, F)
    lib.orc_clearance_batch(ptr(worlds), ptr(pts), ptr(times), ptr(clr), n)
    depth = np.zeros(n, F)
    lib.orc_ray_world_batch(ptr(worlds), ptr(rays), ptr(times), 1, ptr(depth), n)
    assert np.abs(clr - 1).max() < 1e-5, np.abs(clr - 1).max()
    assert np.abs(depth - F(1.18)).max() < 1e-5, np.abs(depth - F(1.18)).max()
    # the sphere really travels: its y spans nearly [-2.7, 2.7] over 20 s
    ys = [centre(lib, "orc_obstacle_center", w, 0, t)[1] for t in times]
    assert min(ys) < -2.69 and max(ys) > 2.69


def test_mover_motion_bounds():
    """|c(t) - c0| <= A along v / |v|, speed <= |v|, extremes +-A at phases
    +-pi/2, and the guards: |v| <= 1e-8 or A <= 1e-8 freezes the centre."""
    lib = oracle()
    rng = np.random.default_rng(3)
    for _ in range(40):
        c0 = rng.uniform(-3, 8, 3).astype(F)
        v = rng.uniform(-1, 1, 3).astype(F)
        speed = float(np.linalg.norm(v.astype(np.float64)))
        amp, phase = F(rng.uniform(0.3, 3)), F(rng.uniform(-math.pi, math.pi))
        w = one_mover(c0, 0.3, amp, phase, v)
        ts = np.linspace(0, 12, 601).astype(F)
        cs = np.array([centre(lib, "orc_obstacle_center", w, 0, t) for t in ts], np.float64)
        disp = cs - c0.astype(np.float64)
        # displacement is along v: its cross product with v vanishes
        assert np.abs(np.cross(disp, v.astype(np.float64))).max() < 1e-5
        assert np.linalg.norm(disp, axis=1).max() <= float(amp) * (1 + 1e-5) + 1e-6
        step = np.linalg.norm(np.diff(cs, axis=0), axis=1) / np.diff(ts.astype(np.float64))
        assert step.max() <= speed * (1 + 1e-3) + 1e-5
        # phase pi/2 -> +A v/|v|, phase -pi/2 -> -A v/|v|
        t_hi = (math.pi / 2 - float(phase)) % (2 * math.pi) * float(amp) / speed
        t_lo = (-math.pi / 2 - float(phase)) % (2 * math.pi) * float(amp) / speed
        for t, sgn in ((t_hi, 1), (t_lo, -1)):
            c = centre(lib, "orc_obstacle_center", w, 0, t).astype(np.float64)
            want = c0.astype(np.float64) + sgn * float(amp) * v.astype(np.float64) / speed
            assert np.abs(c - want).max() < 1e-4, (t, c, want)
    for v, amp in (([0, 0, 0], 2.0), ([5e-9, 0, 0], 2.0), ([0.5, 0, 0], 0.0), ([0.5, 0, 0], 5e-9)):
        w = one_mover([1, 2, 3], 0.3, amp, 0.4, v)
        for t in (0.0, 0.7, 13.1):
            assert np.array_equal(centre(lib, "orc_obstacle_center", w, 0, t), np.array([1, 2, 3], F))
    # just above the guards the sphere moves (centred at 0, where a 1e-8 m
    # offset is representable), just below it stays
    w = one_mover([1, 2, 3], 0.3, 2.0, 0.4, [2e-8, 0, 0])
    assert centre(lib, "orc_obstacle_center", w, 0, 100.0)[0] != F(1)
    for amp, moves in ((1.1e-8, True), (9e-9, False)):
        w = one_mover([0, 0, 0], 0.3, amp, 0.4, [0, 0.5, 0])
        ys = [centre(lib, "orc_obstacle_center", w, 0, t)[1] for t in (0.0, 0.3, 1.7)]
        assert any(y != 0 for y in ys) == moves, (amp, ys)


def guard_worlds():
    """Kind-3 obstacles either side of the 1e-8 guards of world.hpp:36, with
    a box and a plain sphere beside them."""
    out = []
    for v, amp in (([0, 0, 0], 1.5), ([5e-9, 5e-9, 0], 1.5), ([1.2e-8, 0, 0], 1.5), ([0, 0.9, 0], 0.0),
                   ([0, 0.9, 0], 9e-9), ([0, 0.9, 0], 1.1e-8), ([0.6, -0.8, 0.2], 2.2), ([0, 1.49, 0], 0.6)):
        w = one_mover([4.0, 0.3, 1.6], 0.45, amp, 0.7, v)
        w["count"] = 3
        b = w["obstacles"][1]
        b["kind"] = 0
        b["center"] = [6.0, -1.0, 1.0]
        b["size"] = [0.5, 0.4, 0.9]
        s = w["obstacles"][2]
        s["kind"] = 1
        s["center"] = [5.0, 1.5, 2.0]
        s["size"] = [0.35, 0.35, 0.35]
        s["velocity"] = [0, -0.3, 0]
        out.append(w)
    return out


@needs_ref
def test_kind3_against_reference():
    """Centres, depth and clearance of kind-3 worlds at t != 0 against the
    reference's wc / wray / wclearance.  The oracle's sin differs from
    std::sin by an ulp or so (world.hpp calls the platform's), so the
    centres agree to 2e-6 m and depths and clearances to the reference's own
    CPU/Metal gate of 3e-5 (world_tests, main.mm:107-125)."""
    worlds = [world(f, s, d) for f in (MOVERS, LONG, COURSE) for s, d in ((7, 4.0), (91, 8.0), (2024, 6.0))]
    worlds += guard_worlds()
    times = [0.37, 1.1, 5.3, 19.9]
    cam = np.zeros((320, 3), F)
    oracle().orc_camera_rays(ptr(cam))
    worst_c = worst_d = worst_k = 0.0
    for w in worlds:
        kinds = w["obstacles"]["kind"][:w["count"]]
        assert 3 in kinds
        for t in times:
            for i in range(int(w["count"])):
                a = centre(oracle(), "orc_obstacle_center", w, i, t)
                b = centre(ref(), "ref_obstacle_center", w, i, t)
                worst_c = max(worst_c, float(np.abs(a - b).max()))
            # 320 camera rays from three origins along the route
            n = 3 * 320
            rays = np.zeros((n, 6), F)
            for k, org in enumerate(([0, 0, 1.5], [2.5, 0.4, 1.4], [5.0, -0.5, 1.8])):
                rays[k * 320:(k + 1) * 320, 0:3] = org
                rays[k * 320:(k + 1) * 320, 3:6] = cam
            ws = np.repeat(w, 1)
            tt = np.array([t], F)
            da, db = np.zeros(n, F), np.zeros(n, F)
            oracle().orc_ray_world_batch(ptr(ws), ptr(rays), ptr(tt), n, ptr(da), n)
            ref().ref_ray_world_batch(ptr(ws), ptr(rays), ptr(tt), n, ptr(db), n)
            worst_d = max(worst_d, float(np.abs(da - db).max()))
            pts = np.array([[x, y, z] for x in (0.5, 3.0, 5.5) for y in (-1.0, 0.3) for z in (1.2, 1.9)], F)
            m = len(pts)
            wm = np.repeat(w, m)
            tm = np.full(m, t, F)
            ka, kb = np.zeros(m, F), np.zeros(m, F)
            oracle().orc_clearance_batch(ptr(wm), ptr(pts), ptr(tm), ptr(ka), m)
            ref().ref_clearance_batch(ptr(wm), ptr(pts), ptr(tm), ptr(kb), m)
            worst_k = max(worst_k, float(np.abs(ka - kb).max()))
    assert worst_c < 2e-6, worst_c
    assert worst_d < 3e-5, worst_d
    assert worst_k < 3e-5, worst_k


def test_mover_world_contract():
    """Families 33/34: family 1's eight boxes, then four kind-3 movers with
    radius [0.2, 0.5] m, peak speed [0.3, 1.5] m/s on a horizontal heading,
    amplitude [0.5, 2] m and phase [-pi, pi); 34 puts the goal 8-13 m out."""
    for family in (MOVERS, LONG):
        for seed in range(1, 400, 7):
            w = world(family, seed, 4.0)
            assert int(w["count"]) == 12 and int(w["family"]) == family
            o = w["obstacles"]
            assert list(o["kind"][:12]) == [0] * 8 + [3] * 4
            m = o[8:12]
            assert np.all((m["size"][:, 0] >= 0.2) & (m["size"][:, 0] <= 0.5))
            assert np.all((m["size"][:, 1] >= 0.5) & (m["size"][:, 1] <= 2.0))
            assert np.all(np.abs(m["size"][:, 2]) <= np.float32(math.pi))
            speed = np.linalg.norm(m["velocity"].astype(np.float64), axis=1)
            assert np.all((speed >= 0.3 - 1e-6) & (speed <= 1.5 + 1e-6)), speed
            assert np.all(m["velocity"][:, 2] == 0)
            goal = float(w["goal"][0])
            if family == MOVERS:
                assert goal == 4.0
            else:
                assert 8.0 <= goal <= 13.0
            assert np.all((m["center"][:, 0] >= 1.5) & (m["center"][:, 0] <= 1.5 + max(0.5, goal - 2.5) + 1e-5))
    # the box part draws exactly as family 1 does (world.hpp:311-317)
    for seed in (5, 77, 123456):
        a, b = world(MOVERS, seed, 6.0), world(1, seed, 6.0)
        assert a["obstacles"][:8].tobytes() == b["obstacles"][:8].tobytes()
        assert a["goal"].tobytes() == b["goal"].tobytes()


def test_course_contract():
    """Family 35, the combined course (navigation_challenge_tasks.py:47-117):
    corridor walls at y = +-1.66 with the side opening at 0.59 L, two
    openings at 0.32 L and 0.68 L on opposite sides, the hanging beam at
    0.5 L, and one kind-3 sphere of radius 0.28 crossing at 0.59 L."""
    for seed in range(1, 300, 11):
        w = world(COURSE, seed)
        o = w["obstacles"]
        assert int(w["count"]) == 10 and int(w["family"]) == COURSE
        assert list(o["kind"][:10]) == [0] * 9 + [3]
        L = float(w["goal"][0])
        assert 8.5 <= L <= 11.5 and abs(float(w["goal"][1])) <= 0.2 and float(w["goal"][2]) == 1.5
        walls = o[:4]
        assert np.allclose(np.abs(walls["center"][:, 1]), 1.66)
        # the corridor walls leave exactly the 1.4 m side opening around 0.59 L
        ends = sorted((float(c[0] - e[0]), float(c[0] + e[0])) for c, e in zip(walls["center"], walls["size"]))
        assert abs(ends[0][0] + 2) < 1e-5 and abs(ends[-1][1] - 14) < 1e-5
        assert abs(ends[1][1] - (0.59 * L - 0.7)) < 1e-4 and abs(ends[2][0] - (0.59 * L + 0.7)) < 1e-4
        # each opening's two panels span the corridor, leaving one gap
        for k, frac in ((4, 0.32), (6, 0.68)):
            p = o[k:k + 2]
            assert np.allclose(p["center"][:, 0], frac * L, atol=1e-5)
            lo = p["center"][0][1] + p["size"][0][1]
            hi = p["center"][1][1] - p["size"][1][1]
            gap = hi - lo
            assert 0.85 - 1e-5 <= gap <= 1.55 + 1e-5
            assert abs((p["center"][0][1] - p["size"][0][1]) + 1.6) < 1e-5
            assert abs((p["center"][1][1] + p["size"][1][1]) - 1.6) < 1e-5
        gap_mid = [(o[k]["center"][1] + o[k]["size"][1] + o[k + 1]["center"][1] - o[k + 1]["size"][1]) / 2
                   for k in (4, 6)]
        assert gap_mid[0] * gap_mid[1] < 0  # staggered to opposite sides
        beam = o[8]
        assert abs(beam["center"][0] - 0.5 * L) < 1e-5 and beam["center"][2] == np.float32(3.35)
        s = o[9]
        assert abs(s["center"][0] - 0.59 * L) < 1e-5 and s["size"][0] == np.float32(0.28)
        assert 2.2 <= s["size"][1] <= 3.4 and abs(s["size"][2] + math.pi / 2) <= 0.25 + 1e-6
        assert s["velocity"][0] == 0 and s["velocity"][2] == 0 and 0.35 <= abs(s["velocity"][1]) <= 1.0


def test_mix_lanes():
    """Family 32 takes the world family from the env's lane n % 4:
    lanes 0, 1 -> 33, lane 2 -> 34, lane 3 -> 35 (50/25/25)."""
    cfg = abi.default_config(n=64, family=MIX, speed=1.5, distance=4.0, sensor_delay=2, command_delay=2)
    ora = OracleTrainer(cfg, 4, raptor_fixture()[0])
    fam = ora.get("worlds")["family"]
    want = [MOVERS if n % 4 < 2 else (LONG if n % 4 == 2 else COURSE) for n in range(64)]
    assert list(fam) == want
    # the worlds are those of their families' generator, seeded from the env's stream
    counts = ora.get("worlds")["count"]
    assert set(counts[np.array(want) == COURSE]) == {10} and set(counts[np.array(want) != COURSE]) == {12}
