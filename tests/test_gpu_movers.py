"""Kind-3 bounded movers on the GPU (world.hpp:26-41) and the moving-threat
mix: the 8,192 x 256 workload with four movers per world, the env % 4
static / long / course lanes and 100 ms sensor and command delays.

- the reference's motion known answer (navigation_motion_check.mm:19-31)
  through the device ray cast and clearance;
- kind-3 depth and clearance of the mix worlds and of guard cases either
  side of the 1e-8 guards, bit-identical to the oracle;
- a rollout and PPO update of the mix at 2,048 envs (every wavefront mixes
  lanes, so box-only and mover worlds meet in one wavefront), through
  resets, every buffer at tolerance 0.
"""
import sys

import numpy as np
import pytest

from gpu_compare import ENV_BUFFERS, ROW_BUFFERS, compare, config, make_pair
from mdnav import abi, ops
from oracle_lib import oracle, ptr
from test_oracle_movers import COURSE, LONG, MIX, MOVERS, guard_worlds, one_mover, world

pytestmark = pytest.mark.gpu

F = np.float32


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def test_motion_check_known_answer_gpu():
    say("case: kind-3 motion known answer, 1001 times")
    w = one_mover([6, 0, 1.5], 0.28, 2.7, -1.57079632679, [0, 0.8, 0])
    n = 1001
    times = (np.arange(n) * F(0.02)).astype(F)
    pts = np.zeros((n, 3), F)
    for i, t in enumerate(times):
        c = np.zeros(3, F)
        oracle().orc_obstacle_center(ptr(w), 0, F(t), ptr(c))
        pts[i] = [c[0] + F(0.28) + F(0.18) + F(1), c[1], c[2]]
    worlds = np.repeat(w, n)
    clr = ops.clearance(worlds, pts, times)
    rays = np.concatenate([pts, np.tile(np.array([-1, 0, 0], F), (n, 1))], axis=1)
    depth = ops.ray_world(worlds, rays, times, 1)
    assert np.abs(clr - 1).max() < 1e-5, np.abs(clr - 1).max()
    assert np.abs(depth - F(1.18)).max() < 1e-5, np.abs(depth - F(1.18)).max()
    want_c, want_d = np.zeros(n, F), np.zeros(n, F)
    oracle().orc_clearance_batch(ptr(worlds), ptr(pts), ptr(times), ptr(want_c), n)
    oracle().orc_ray_world_batch(ptr(worlds), ptr(np.ascontiguousarray(rays)), ptr(times), 1, ptr(want_d), n)
    assert np.array_equal(clr, want_c) and np.array_equal(depth, want_d)


def test_kind3_depth_and_clearance_bit_exact():
    say("case: kind-3 worlds (mix families + guards) x 320 rays x 4 times")
    ws = [world(f, s, d) for f in (MOVERS, LONG, COURSE) for s, d in ((7, 4.0), (91, 8.0), (2024, 6.0))]
    ws += guard_worlds()
    times_each = [0.37, 1.1, 5.3, 19.9]
    worlds = np.array([w for w in ws for _ in times_each], abi.WORLD)
    times = np.array([t for _ in ws for t in times_each], F)
    n = len(worlds)
    cam = np.zeros((320, 3), F)
    oracle().orc_camera_rays(ptr(cam))
    rays = np.zeros((n, 320, 6), F)
    for i in range(n):
        rays[i, :, 0:3] = [0.5 + 0.4 * (i % 7), 0.3 * (i % 5 - 2), 1.4 + 0.1 * (i % 3)]
        rays[i, :, 3:6] = cam
    got = ops.ray_world(worlds, rays, times, 320)
    want = np.zeros(n * 320, F)
    oracle().orc_ray_world_batch(ptr(worlds), ptr(rays), ptr(times), 320, ptr(want), n * 320)
    assert np.array_equal(got, want), np.abs(got - want).max()
    assert (got < 12).mean() > 0.5
    pts = np.ascontiguousarray(rays[:, 0, 0:3])
    c = ops.clearance(worlds, pts, times)
    cw = np.zeros(n, F)
    oracle().orc_clearance_batch(ptr(worlds), ptr(pts), ptr(times), ptr(cw), n)
    assert np.array_equal(c, cw), np.abs(c - cw).max()


@pytest.mark.parametrize("n,T,max_steps", [(2048, 24, 9), (96, 40, 30)])
def test_threat_mix_rollout_update_bit_exact(n, T, max_steps):
    """The moving-threat mix (family 32: lanes 0-1 mover worlds, lane 2 long
    goals, lane 3 courses) with 100 ms sensor and command delays (2 ticks),
    rollout + GAE + one epoch of four minibatches: every buffer, float
    fields included, equal to the oracle's."""
    say("case: threat mix N=%d T=%d max_steps=%d delays 2/2, rollout + update" % (n, T, max_steps))
    cfg = config(n=n, family=MIX, speed=1.5, distance=4.0, sensor_delay=2, command_delay=2, max_steps=max_steps)
    rows = n * T
    mb = 1 << max(8, int(np.ceil(np.log2(rows / 4))))
    sim, ppo, ora = make_pair(cfg, T, epochs=1, minibatch=mb)
    try:
        sim.collect()
        ppo.rollout_update(0)
        sim.sync()
        ora.iteration(0)
        bad = compare(sim, ora, ["advantages", "returns", "actor", "critic", "actor_m", "actor_v", "critic_m",
                                 "critic_v", "metric_rows"] + ENV_BUFFERS + ROW_BUFFERS, tol=0.0)
        assert not bad, bad
        runs = ora.get("runs")
        fams = ora.get("worlds")["family"]
        assert set(fams.tolist()) == {MOVERS, LONG, COURSE}
        assert runs["episodes"].sum() >= n  # every env was reset at least once inside the rollout
        say("  episodes %d, collisions %d, successes %d" % (runs["episodes"].sum(), runs["collisions"].sum(),
                                                            runs["successes"].sum()))
    finally:
        ppo.close()
        sim.close()


def test_small_radius_worlds_take_the_lane_cast():
    """Spheres below the strip cast's 0.05 m radius bound (its culling proof
    needs it) send their wavefronts to the per-lane cast: family-3 worlds
    whose spheres shrink to 0.03 m in every other env, 256 envs x 12 ticks,
    every buffer equal to the oracle's."""
    say("case: small-radius spheres, N=256 T=12")
    cfg = config(n=256, family=3, speed=1.0, distance=4.0, max_steps=200)
    sim, _, ora = make_pair(cfg, 12)
    w = ora.get("worlds")
    w["obstacles"]["size"][0::2, :, 0] = np.float32(0.03)
    for side in (sim, ora):
        side.set("worlds", w)
    sim.collect()
    sim.sync()
    ora.collect()
    bad = compare(sim, ora, ENV_BUFFERS + ROW_BUFFERS, tol=0.0)
    assert not bad, bad
