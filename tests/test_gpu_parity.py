"""HIP path against the CPU oracle and the reference's golden vectors.

Integer outcomes (flags, counters, RNG states, world seeds/families) must
match exactly.  Floating-point fields carry the stated tolerances; the
arithmetic is designed to round identically on both sides, and the observed
error is reported in each assertion message.
"""
import sys

import numpy as np
import pytest

from gpu_compare import ENV_BUFFERS, ROW_BUFFERS, compare, config, make_pair
from mdnav import PPOTrainer, Sim, abi, ops
from oracle_lib import OracleTrainer, crazyflie, oracle, physics_fixture, ptr, raptor_fixture

pytestmark = pytest.mark.gpu

TOL = 1e-5  # absolute, fp32 fields (reference gates: 2e-5 physics/RAPTOR, 3e-5 depth)


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def flat_state(s):
    return np.ascontiguousarray(s).view(np.float32).reshape(len(s), 17)


def test_physics_golden():
    say("case: physics golden 64x8")
    params, recs, _, _ = physics_fixture()
    out = ops.physics_step(recs["state"], recs["action"], recs["wind"], params)
    err = np.abs(flat_state(out) - flat_state(recs["next"])).max()
    assert err < 2e-5, err
    ora = np.zeros(len(recs), abi.PHYSICS_STATE)
    p = np.array(params, abi.PHYSICS_PARAMS)
    s, a, w = (np.ascontiguousarray(recs[k]) for k in ("state", "action", "wind"))
    oracle().orc_physics_step_batch(ptr(s), ptr(a), ptr(w), ptr(p), ptr(ora), len(recs))
    assert out.tobytes() == ora.tobytes(), np.abs(flat_state(out) - flat_state(ora)).max()


def test_constant_division_exhaustive():
    """The kernels divide by constants as (float)((double)x * RN64(1/b)).  Over
    all 2^32 numerators (signed zeros, subnormals, infinities, NaN) this must
    equal the correctly rounded fp32 x / b for every divisor they use: the
    plant's mass and rotor time constants (default and golden-fixture
    parameters), the RK4 weight 6, the observation scales and the guidance
    hint's sensor period (period x dt x substeps for periods 1-4)."""
    say("case: exhaustive fp64-reciprocal division, all 2^32 numerators")
    from mdnav import native
    divs = [6.0, 12.0, 10.0, 5.0, 200.0]
    for p in (crazyflie(), physics_fixture()[0]):
        divs += [float(p["mass"])] + [float(v) for v in p["rotor_time_constants_rising"]] + \
                [float(v) for v in p["rotor_time_constants_falling"]]
        for period in range(1, 5):
            dt = np.float32(period) * np.float32(p["dt"]) * np.float32(5)
            divs.append(float(max(dt, np.float32(1e-3))))
    d = np.unique(np.array(divs, np.float32))
    out = np.zeros(len(d), np.uint64)
    assert native.lib().mdn_op_check_division(ptr(d), len(d), ptr(out)) == 0
    assert not out.any(), dict(zip(d.tolist(), out.tolist()))


def test_raptor_golden_all_lane_widths():
    say("case: RAPTOR official sequence, 48 copies over lane widths 4/8/16")
    weights, obs, expected = raptor_fixture()
    actions, hidden = ops.raptor_sequence(weights, obs, copies=48)
    err = np.abs(actions - expected[None]).max()
    assert err < 2e-5, err
    ref_a = np.zeros((16, 4), np.float32)
    ref_h = np.zeros(16, np.float32)
    w = np.array(weights, abi.RAPTOR_WEIGHTS)
    oracle().orc_raptor_sequence(ptr(w), ptr(obs), 16, ptr(ref_a), ptr(ref_h))
    assert np.array_equal(actions, np.broadcast_to(ref_a, actions.shape)), np.abs(actions - ref_a).max()
    assert np.array_equal(hidden, np.broadcast_to(ref_h, hidden.shape))


def test_ray_cast_and_clearance():
    say("case: world_tests setup, 128 worlds x 320 rays")
    n = 128
    worlds = np.zeros(n, abi.WORLD)
    for i in range(n):
        oracle().orc_generate_world(ptr(worlds[i:i + 1]), i + 197, i % 4, np.float32(8.0))
    times = np.array([(i % 7) * 0.1 for i in range(n)], np.float32)
    cam = np.zeros((320, 3), np.float32)
    oracle().orc_camera_rays(ptr(cam))
    rays = np.zeros((n, 320, 6), np.float32)
    for i in range(n):
        rays[i, :, 0:3] = [0, (i % 5 - 2) * 0.3, 1.5]
        rays[i, :, 3:6] = cam
    got = ops.ray_world(worlds, rays, times, 320)
    want = np.zeros(n * 320, np.float32)
    oracle().orc_ray_world_batch(ptr(worlds), ptr(rays), ptr(times), 320, ptr(want), n * 320)
    assert np.array_equal(got, want), np.abs(got - want).max()
    pts = np.ascontiguousarray(rays[:, 0, 0:3])
    c = ops.clearance(worlds, pts, times)
    cw = np.zeros(n, np.float32)
    oracle().orc_clearance_batch(ptr(worlds), ptr(pts), ptr(times), ptr(cw), n)
    assert np.array_equal(c, cw), np.abs(c - cw).max()


def test_gae_and_normalize_operators():
    say("case: GAE hand case + random, normalisation")
    adv, ret = ops.gae(3, 2, [1, 2, 3, 4, 5, 6], [.1, .2, .3, .4, .5, .6], [.2, .3, .4, .5, .6, .7],
                       [0, 0, 1, 0, 0, 0], [0, 0, 0, 1, 0, 0])
    gl = 0.99 * 0.95
    want = np.array([1 + .99 * .2 - .1 + gl * 2.7, 2 + .99 * .3 - .2 + gl * (4 + .99 * .5 - .4), 3 - .3,
                     4 + .99 * .5 - .4, 5 + .99 * .6 - .5, 6 + .99 * .7 - .6])
    assert np.abs(adv - want).max() < 2e-5
    rng = np.random.default_rng(0)
    T, N = 37, 101
    r, v, nv = (rng.normal(0, 1, T * N).astype(np.float32) for _ in range(3))
    te = (rng.random(T * N) < 0.05).astype(np.uint8)
    tr = ((rng.random(T * N) < 0.03) & (te == 0)).astype(np.uint8)
    a_g, r_g = ops.gae(T, N, r, v, nv, te, tr)
    a_o, r_o = np.zeros(T * N, np.float32), np.zeros(T * N, np.float32)
    oracle().orc_compute_gae(T, N, ptr(r), ptr(v), ptr(nv), ptr(te), ptr(tr), np.float32(.99), np.float32(.95),
                             ptr(a_o), ptr(r_o))
    assert np.array_equal(a_g, a_o) and np.array_equal(r_g, r_o)
    x = rng.normal(3, 5, 300_001).astype(np.float32)
    y = ops.normalize(x)
    z = x.copy()
    oracle().orc_normalize_advantages(ptr(z), len(z), np.float32(1e-8))
    assert np.array_equal(y, z), np.abs(y - z).max()


@pytest.mark.parametrize("n,T,epochs,minibatch", [(512, 40, 2, 256), (2048, 136, 1, 1 << 20),
                                                   (8192, 33, 2, 65536), (96, 20, 2, 1000)])
def test_gae_normalize_in_update_bit_exact(n, T, epochs, minibatch):
    """PPOTrainer::rollout_update's GAE and advantage normalisation
    (ppo.hpp:108-140; main.mm:1327-1330) on synthetic rollouts equal the
    oracle's bit for bit.  The update's first epoch rescales the rows as it
    reads them and stores them back, so the advantages after the update are
    the normalised ones: 512 envs (16 slices of 32 envs in plain order; 256-row
    minibatches, two epochs), 2,048 envs over 136 ticks (two 128-tick tiles,
    slices grouped by XCD; one minibatch of many chunks), 8,192 envs over 33
    ticks (17 groups of 64 chunks, the last partial) and 96 envs (scalar row
    loads; a partial last minibatch).  Two updates in a row on one trainer."""
    say("case: GAE + normalisation in rollout_update, N=%d T=%d epochs=%d minibatch=%d" % (n, T, epochs, minibatch))
    rng = np.random.default_rng(n + T)
    R = n * T
    sim = Sim(config(n=n, family=1), T, raptor=raptor_fixture()[0])
    ppo = PPOTrainer(sim, epochs, minibatch)
    try:
        for it in range(2):
            r = (rng.normal(0.2, 1.5, R) * rng.uniform(0.1, 2.0, R)).astype(np.float32)
            v, nv = (rng.normal(0, 3, R).astype(np.float32) for _ in range(2))
            te = (rng.random(R) < 0.04).astype(np.uint8)
            tr = ((rng.random(R) < 0.03) & (te == 0)).astype(np.uint8)
            for name, x in (("rewards", r), ("values", v), ("next_values", nv), ("terminated", te),
                            ("truncated", tr)):
                sim.set(name, x)
            ppo.rollout_update(it)
            sim.sync()
            a_o, r_o = np.zeros(R, np.float32), np.zeros(R, np.float32)
            oracle().orc_compute_gae(T, n, ptr(r), ptr(v), ptr(nv), ptr(te), ptr(tr), np.float32(.99),
                                     np.float32(.95), ptr(a_o), ptr(r_o))
            oracle().orc_normalize_advantages(ptr(a_o), R, np.float32(1e-8))
            assert np.array_equal(sim.get("returns"), r_o), it
            got = sim.get("advantages")
            assert np.array_equal(got, a_o), (it, np.abs(got - a_o).max())
    finally:
        ppo.close()
        sim.close()


@pytest.mark.parametrize("lanes", [8, 16, 4])
def test_rollout_parity(lanes):
    say("case: rollout N=64 T=40 family=1 lanes=%d" % lanes)
    cfg = config(n=64, family=1, speed=1.0, distance=3.0, max_steps=25)
    sim, _, ora = make_pair(cfg, 40, lanes=lanes)
    bad = compare(sim, ora, ENV_BUFFERS)
    assert not bad, ("after reset", bad)
    sim.collect()
    sim.sync()
    ora.collect()
    bad = compare(sim, ora, ENV_BUFFERS + ROW_BUFFERS, tol=TOL)
    assert not bad, bad
    assert ora.get("runs")["episodes"].sum() > 0


@pytest.mark.parametrize("plant", ["crazyflie", "heavier", "tilted_rotor"])
def test_rollout_parity_plants(plant):
    """The fused 8-lane kernel with the Crazyflie plant runs an instance whose
    plant constants are compiled in; any other plant runs the instance that
    reads the launch's plant (standard structure: `heavier`, 10 % more mass;
    general derivative: `tilted_rotor`, rotor 0 thrust tilted)."""
    say("case: rollout N=64 T=40 plant=%s" % plant)
    p = crazyflie().copy()
    if plant == "heavier":
        p["mass"] = np.float32(p["mass"] * np.float32(1.1))
    elif plant == "tilted_rotor":
        p["rotor_thrust_directions"][:3] = np.array([0.05, 0.0, 0.99875], np.float32)
    cfg = config(n=64, family=1, speed=1.0, distance=3.0, max_steps=25)
    weights = raptor_fixture()[0]
    sim = Sim(cfg, 40, raptor=weights, physics=p)
    ora = OracleTrainer(cfg, 40, weights, physics=p)
    try:
        sim.collect()
        sim.sync()
        ora.collect()
        bad = compare(sim, ora, ENV_BUFFERS + ROW_BUFFERS, tol=0.0)
        assert not bad, bad
        assert ora.get("runs")["episodes"].sum() > 0
    finally:
        sim.close()


@pytest.mark.parametrize("variant", ["delays_wind_noise", "eval", "movers3", "mixed6", "rehearsal13",
                                     "goal_script", "threat_mix_delays", "sensor_period2"])
def test_rollout_parity_variants(variant):
    kw = dict(n=48, family=1, speed=1.0, distance=3.0, max_steps=30)
    if variant == "delays_wind_noise":
        kw.update(sensor_delay=2, command_delay=1, wind=0.5, depth_noise=0.05, dropout=0.1)
    elif variant == "eval":
        kw.update(eval=1, max_steps=14)
    elif variant == "movers3":
        kw.update(family=3)
    elif variant == "mixed6":
        kw.update(family=6, distance=4.0)
    elif variant == "rehearsal13":
        kw.update(family=13, speed=1.5, distance=4.0, sensor_delay=2, command_delay=1, wind=0.5)
    elif variant == "threat_mix_delays":  # moving-threat mix with 100 ms sensor and command delays
        kw.update(family=13, speed=1.5, distance=4.0, sensor_delay=2, command_delay=2, max_steps=60)
    elif variant == "sensor_period2":  # a depth frame every other tick, one frame of sensor delay
        kw.update(sensor_period=2, sensor_delay=1, command_delay=1)
    elif variant == "goal_script":
        kw.update(mode=2, family=0, eval=1, speed=0.5, distance=4.0, max_steps=200)
    say("case: rollout variant %s" % variant)
    cfg = config(**kw)
    sim, _, ora = make_pair(cfg, 36)
    sim.collect()
    sim.sync()
    ora.collect()
    bad = compare(sim, ora, ENV_BUFFERS + ROW_BUFFERS, tol=TOL)
    assert not bad, bad


@pytest.mark.parametrize("epochs,minibatch", [(2, 256), (1, 512), (1, 200), (2, 200), (1, 17)])
def test_iteration_parity(epochs, minibatch):
    """Two iterations against the oracle.  Minibatches of at most 256 rows
    take the one-chunk path (row-parallel forward, parameter-parallel
    gradient); 200-row minibatches leave a 48-row last one and end an update
    after an odd (11) and an even (22) number of steps; 17-row minibatches
    give the forward a one-row workgroup in every step and an 8-row last
    minibatch (121 steps)."""
    say("case: iteration N=32 T=64 epochs=%d minibatch=%d" % (epochs, minibatch))
    cfg = config(n=32, family=1, speed=1.0, distance=3.0, max_steps=40)
    sim, ppo, ora = make_pair(cfg, 64, epochs=epochs, minibatch=minibatch)
    for it in range(2):
        sim.collect()
        ppo.rollout_update(it)
        sim.sync()
        ora.iteration(it)
        bad = compare(sim, ora, ["advantages", "returns", "actor", "critic", "actor_m", "actor_v", "critic_m",
                                 "critic_v", "metric_rows"] + ENV_BUFFERS + ROW_BUFFERS, tol=TOL)
        assert not bad, (it, bad)
        assert ppo.optimizer_step == ora.optimizer_step
        assert np.abs(ppo.metric_mean() - ora.metric_mean()).max() <= TOL


@pytest.mark.parametrize("n,minibatch", [(256, 4096), (512, 16384)])
def test_baseline_schedule_parity_large_minibatch(n, minibatch):
    """One epoch of four minibatches (the benchmark schedule) at T=64:
    minibatches of 4096 rows exercise the multi-chunk gradient reduction,
    16384 rows (64 chunks) its two-level grouping, and 32768 rows (128
    chunks) the grouped advantage statistics."""
    say("case: iteration N=%d T=64 epochs=1 minibatch=%d" % (n, minibatch))
    cfg = config(n=n, family=1, speed=1.0, distance=3.0)
    sim, ppo, ora = make_pair(cfg, 64, epochs=1, minibatch=minibatch)
    sim.collect()
    ppo.rollout_update(0)
    sim.sync()
    ora.iteration(0)
    bad = compare(sim, ora, ["advantages", "returns", "actor", "critic", "actor_m", "critic_v", "metric_rows"]
                  + ROW_BUFFERS + ENV_BUFFERS, tol=TOL)
    assert not bad, bad


def test_production_path_bit_exact():
    """The benchmark's code path (8 lanes per env, 2 ring slots: the 4-wavefront
    workgroup with matrix-core layers) and one PPO iteration of 4096-row
    minibatches reproduce the oracle bit for bit: every buffer, float fields
    included, compared at tolerance 0."""
    say("case: bit-exact iteration N=128 T=64 epochs=1 minibatch=4096")
    cfg = config(n=128, family=1, speed=1.0, distance=3.0, max_steps=40)
    sim, ppo, ora = make_pair(cfg, 64, epochs=1, minibatch=4096)
    sim.collect()
    ppo.rollout_update(0)
    sim.sync()
    ora.iteration(0)
    bad = compare(sim, ora, ["advantages", "returns", "actor", "critic", "actor_m", "actor_v", "critic_m", "critic_v",
                             "metric_rows"] + ENV_BUFFERS + ROW_BUFFERS, tol=0.0)
    assert not bad, bad


@pytest.mark.parametrize("actor_obs", [181, 184])
def test_partial_chunks_bit_exact(actor_obs):
    """Minibatches whose last chunk is partial: 1,920 rows in minibatches of
    600 (chunks of 256, 256 and 88 rows: the row sums' general loop, the
    masked rows of the forward tiles and of the weight-gradient slabs with
    their ones column) and a last minibatch of 120 rows (the one-chunk
    path), two epochs and two iterations: every buffer at tolerance 0."""
    say("case: partial chunks N=48 T=40 epochs=2 minibatch=600 actor_obs=%d" % actor_obs)
    cfg = config(n=48, family=1, speed=1.0, distance=3.0, max_steps=30)
    sim, ppo, ora = make_pair(cfg, 40, epochs=2, minibatch=600, actor_obs=actor_obs)
    for it in range(2):
        sim.collect()
        ppo.rollout_update(it)
        sim.sync()
        ora.iteration(it)
        bad = compare(sim, ora, ["advantages", "returns", "actor", "critic", "actor_m", "actor_v", "critic_m",
                                 "critic_v", "metric_rows", "grad_norm_rows"] + ENV_BUFFERS + ROW_BUFFERS, tol=0.0)
        assert not bad, (it, bad)


def test_stress_scale_bit_exact():
    """65,536 envs (the scale-stress env count: 2,048 workgroups of the
    benchmark kernel), 4 ticks with episodes ending after 3 steps (resets at
    scale) and one PPO iteration of four 65,536-row minibatches (256 chunks
    each, the two-level gradient grouping): every buffer bit-identical to the
    oracle."""
    say("case: bit-exact N=65536 T=4 max_steps=3, 1 epoch x 4 minibatches of 65536")
    cfg = config(n=65536, family=1, speed=1.0, distance=3.0, max_steps=3)
    sim, ppo, ora = make_pair(cfg, 4, epochs=1, minibatch=65536)
    sim.collect()
    ppo.rollout_update(0)
    sim.sync()
    ora.iteration(0)
    bad = compare(sim, ora, ["advantages", "returns", "actor", "critic", "actor_m", "actor_v", "critic_m", "critic_v",
                             "metric_rows"] + ENV_BUFFERS + ROW_BUFFERS, tol=0.0)
    assert not bad, bad
    assert ora.get("runs")["episodes"].sum() >= 65536


@pytest.mark.parametrize("family,ticks", [(13, 12), (6, 6), (2, 6), (3, 6), (7, 6)])
def test_mixed_world_depth_bit_exact(family, ticks):
    """Worlds of boxes, spheres (moving ones among them) and cylinders at
    scale (2,048 envs, so wavefronts mix world kinds): the per-kind LDS
    tables of the ray cast and the generic cast give depth frames, pooled
    observations and every other buffer bit-identical to the oracle, through
    resets (episodes end after 4 steps)."""
    say("case: mixed worlds family %d, N=2048 T=%d" % (family, ticks))
    cfg = config(n=2048, family=family, speed=1.5, distance=4.0, max_steps=4)
    sim, _, ora = make_pair(cfg, ticks)
    sim.collect()
    sim.sync()
    ora.collect()
    bad = compare(sim, ora, ENV_BUFFERS + ROW_BUFFERS, tol=0.0)
    assert not bad, bad
    kinds = ora.get("worlds")["obstacles"]["kind"]
    counts = ora.get("worlds")["count"]
    present = {int(k) for n in range(len(counts)) for k in kinds[n][:counts[n]]}
    say("  obstacle kinds present: %s" % sorted(present))


@pytest.mark.parametrize("variant", ["k2_production", "k4_threats_delays", "k8_sensor_delay6"])
def test_geometry_prior_bit_exact(variant):
    """The 184-input actor (ppo.hpp:30-34): the geometry-prior hint computed in
    the observe phase (sim.metal:226, guidance.hpp:38-96) and added to the
    first three means (ppo.hpp:77), then a PPO iteration over the 184-wide rows.
    Every buffer bit-identical to the oracle, on each ring-slot variant of the
    8-lane kernel."""
    kw = dict(n=128, family=1, speed=1.0, distance=3.0, max_steps=40)
    if variant == "k4_threats_delays":
        kw.update(family=13, speed=1.5, distance=4.0, sensor_delay=2, command_delay=1, wind=0.5,
                  sensor_period=2)
    elif variant == "k8_sensor_delay6":
        kw.update(family=6, distance=4.0, sensor_delay=6, depth_noise=0.05, dropout=0.1)
    say("case: 184-input actor %s N=128 T=48 epochs=1 minibatch=2048" % variant)
    cfg = config(**kw)
    sim, ppo, ora = make_pair(cfg, 48, epochs=1, minibatch=2048, actor_obs=184)
    assert sim.actor_obs == 184
    sim.collect()
    ppo.rollout_update(0)
    sim.sync()
    ora.iteration(0)
    bad = compare(sim, ora, ["advantages", "returns", "actor", "critic", "actor_m", "actor_v", "critic_m", "critic_v",
                             "metric_rows"] + ENV_BUFFERS + ROW_BUFFERS, tol=0.0)
    assert not bad, bad
    hint = sim.get("obs").reshape(-1, 184)[:, 181:]
    assert np.count_nonzero(hint) > hint.size // 2, "hint mostly zero"


@pytest.mark.parametrize("variant", ["k2_production", "k4_threats_delays", "k8_sensor_delay6", "eval_inactive"])
def test_geometry_memory_bit_exact(variant):
    """The history-aware hint (cfg.geometry_memory = 1, guidance.hpp:152-194 as
    cpu_reference.hpp:364-372 calls it): per tick the env kernel stops after
    the observation, the memory kernel scores the 85 candidate sweeps against
    the remembered points of up to 8 frames and writes the hint, and the next
    launch acts on the row.  Every buffer after a rollout and a PPO update
    bit-identical to the oracle.  "eval_inactive": evaluation mode, where envs
    stop after one episode and must be left alone by the memory kernel."""
    kw = dict(n=128, family=1, speed=1.0, distance=3.0, max_steps=40, geometry_memory=1)
    if variant == "k4_threats_delays":
        kw.update(family=13, speed=1.5, distance=4.0, sensor_delay=2, command_delay=1, wind=0.5, sensor_period=2)
    elif variant == "k8_sensor_delay6":
        kw.update(family=6, distance=4.0, sensor_delay=6, depth_noise=0.05, dropout=0.1)
    elif variant == "eval_inactive":
        kw.update(eval=1, max_steps=14)
    say("case: geometry memory %s N=128 T=48 epochs=1 minibatch=2048" % variant)
    cfg = config(**kw)
    sim, ppo, ora = make_pair(cfg, 48, epochs=1, minibatch=2048, actor_obs=184)
    sim.collect()
    ppo.rollout_update(0)
    sim.sync()
    ora.iteration(0)
    bad = compare(sim, ora, ["advantages", "returns", "actor", "critic", "actor_m", "actor_v", "critic_m", "critic_v",
                             "metric_rows"] + ENV_BUFFERS + ROW_BUFFERS, tol=0.0)
    assert not bad, bad
    hint = sim.get("obs").reshape(-1, 184)[:, 181:]
    assert np.count_nonzero(hint) > hint.size // 4, "hint mostly zero"


@pytest.mark.parametrize("mode", [12, 13, 16, 17, 18, 19, 22])
def test_guided_modes_bit_exact(mode):
    """Guided evaluation modes of the 184-input actor (sim.metal:211-213,
    233-269; memory.metal:34): means pulled toward the hint by a fixed or
    overhead-dependent scale (12, 13, 16, 17, 19), the previous frame dropped
    (18), fixed-speed commands (19), and mode 22's training through the
    deployed map.  Evaluation settings as main.mm:605-610 uses them (family 8,
    1.5 m/s, 4 m goals, geometry memory from mode 13 on); mode 22 trains
    (sampling on, one PPO update).  Every buffer bit-identical to the oracle."""
    train = mode == 22
    kw = dict(n=128, family=8, speed=1.5, distance=4.0, max_steps=40, mode=mode, eval=0 if train else 1,
              seed=800001, geometry_memory=1 if mode >= 13 else 0)
    say("case: guided mode %d N=128 T=48 (%s)" % (mode, "train + update" if train else "eval"))
    cfg = config(**kw)
    sim, ppo, ora = make_pair(cfg, 48, epochs=1, minibatch=2048, actor_obs=184)
    names = ENV_BUFFERS + ROW_BUFFERS
    if train:
        sim.collect()
        ppo.rollout_update(0)
        sim.sync()
        ora.iteration(0)
        names = names + ["advantages", "returns", "actor", "critic", "actor_m", "actor_v", "metric_rows"]
    else:
        sim.collect()
        sim.sync()
        ora.collect()
    bad = compare(sim, ora, names, tol=0.0)
    assert not bad, bad


@pytest.mark.parametrize("variant", ["boxes_production", "mixed_family3", "guided184", "memory184", "plants_tasks"])
def test_native_camera_bit_exact(variant):
    """The native camera profile (sensor_profile.hpp:18-25, 111-126): vertical
    half-tangent 0.8 and rays cast from 0.08 m ahead of the body point
    (sim.metal:147-152), set on both sides after creation.  Depth frames and
    poses, observations (with the guidance hint's and the geometry memory's
    cell and pixel directions of the same profile), the outcome and a PPO
    update are bit-identical to the oracle at tolerance 0, on the benchmark
    kernel, the mixed-world tables, the 184-input actor with and without the
    geometry memory, and the per-episode path."""
    kw = dict(n=128, family=1, speed=1.0, distance=3.0, max_steps=40)
    actor_obs, ticks = 181, 48
    if variant == "mixed_family3":
        kw.update(family=3, n=512, speed=1.5, distance=4.0, max_steps=8)
    elif variant == "guided184":
        actor_obs = 184
    elif variant == "memory184":
        actor_obs = 184
        kw.update(geometry_memory=1, max_steps=30)
        ticks = 24
    elif variant == "plants_tasks":
        kw.update(family=12, mode=22, speed=1.5, distance=8.0, max_steps=60, geometry_memory=1)
        actor_obs, ticks = 184, 16
    say("case: native camera %s" % variant)
    cfg = config(**kw)
    sim, ppo, ora = make_pair(cfg, ticks, epochs=1, minibatch=2048, actor_obs=actor_obs)
    if variant == "plants_tasks":
        from oracle_lib import task_runtime, task_settings
        rt, ts = task_runtime(1.0), task_settings(2, 12)
        sim.set_runtime(rt); sim.set_tasks(ts); sim.reset()
        ora.set_runtime(rt); ora.set_tasks(ts); ora.reset()
    sim.set_camera(abi.CAMERA_NATIVE)
    ora.set_camera(abi.CAMERA_NATIVE)
    cam = sim.camera
    assert int(cam["id"]) == 2 and float(cam["tan_v"]) == np.float32(0.8)
    sim.collect()
    ppo.rollout_update(0)
    sim.sync()
    ora.iteration(0)
    bad = compare(sim, ora, ["advantages", "returns", "actor", "critic", "actor_m", "actor_v", "critic_m", "critic_v",
                             "metric_rows"] + ENV_BUFFERS + ROW_BUFFERS, tol=0.0)
    assert not bad, bad
    if variant == "boxes_production":  # the same envs with the legacy camera see other depths
        leg = Sim(cfg, ticks, raptor=raptor_fixture()[0])
        leg.collect()
        leg.sync()
        assert not np.array_equal(leg.get("sensors"), sim.get("sensors"))
        assert not np.array_equal(leg.get("poses"), sim.get("poses"))
