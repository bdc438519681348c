"""The oracle's batched simulator and trainer (cpu_reference::Trainer
restated): the reference's closed-loop check, episode/reset semantics and
rollout invariants."""
import numpy as np
import pytest

from oracle_lib import OracleTrainer, crazyflie, oracle, ptr, raptor_fixture, ref, ref_available
from mdnav import abi

F = np.float32


@pytest.fixture(scope="module")
def weights():
    return raptor_fixture()[0]


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built")
def test_closed_loop_against_reference_adapter(weights):
    """closed_loop_tests (main.mm:809-829): 32 envs x 32 ticks x 5 substeps of
    goal script -> PX4 adapter -> RAPTOR -> RK4.  The scalar side uses the
    reference's own raptor_pack_observation, raptor_forward and rl_physics_step;
    gate 5e-4 on state and hidden."""
    cfg = abi.default_config(n=32, mode=2, family=0, eval=1, speed=0.5, distance=4.0)
    t = OracleTrainer(cfg, 32, weights)
    states, runs, worlds = t.get("states"), t.get("runs"), t.get("worlds")
    lib = ref()
    w = np.array(weights, abi.RAPTOR_WEIGHTS)
    params = np.array(crazyflie(), abi.PHYSICS_PARAMS)
    dt = float(params["dt"])
    for n in range(32):
        s = states[n:n + 1].copy()
        hidden = runs[n]["hidden"].astype(F).copy()
        motors = runs[n]["motors"].astype(F).copy()
        refpos = runs[n]["reference_position"].astype(F).copy()
        goal = worlds[n]["goal"].astype(F)
        for _ in range(32):
            q = np.ascontiguousarray(s["orientation_wxyz"][0])
            rot = np.zeros(9, F)
            lib.ref_quaternion_matrix(ptr(q), ptr(rot))
            delta = (goal - s["position"][0]).astype(F)
            ln = np.float32(np.sqrt(np.float32(delta @ delta)))
            d = (delta * F(1 / max(ln, 1e-8)) * F(min(ln, 0.5))).astype(F)
            r = rot.reshape(3, 3)
            body = (r.T @ d).astype(F)
            vel = (r @ body).astype(F)
            for _ in range(5):
                refpos = (refpos + vel * F(dt)).astype(F)
                obs = np.zeros(22, F)
                args = [np.ascontiguousarray(x, F) for x in (s["position"][0], s["orientation_wxyz"][0],
                                                             s["linear_velocity"][0], s["angular_velocity_body"][0],
                                                             refpos, [1, 0, 0, 0], vel, motors)]
                lib.ref_raptor_pack_observation(*[ptr(a) for a in args], ptr(obs))
                act = np.zeros(4, F)
                lib.ref_raptor_forward(ptr(w), ptr(obs), ptr(hidden), ptr(act))
                motors = np.clip(act, -1, 1).astype(F)
                nxt = np.zeros(1, abi.PHYSICS_STATE)
                lib.ref_physics_step_batch(ptr(s), ptr(motors), ptr(np.zeros(3, F)), ptr(params), ptr(nxt), 1)
                s = nxt
        states[n] = s[0]
        runs[n]["hidden"] = hidden
    t.collect(32)
    got_s, got_r = t.get("states"), t.get("runs")
    assert np.all(got_r["episodes"] == 0)
    flat = lambda x: np.ascontiguousarray(x).view(F).reshape(len(x), 17)
    state_err = np.abs(flat(got_s) - flat(states)).max()
    hidden_err = np.abs(got_r["hidden"] - runs["hidden"]).max()
    assert state_err < 5e-4 and hidden_err < 5e-4, (state_err, hidden_err)
    # the goal script actually moved the vehicles
    assert np.abs(got_s["position"][:, 0]).max() > 0.3


def test_first_reset(weights):
    """sim_reset_one (sim.metal:55-94): hover rpm root, start pose, ring fill."""
    cfg = abi.default_config(n=8, family=1, distance=3.0)
    t = OracleTrainer(cfg, 4, weights)
    s, r, w = t.get("states"), t.get("runs"), t.get("worlds")
    assert np.all(s["position"] == np.array([0, 0, 1.5], F))
    assert np.all(s["orientation_wxyz"] == np.array([1, 0, 0, 0], F))
    p = crazyflie()
    c0, c1, c2 = (float(x) for x in p["rotor_thrust_coefficients"][:3])
    hover = (-c1 + np.sqrt(c1 * c1 - 4 * c2 * (c0 - float(p["mass"]) * 9.81 / 4))) / (2 * c2)
    assert np.abs(s["rpm"] - hover).max() < 1e-6
    assert np.all(r["hidden"] == weights["initial_hidden_state"])
    assert np.all(w["count"] == 8) and np.all(w["family"] == 1)
    assert np.all(t.get("sensors") == 12) and np.all(t.get("commands") == 0)
    # first rng = seed + n*747796405 + 2891336453 advanced by one draw (world seed)
    for n in range(8):
        x = (42 + n * 747796405 + 2891336453) & 0xffffffff
        x ^= (x << 13) & 0xffffffff
        x ^= x >> 17
        x ^= (x << 5) & 0xffffffff
        assert w["seed"][n] == x and r["rng"][n] == x


def test_rollout_invariants(weights):
    cfg = abi.default_config(n=64, family=1, speed=1.0, distance=3.0, max_steps=30)
    t = OracleTrainer(cfg, 48, weights)
    t.collect()
    term, trunc = t.get("terminated"), t.get("truncated")
    assert set(np.unique(term)) <= {0, 1} and set(np.unique(trunc)) <= {0, 1}
    assert not np.any(term & trunc)
    s = t.get("states")
    assert np.abs(np.linalg.norm(s["orientation_wxyz"].astype(np.float64), axis=1) - 1).max() < 1e-5
    rew = t.get("rewards").reshape(48, 64)
    assert np.all(np.isfinite(rew))
    # collisions pay -10, successes +10, others lie in the shaping band
    ends = (term.reshape(48, 64) == 1)
    assert np.all(np.abs(rew[~ends]) < 1.0)
    runs = t.get("runs")
    assert runs["episodes"].sum() == term.sum() + trunc.sum()
    assert runs["episodes"].sum() > 0
    # obs: pooled depth in (0,1], goal direction unit length, critic obs in range
    obs = t.get("obs").reshape(48, 64, 181)
    assert np.all(obs[:, :, :160] > 0) and np.all(obs[:, :, :160] <= 1)
    assert np.abs(np.linalg.norm(obs[:, :, 160:163].astype(np.float64), axis=2) - 1).max() < 1e-5
    lp = t.get("logp")
    assert np.all(np.isfinite(lp))


def test_eval_stops_after_first_episode(weights):
    """sim.metal:146/183/230/273: with eval set an env stops after its first
    episode and is not reset (sim.metal:330)."""
    cfg = abi.default_config(n=16, family=1, eval=1, speed=1.0, distance=3.0, max_steps=12)
    t = OracleTrainer(cfg, 40, weights)
    t.collect()
    r = t.get("runs")
    assert np.all(r["episodes"] == 1)
    assert np.all(r["steps"] <= 12)


def test_training_iteration_updates(weights):
    cfg = abi.default_config(n=32, family=1, speed=1.0, distance=3.0)
    t = OracleTrainer(cfg, 16, weights, epochs=2, minibatch=128)
    a0 = t.get("actor")
    t.iteration(0)
    assert t.optimizer_step == 2 * 4
    assert np.abs(t.get("actor") - a0).max() > 0
    m = t.metric_mean()
    assert np.all(np.isfinite(m)) and 0.5 < m[3] < 1.5
    adv = t.get("advantages").astype(np.float64)
    assert abs(adv.mean()) < 1e-5 and abs(adv.std() - 1) < 1e-4
    ls = t.get("actor")[abi.policy_shape()["actor_log_std"]:]
    assert np.all(ls >= -2) and np.all(ls <= 0.5)


# ---------------------------------------------------------------- reward and critic observation
# Pins of the default-mode shaping reward (cpu_reference.hpp:497-500 ==
# sim.metal:305) and the critic observation (cpu_reference.hpp:379-394 ==
# sim.metal:159-181) with values worked out by hand, so that a dropped term,
# a wrong sign, scale or index fails.

def step_reward(before, after, clearance, risk, success=False, collision=False):
    return oracle().orc_step_reward(before, after, clearance, risk, int(success), int(collision))


def test_step_reward_closed_forms():
    # hovering in open space: only the 0.01 step cost
    assert step_reward(3.0, 3.0, 1.32, 0.0) == F(-0.01)
    assert step_reward(3.0, 3.0, 1.32, 0.8) == F(-0.01)  # clearance >= 0.6: no risk penalty
    # 0.25 m of progress toward the goal earns twice that
    assert step_reward(3.0, 2.75, 1.0, 0.0) == pytest.approx(0.49, abs=1e-6)
    # moving away costs symmetrically
    assert step_reward(2.75, 3.0, 1.0, 0.0) == pytest.approx(-0.51, abs=1e-6)
    # clearance 0.3 m is halfway into the 0.6 m risk band: -risk * 0.5
    assert step_reward(3.0, 3.0, 0.3, 0.8) == pytest.approx(-0.01 - 0.4, abs=1e-6)
    assert step_reward(3.0, 3.0, 0.45, 0.8) == pytest.approx(-0.01 - 0.2, abs=1e-6)
    # the band is clamped: at the edge nothing, at or below 0 the full coefficient
    assert step_reward(3.0, 3.0, 0.6, 0.8) == pytest.approx(-0.01, abs=1e-7)
    assert step_reward(3.0, 3.0, -0.2, 0.8) == pytest.approx(-0.81, abs=1e-6)
    # terminal bonuses
    assert step_reward(0.5, 0.3, 0.9, 0.0, success=True) == pytest.approx(0.4 - 0.01 + 10, abs=1e-5)
    assert step_reward(3.0, 3.0, -0.05, 0.0, collision=True) == pytest.approx(-10.01, abs=1e-5)
    assert step_reward(3.0, 2.9, -0.05, 1.0, collision=True) == pytest.approx(0.2 - 0.01 - 1.0 - 10, abs=1e-5)


def _state(position, q, vel, omega):
    s = np.zeros((), abi.PHYSICS_STATE)
    s["position"], s["orientation_wxyz"] = position, q
    s["linear_velocity"], s["angular_velocity_body"] = vel, omega
    return s


def _obstacle(w, i, kind, center, size, velocity=(0, 0, 0)):
    o = w["obstacles"][i]
    o["kind"], o["center"], o["size"], o["velocity"] = kind, center, size, velocity


def test_critic_observation_by_hand():
    s = _state((1, 2, 1.5), (0.8, 0.36, 0.48, 0.0), (4, -2, 1), (0.8, -0.4, 2))
    w = np.zeros((), abi.WORLD)
    w["goal"], w["wind"] = (6, -3, 2.5), (0.3, -0.2, 0.1)
    _obstacle(w, 0, 0, (2, 2, 1.5), (0.5, 0.5, 0.5))                     # static box, 0.5 m ahead
    _obstacle(w, 1, 0, (1, 5, 1.5), (0.25, 0.25, 0.25), (1, -2, 0))      # drifting box
    # kind-3 bounded mover: centre + v * a sin(t |v| / a + phase) / |v|; at
    # t = 0.5 with |v| = 5, a = 2 the argument is 1.25 + phase = pi/2, so the
    # centre is displaced by v * 0.4 = (1.2, 1.6, 0)
    _obstacle(w, 2, 3, (-1, 2, 2), (0.3, 2.0, np.pi / 2 - 1.25), (3, 4, 0))
    _obstacle(w, 3, 1, (10, 0, 2), (0.5, 0, 0))                          # fourth: not observed
    w["count"] = 4
    r = np.zeros((), abi.SIM_RUN)
    r["reference_position"], r["steps"], r["elapsed"] = (1.25, 1.5, 1.5), 50, 0.5
    out = np.full(32, np.nan, F)
    oracle().orc_critic_observation(ptr(s), ptr(w), ptr(r), ptr(out))
    want = np.array([
        0.5, -0.5, 0.1,          # goal - position, / 10
        1.0, -0.5, 0.25,         # linear velocity / 4
        0.2, -0.1, 0.5,          # body rates / 4
        0.8, 0.36, 0.48, 0.0,    # orientation wxyz
        0.1, 0.2, 0.15,          # position / 10
        0.5, -1.0, 0.0,          # (reference - position) * 2
        (0.5 - 0.18) / 5,        # clearance / 5: the static box face is 0.5 m away
        0.25,                    # steps / 200
        0.1, 0.0, 0.0,           # static box centre - position, / 10
        0.05, 0.2, 0.0,          # drifting box at t = 0.5: (1.5, 4, 1.5)
        -0.08, 0.16, 0.05,       # kind-3 mover at t = 0.5: (0.2, 3.6, 2)
        0.3, -0.2], np.float64)  # wind x, y
    assert np.abs(out - want).max() < 2e-6, np.abs(out - want)
    # fewer than three obstacles leave the remaining centre slots at zero
    w["count"] = 1
    oracle().orc_critic_observation(ptr(s), ptr(w), ptr(r), ptr(out))
    assert np.all(out[24:30] == 0) and out[21] == pytest.approx(0.1)
    # the nearest surface decides the clearance entry: a wall 0.4 m below
    s2 = _state((1, 2, 0.4), (1, 0, 0, 0), (0, 0, 0), (0, 0, 0))
    w["count"] = 0
    oracle().orc_critic_observation(ptr(s2), ptr(w), ptr(r), ptr(out))
    assert out[19] == pytest.approx((0.4 - 0.18) / 5, abs=1e-7)


def test_reward_and_critic_rows_in_the_trainer(weights):
    """One tick of the trainer on hand-placed worlds: each row's reward equals
    2 (d_before - d_after) - 0.01 - risk clamp((0.6 - c)/0.6) +- 10 from the
    env's own positions, and the critic rows are the critic observation of
    the state before (co) and after (next critic obs) the tick."""
    risk = 0.5
    cfg = abi.default_config(n=4, family=1, eval=1, speed=1.0, distance=3.0, risk_coef=risk)
    t = OracleTrainer(cfg, 1, weights)
    w = t.buffer("worlds")
    w["count"] = 0
    w["goal"] = [(4, 0, 1.5), (4, 0, 1.5), (4, 0, 1.5), (0.1, 0, 1.5)]
    # env 1: a box face 0.5 m in front (clearance 0.32, inside the risk band);
    # env 2: a box around the start (collision in the first substep)
    _obstacle(w[1], 0, 0, (0.7, 0, 1.5), (0.2, 1, 1))
    _obstacle(w[2], 0, 0, (0.2, 0, 1.5), (0.3, 0.3, 0.3))
    w["count"][1] = 1
    w["count"][2] = 1
    s0 = t.get("states")
    runs0, worlds = t.get("runs"), t.get("worlds")
    t.collect(1)
    s1, runs1 = t.get("states"), t.get("runs")
    rew, term = t.get("rewards"), t.get("terminated")
    d = lambda s, n: np.linalg.norm(worlds["goal"][n].astype(np.float64) - s["position"][n].astype(np.float64))
    progress = np.array([2 * (d(s0, n) - d(s1, n)) for n in range(4)])
    assert abs(rew[0] - (progress[0] - 0.01)) < 1e-5                          # open space
    c_end = 0.7 - 0.2 - float(s1["position"][1][0]) - 0.18
    assert 0.25 < c_end < 0.4
    assert abs(rew[1] - (progress[1] - 0.01 - risk * (0.6 - c_end) / 0.6)) < 5e-3  # risk band
    assert term[2] == 1 and abs(rew[2] - (progress[2] - 0.01 - risk - 10)) < 1e-5  # collision
    assert term[3] == 1 and abs(rew[3] - (progress[3] - 0.01 + 10)) < 1e-5         # success
    assert term[0] == 0 and term[1] == 0
    co, nco = t.get("critic_obs").reshape(4, 32), t.get("next_critic_obs").reshape(4, 32)
    out = np.zeros(32, F)
    for n in range(4):
        oracle().orc_critic_observation(ptr(s0[n:n + 1]), ptr(worlds[n:n + 1]), ptr(runs0[n:n + 1]), ptr(out))
        assert np.array_equal(co[n], out)
        oracle().orc_critic_observation(ptr(s1[n:n + 1]), ptr(worlds[n:n + 1]), ptr(runs1[n:n + 1]), ptr(out))
        assert np.array_equal(nco[n], out)
    assert np.all(runs1["steps"] == 1) and np.all(nco[:, 20] == F(1 / 200))
