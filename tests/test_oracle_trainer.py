"""The oracle's batched simulator and trainer (cpu_reference::Trainer
restated): the reference's closed-loop check, episode/reset semantics and
rollout invariants."""
import numpy as np
import pytest

from oracle_lib import OracleTrainer, crazyflie, ptr, raptor_fixture, ref, ref_available
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
