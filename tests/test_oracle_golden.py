"""The oracle against the golden vectors the reference's own tests hold:
official L2F transitions (main.mm:138-176, gate 2e-5) and the official
RLtools RAPTOR sequence (main.mm:127-137, gate 2e-5)."""
import numpy as np

from oracle_lib import crazyflie, oracle, physics_fixture, ptr, raptor_fixture
from mdnav import abi


def _step(params, recs):
    lib = oracle()
    states = np.ascontiguousarray(recs["state"])
    actions = np.ascontiguousarray(recs["action"])
    winds = np.ascontiguousarray(recs["wind"])
    out = np.zeros(len(recs), abi.PHYSICS_STATE)
    p = np.array(params, abi.PHYSICS_PARAMS)
    lib.orc_physics_step_batch(ptr(states), ptr(actions), ptr(winds), ptr(p), ptr(out), len(recs))
    return out


def _flat(s):
    return np.ascontiguousarray(s).view(np.float32).reshape(len(s), 17)


def test_physics_official_l2f():
    params, recs, cases, horizon = physics_fixture()
    assert (cases, horizon) == (64, 8)
    err = np.abs(_flat(_step(params, recs)) - _flat(recs["next"])).max()
    assert err < 2e-5, err
    # the fixture's params are the Crazyflie profile of physics.hpp:184-219
    assert params.tobytes() == crazyflie().tobytes()


def test_physics_fixture_discriminates_planted_mistakes():
    """A dropped or sign-flipped term in the plant must fail the golden gate."""
    params, recs, _, _ = physics_fixture()
    for field, idx, value in [("rotor_torque_directions", 2, 1.0), ("inertia_inverse", 0, 1.1e5),
                              ("rotor_time_constants_falling", 0, 0.05)]:
        bad = params.copy()
        bad[field][idx] = value
        err = np.abs(_flat(_step(bad, recs)) - _flat(recs["next"])).max()
        assert err > 2e-5, (field, err)
    # wind applied with the wrong sign
    flipped = recs.copy()
    flipped["wind"] = -flipped["wind"]
    assert np.abs(flipped["wind"]).max() > 0
    err = np.abs(_flat(_step(params, flipped)) - _flat(recs["next"])).max()
    assert err > 2e-5


def test_physics_invariants():
    params, recs, _, _ = physics_fixture()
    nxt = _step(params, recs)
    norms = np.linalg.norm(nxt["orientation_wxyz"].astype(np.float64), axis=1)
    assert np.abs(norms - 1).max() < 1e-6
    assert np.all(nxt["rpm"] >= params["action_min"]) and np.all(nxt["rpm"] <= params["action_max"])


def test_physics_hover_equilibrium():
    """At the hover root of c2 a^2 + c1 a + c0 = m g / 4 the vertical
    acceleration vanishes (closed form)."""
    p = crazyflie()
    c0, c1, c2 = (float(x) for x in p["rotor_thrust_coefficients"][:3])
    target = float(p["mass"]) * 9.81 / 4
    hover = (-c1 + np.sqrt(c1 * c1 - 4 * c2 * (c0 - target))) / (2 * c2)
    s = np.zeros(1, abi.PHYSICS_STATE)
    s["position"] = [0, 0, 1.5]
    s["orientation_wxyz"] = [1, 0, 0, 0]
    s["rpm"] = hover
    rec = np.zeros(1, [("state", abi.PHYSICS_STATE), ("action", np.float32, 4), ("wind", np.float32, 3),
                       ("next", abi.PHYSICS_STATE)])
    rec["state"] = s
    rec["action"] = 2 * hover - 1  # setpoint == hover for action range [0,1]
    out = _step(p, rec)
    assert abs(float(out["linear_velocity"][0, 2])) < 2e-4
    assert abs(float(out["position"][0, 2]) - 1.5) < 1e-5
    assert np.abs(out["angular_velocity_body"]).max() < 1e-5


def test_raptor_official_sequence():
    weights, obs, expected = raptor_fixture()
    assert obs.shape == (16, 22) and expected.shape == (16, 4)
    actions = np.zeros((16, 4), np.float32)
    hidden = np.zeros(16, np.float32)
    w = np.array(weights, abi.RAPTOR_WEIGHTS)
    oracle().orc_raptor_sequence(ptr(w), ptr(obs), 16, ptr(actions), ptr(hidden))
    err = np.abs(actions - expected).max()
    assert err < 2e-5, err
    # recurrent state matters: resetting the hidden state every step breaks parity
    single = np.zeros((16, 4), np.float32)
    for t in range(16):
        o = np.ascontiguousarray(obs[t:t + 1])
        a = np.zeros((1, 4), np.float32)
        oracle().orc_raptor_sequence(ptr(w), ptr(o), 1, ptr(a), ptr(hidden))
        single[t] = a[0]
    assert np.abs(single - expected).max() > 2e-5
