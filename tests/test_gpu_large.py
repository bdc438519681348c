"""Wide-policy PPO (bf16 matrix-core GEMMs, fp32 master weights) against the
fp32 CPU oracle with the same hidden width.

The rollout itself comes from the bit-exact small-policy path, so both sides
hold identical rollout buffers.  The wide policy then re-evaluates them
(log-probabilities of the stored actions, values at s and s'), which is where
bf16 enters: those outputs are compared at stated tolerances.  For the update
both sides start from the GPU's evaluation, so GAE and normalisation must
agree bit for bit, and the post-Adam weights are bounded by the first Adam
steps: each step moves a weight by at most about lr (m/sqrt(v) <= 1 for
the first steps), so two implementations whose gradients differ can differ
by at most 2 * lr * updates per weight; almost all weights, whose gradients
agree in sign and scale, must agree far more closely.
"""
import sys

import numpy as np
import pytest

from gpu_compare import config, make_pair
from mdnav import LargePPOTrainer

pytestmark = pytest.mark.gpu

LOGP_TOL = 5e-2    # abs, sum over 4 action dims of (a - mu)^2 / sigma^2 terms; sigma = e^-1
VALUE_TOL = 2e-2   # abs
MEAN_TOL = 1e-2    # abs, actor means (bf16 inputs and first-layer weights, fp32 accumulation)
# gradients through bf16 GEMMs (inputs and weights rounded to 8 significant
# bits, fp32 accumulation over 32,768 rows): whole-vector and per-block
# relative L2 errors, and the cosine between the two gradients (measured on
# MI355X: 1.9e-3 / 2.8e-3 for actor / critic, blocks <= 2.0e-3, cosine
# 0.999996)
GRAD_REL_TOL = 1e-2
GRAD_BLOCK_REL_TOL = 1e-2
GRAD_COS_MIN = 0.9999


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("hidden,actor_obs", [(256, 181), (5120, 181), (5120, 184)])
def test_wide_policy_against_oracle(hidden, actor_obs):
    """(5120, 184) is the reference's 967,688-parameter capacity actor."""
    say("case: wide policy hidden=%d actor_obs=%d, N=64 T=32, 1 epoch x 2 minibatches of 1024" % (hidden, actor_obs))
    cfg = config(n=64, family=1, speed=1.0, distance=3.0, max_steps=40)
    sim, _, ora = make_pair(cfg, 32, epochs=1, minibatch=1024, actor_obs=actor_obs)
    sim.collect()
    sim.sync()
    ora.collect()
    for name in ("obs", "critic_obs", "next_critic_obs", "actions", "rewards", "terminated", "truncated"):
        assert np.array_equal(sim.get(name), ora.get(name)), name
    lp = LargePPOTrainer(sim, hidden, epochs=1, minibatch=1024)
    ora.set_hidden(hidden)
    for name in ("actor", "critic"):
        assert np.array_equal(lp.get(name), ora.get(name)), ("initialisation", name)
    if (hidden, actor_obs) == (5120, 184):
        assert lp.get("actor").size == 967_688

    lp.evaluate()
    sim.sync()
    ora.evaluate()
    errs = {name: float(np.abs(sim.get(name).astype(np.float64) - ora.get(name)).max())
            for name in ("logp", "values", "next_values")}
    say("  evaluation max |gpu - oracle|:", errs)
    assert errs["logp"] <= LOGP_TOL and errs["values"] <= VALUE_TOL and errs["next_values"] <= VALUE_TOL, errs

    for name in ("logp", "values", "next_values"):
        ora.set(name, sim.get(name))
    lp.rollout_update(0)
    sim.sync()
    ora.gae()
    ora.normalize()
    ora.update(0)
    assert np.array_equal(sim.get("advantages"), ora.get("advantages"))
    assert np.array_equal(sim.get("returns"), ora.get("returns"))
    assert lp.optimizer_step == 2
    lr = float(cfg["learning_rate"])
    bound = 2 * lr * lp.optimizer_step
    for name in ("actor", "critic"):
        d = np.abs(lp.get(name).astype(np.float64) - ora.get(name))
        close = float(np.mean(d <= 0.1 * lr))
        say("  %s after update: max |diff| %.3g (bound %.3g), fraction within 0.1*lr %.4f" % (name, d.max(), bound, close))
        assert d.max() <= bound * 1.01, (name, d.max())
        assert close >= 0.95, (name, close)
    m_gpu, m_ora = lp.metric_mean(), ora.metric_mean()
    say("  metric means gpu", m_gpu, "oracle", m_ora)
    assert np.all(np.isfinite(m_gpu))
    assert np.abs(m_gpu - m_ora).max() <= 1e-2 + 1e-2 * np.abs(m_ora).max()


def test_wide_policy_production_minibatch():
    """The capacity actor (hidden 5120, 184 inputs) at its production
    minibatch: N=1024 x T=32 = 32,768 rows in one minibatch of one epoch, so
    the row-chunk partial slots and their sum over the whole minibatch are
    exercised at full size.  After one Adam step from zero moments the first
    moment is (1 - beta1) times the (clipped, decayed) gradient on both sides,
    so the GPU's gradient is compared with the fp32 oracle's directly: as a
    vector (relative L2 error and cosine) and block by block, at bf16
    tolerances."""
    hidden, actor_obs, n, T = 5120, 184, 1024, 32
    say("case: wide policy production minibatch hidden=%d actor_obs=%d N=%d T=%d, 1 epoch x 1 minibatch of %d" % (
        hidden, actor_obs, n, T, n * T))
    cfg = config(n=n, family=1, speed=1.0, distance=3.0, max_steps=40)
    sim, _, ora = make_pair(cfg, T, epochs=1, minibatch=n * T, actor_obs=actor_obs)
    sim.collect()
    sim.sync()
    ora.collect()
    for name in ("obs", "critic_obs", "next_critic_obs", "actions", "rewards", "terminated", "truncated"):
        assert np.array_equal(sim.get(name), ora.get(name)), name
    lp = LargePPOTrainer(sim, hidden, epochs=1, minibatch=n * T)
    ora.set_hidden(hidden)
    for name in ("actor", "critic"):
        assert np.array_equal(lp.get(name), ora.get(name)), ("initialisation", name)
    lp.evaluate()
    sim.sync()
    ora.evaluate()
    errs = {name: float(np.abs(sim.get(name).astype(np.float64) - ora.get(name)).max())
            for name in ("logp", "values", "next_values")}
    say("  evaluation max |gpu - oracle|:", errs)
    assert errs["logp"] <= LOGP_TOL and errs["values"] <= VALUE_TOL and errs["next_values"] <= VALUE_TOL, errs
    for name in ("logp", "values", "next_values"):
        ora.set(name, sim.get(name))
    lp.rollout_update(0)
    sim.sync()
    ora.gae()
    ora.normalize()
    ora.update(0)
    assert np.array_equal(sim.get("advantages"), ora.get("advantages"))
    assert lp.optimizer_step == 1
    D, H = actor_obs, hidden
    blocks = {"actor": [("W1", 0, H * D), ("b1", H * D, H * D + H), ("W2", H * D + H, H * D + 5 * H),
                        ("b2+log_std", H * D + 5 * H, H * D + 5 * H + 8)],
              "critic": [("all", 0, None)]}
    for name in ("actor", "critic"):
        mg = lp.get(name + "_m").astype(np.float64)
        mo = ora.get(name + "_m").astype(np.float64)
        rel = float(np.linalg.norm(mg - mo) / np.linalg.norm(mo))
        cos = float(mg @ mo / (np.linalg.norm(mg) * np.linalg.norm(mo)))
        say("  %s first moment: relative L2 error %.3g, cosine %.6f" % (name, rel, cos))
        assert rel <= GRAD_REL_TOL and cos >= GRAD_COS_MIN, (name, rel, cos)
        for label, b, e in blocks[name]:
            g, o = mg[b:e], mo[b:e]
            brel = float(np.linalg.norm(g - o) / max(np.linalg.norm(o), 1e-30))
            say("    %s %s: relative L2 error %.3g" % (name, label, brel))
            assert brel <= GRAD_BLOCK_REL_TOL, (name, label, brel)
        d = np.abs(lp.get(name).astype(np.float64) - ora.get(name))
        close = float(np.mean(d <= 0.1 * float(cfg["learning_rate"])))
        say("  %s weights after the step: fraction within 0.1*lr %.4f" % (name, close))
        assert close >= 0.95, (name, close)


@pytest.mark.parametrize("variant", ["static", "threat_mix_delays", "sensor_period2", "guided", "guided_memory"])
def test_wide_policy_closed_loop(variant):
    """Sim::collect with the wide actor choosing every action (split ticks:
    env kernel up to the observation, wide forward, env kernel from act).

    The env step is checked bit for bit against the oracle driven by the same
    means (the oracle's act() takes them in place of its own forward pass);
    the means themselves against the oracle's fp32 forward of the same
    observation rows at bf16 tolerance, and the values at s and s' likewise.
    Two collects in a row cover the hand-over at a collect boundary; resets
    happen inside the split launches (max_steps below the ticks run).
    "guided": the 184-input actor, hint computed in the env step and added to
    the wide means; "guided_memory": the history-aware hint from the memory
    kernel between the env launches."""
    from gpu_compare import ENV_BUFFERS, compare
    from oracle_lib import oracle, ptr

    hidden, T = 256, 24
    kw = dict(n=64, family=1, speed=1.0, distance=3.0, max_steps=25)
    if variant == "threat_mix_delays":  # 4 ring slots: the one-wavefront kernel
        kw.update(family=13, speed=1.5, distance=4.0, sensor_delay=2, command_delay=2, max_steps=30)
    elif variant == "sensor_period2":   # a frame every other tick, one frame of delay
        kw.update(sensor_period=2, sensor_delay=1, command_delay=1)
    if variant == "guided_memory":
        kw.update(geometry_memory=1)
    D = 184 if variant.startswith("guided") else 181
    say("case: wide closed loop %s hidden=%d N=64 T=%d, two collects" % (variant, hidden, T))
    cfg = config(**kw)
    sim, _, ora = make_pair(cfg, T, epochs=1, minibatch=1024, actor_obs=D)
    lp = LargePPOTrainer(sim, hidden, epochs=1, minibatch=1024)
    ora.set_hidden(hidden)
    actor = lp.get("actor")
    assert np.array_equal(actor, ora.get("actor"))
    exact = ["obs", "critic_obs", "next_critic_obs", "actions", "logp", "rewards", "terminated", "truncated"]
    for rollout in range(2):
        lp.collect()
        sim.sync()
        means = lp.means()
        obs = np.ascontiguousarray(sim.get("obs"), np.float32)
        rows = obs.size // D
        want = np.zeros(rows * 4, np.float32)
        scratch = np.zeros(rows * hidden, np.float32)
        oracle().orc_actor_forward_batch(ptr(actor), ptr(obs), D, hidden, rows, ptr(scratch), ptr(want))
        merr = float(np.abs(means.astype(np.float64) - want).max())
        ora.set_ext_means(means)
        ora.collect()
        ora.set_ext_means(None)
        bad = compare(sim, ora, ENV_BUFFERS + exact, tol=0.0)
        verr = {name: float(np.abs(sim.get(name).astype(np.float64) - ora.get(name)).max())
                for name in ("values", "next_values")}
        say("  collect %d: means max |gpu - fp32| %.3g, values %s, episodes %d" %
            (rollout, merr, verr, int(ora.get("runs")["episodes"].sum())))
        assert not bad, (rollout, bad)
        assert merr <= MEAN_TOL, merr
        assert verr["values"] <= VALUE_TOL and verr["next_values"] <= VALUE_TOL, verr
        # a value at s' whose critic input is the next tick's input is that
        # tick's value at s, bit for bit (the reuse; the last tick's rows and
        # resets are evaluated on their own)
        co = np.ascontiguousarray(sim.get("critic_obs"), np.float32).reshape(T, -1, 32).view(np.uint32)
        nco = np.ascontiguousarray(sim.get("next_critic_obs"), np.float32).reshape(T, -1, 32).view(np.uint32)
        v = np.ascontiguousarray(sim.get("values"), np.float32).reshape(T, -1)
        nv = np.ascontiguousarray(sim.get("next_values"), np.float32).reshape(T, -1)
        same = np.all(nco[:-1] == co[1:], axis=2)
        assert same.any()
        assert np.array_equal(nv[:-1][same].view(np.uint32), v[1:][same].view(np.uint32))
    assert ora.get("runs")["episodes"].sum() > 0
