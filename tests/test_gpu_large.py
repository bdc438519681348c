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


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("hidden", [256, 5120])
def test_wide_policy_against_oracle(hidden):
    say("case: wide policy hidden=%d, N=64 T=32, 1 epoch x 2 minibatches of 1024" % hidden)
    cfg = config(n=64, family=1, speed=1.0, distance=3.0, max_steps=40)
    sim, _, ora = make_pair(cfg, 32, epochs=1, minibatch=1024)
    sim.collect()
    sim.sync()
    ora.collect()
    for name in ("obs", "critic_obs", "next_critic_obs", "actions", "rewards", "terminated", "truncated"):
        assert np.array_equal(sim.get(name), ora.get(name)), name
    lp = LargePPOTrainer(sim, hidden, epochs=1, minibatch=1024)
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
