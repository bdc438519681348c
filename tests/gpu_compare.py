"""Comparison helpers for the GPU parity tests (HIP library vs CPU oracle)."""
import numpy as np

from mdnav import Sim, PPOTrainer, abi
from oracle_lib import OracleTrainer, raptor_fixture

ENV_BUFFERS = ["states", "runs", "worlds", "sensors", "poses", "commands"]
ROW_BUFFERS = ["obs", "critic_obs", "next_critic_obs", "actions", "logp", "values", "rewards", "next_values", "terminated",
               "truncated"]
INT_FIELDS = {"rng", "steps", "successes", "collisions", "timeouts", "episodes", "count", "seed", "family"}


def field_errors(a, b):
    """Max |a-b| per field (structured) or overall; integer fields must match exactly."""
    out = {}
    if a.dtype.names:
        for f in a.dtype.names:
            sub_a, sub_b = a[f], b[f]
            if sub_a.dtype.names:
                for g, v in field_errors(sub_a, sub_b).items():
                    out[f + "." + g] = v
            elif np.issubdtype(sub_a.dtype, np.integer):
                out[f] = float(np.count_nonzero(sub_a != sub_b))
            else:
                out[f] = float(np.max(np.abs(sub_a.astype(np.float64) - sub_b.astype(np.float64)), initial=0.0))
    elif np.issubdtype(a.dtype, np.integer):
        out["_"] = float(np.count_nonzero(a != b))
    else:
        out["_"] = float(np.max(np.abs(a.astype(np.float64) - b.astype(np.float64)), initial=0.0))
    return out


def compare(gpu, ora, names, tol=0.0, int_exact=True):
    """Returns {buffer: {field: error}} for every mismatching field."""
    bad = {}
    for name in names:
        g, o = gpu.get(name), ora.get(name)
        assert g.shape == o.shape and g.dtype == o.dtype, (name, g.shape, o.shape)
        errs = field_errors(g, o)
        worst = {}
        for f, e in errs.items():
            leaf = f.split(".")[-1]
            is_int = leaf in INT_FIELDS or name in ("terminated", "truncated")
            if (is_int and int_exact and e != 0) or (not is_int and e > tol):
                worst[f] = e
        if worst:
            bad[name] = worst
    return bad


def make_pair(cfg, horizon, epochs=2, minibatch=256, lanes=8, actor_obs=181):
    weights = raptor_fixture()[0]
    sim = Sim(cfg, horizon, raptor=weights, lanes=lanes, actor_obs=actor_obs)
    ppo = PPOTrainer(sim, epochs, minibatch)
    ora = OracleTrainer(cfg, horizon, weights, epochs=epochs, minibatch=minibatch)
    if actor_obs != 181:
        ora.set_actor_obs(actor_obs)
    return sim, ppo, ora


def config(**kw):
    return abi.default_config(**kw)
