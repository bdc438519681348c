"""sim_evaluate (main.mm:605-614): one evaluation episode per env on the GPU.

128 envs with eval = 1 (each env stops after its first episode), horizon 32,
max_steps ticks (400 for families 14-16, else 200 unless given), the geometry
memory on for memory = 1 or any mode from 13; the actor parameters replace the
simulator's.  Returns the reference's EvalScore (success, collision and
timeout fractions, mean goal time of the successes; 1e9 without one) and the
Sim::report line of the run."""
import time

import numpy as np

from . import abi
from .sim import Sim


def sim_evaluate(family, mode, actor=None, speed=1.0, distance=3.0, seed=700001, sensor_delay=0, wind=0.0,
                 noise=0.0, dropout=0.0, command_delay=0, velocity_contract=1, memory=0, max_steps=0, raptor=None,
                 physics=None):
    if family in (10, 11, 13) and (abs(speed - 1.5) > 1e-6 or abs(distance - 4.0) > 1e-6):
        raise ValueError("flying-threat evaluation requires 1.5 m/s and 4 m goal")
    if not (max_steps == 0 or 1 <= max_steps <= 2000):
        raise ValueError("evaluation episode length unsupported")
    if sensor_delay > 6 or command_delay > 7:
        raise ValueError("delay rings support <=6 sensor frames and <=7 command steps")
    actor_obs = 181
    if actor is not None:
        actor = np.ascontiguousarray(actor, np.float32).reshape(-1)
        sizes = {abi.policy_shape(obs=d)["actor_count"]: d for d in (181, 184)}
        if actor.size not in sizes:
            raise ValueError("actor parameter count %d is neither the 181- nor the 184-input actor" % actor.size)
        actor_obs = sizes[actor.size]
    if mode in (18, 19) and actor_obs != 184:
        raise ValueError("modes 18/19 require a guided checkpoint")
    cfg = abi.default_config(n=128, family=family, mode=mode, eval=1, seed=seed, distance=distance, speed=speed,
                             sensor_delay=sensor_delay, wind=wind, depth_noise=noise, dropout=dropout,
                             command_delay=command_delay, velocity_contract=velocity_contract,
                             geometry_memory=1 if (memory or mode >= 13) else 0,
                             max_steps=max_steps if max_steps else (400 if 14 <= family <= 16 else 200))
    sim = Sim(cfg, 32, raptor=raptor, physics=physics, actor_obs=actor_obs)
    if actor is not None:
        sim.set("actor", actor)
    start = time.perf_counter()
    sim.collect(int(cfg["max_steps"]))
    gpu = sim.sync()
    report = sim.report("eval family=%d mode=%d" % (family, mode), time.perf_counter() - start)
    r = sim.get("runs")
    if not np.all(r["episodes"] == 1):
        raise RuntimeError("eval must finish exactly one episode per seed")
    n = float(len(r))
    success = float(r["successes"].sum())
    score = dict(success=success / n, collision=float(r["collisions"].sum()) / n,
                 timeout=float(r["timeouts"].sum()) / n,
                 goal_time=float(r["success_time"].astype(np.float64).sum()) / success if success else 1e9)
    sim.close()
    return score, dict(report, gpu_s=gpu)
