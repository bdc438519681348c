"""sim_evaluate (main.mm:605-614): one evaluation episode per env on the GPU.

128 envs with eval = 1 (each env stops after its first episode), horizon 32,
max_steps ticks (400 for families 14-16, else 200 unless given), the geometry
memory on for memory = 1 or any mode from 13; the actor parameters replace the
simulator's.  Returns the reference's EvalScore (success, collision and
timeout fractions, mean goal time of the successes; 1e9 without one) and the
Sim::report line of the run."""
import ctypes
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


# ---------------------------------------------------------------- navigation tasks
TASK_DOMAIN_SEED = abi.TASK_DOMAIN_SEED


def task_settings(stage, family, generation_version=1):
    """task_settings (navigation_training.hpp:7-14): the stage's default task
    (navigation_task_default_config, difficulty 0.5) with the training's time
    cost, smoothness weight and initial-speed cap."""
    from .native import check, lib
    t = np.zeros((), abi.TASK_CONTROL)
    cfg = np.zeros((), abi.TASK_CONFIG)
    check(lib().mdn_task_default_config(stage, family, F32(0.5), cfg.ctypes.data_as(ctypes.c_void_p)))
    t["enabled"] = 1
    t["config"] = cfg
    t["config"]["time_cost_per_s"] = 0.2
    t["config"]["command_smoothness_weight"] = 0.05
    t["config"]["initial_speed_max_mps"] = 0.5 if stage == 1 else 1.0
    t["config"]["generation_version"] = generation_version
    return t


def task_runtime(amplitude):
    """NavigationRuntimeConfig of navigation_training::configure
    (navigation_training.hpp:20-22): enabled, the stress range, seed 0x3f84d5b5."""
    from .native import check, lib
    if not (np.isfinite(amplitude) and 0.0 <= amplitude <= 1.0):
        raise ValueError("domain amplitude must be 0..1")
    r = np.zeros((), abi.RUNTIME_CONFIG)
    rng = np.zeros((), abi.DOMAIN_RANGE)
    check(lib().mdn_domain_stress_range(rng.ctypes.data_as(ctypes.c_void_p)))
    r["enabled"] = 1
    r["domain_amplitude"] = amplitude
    r["domain_seed"] = TASK_DOMAIN_SEED
    r["domain_range"] = rng
    return r


def task_evaluate(actor, stage, family, amplitude, seed=800001, mode=17, generation_version=1, raptor=None,
                  physics=None):
    """navigation_training::evaluate (navigation_training.hpp:68-117): 128
    goal-conditioned tasks of one stage and family with per-episode plants,
    one episode each over 400 ticks, geometry memory on.  Returns the score
    (success, collision, timeout fractions, mean successful arrival time) and
    per-env rows with the columns of the reference's task CSV."""
    actor = np.ascontiguousarray(actor, np.float32).reshape(-1)
    if actor.size != abi.policy_shape(obs=184)["actor_count"]:
        raise ValueError("task evaluation takes the 184-input guided actor")
    cfg = abi.default_config(n=128, eval=1, mode=mode, seed=seed, family=family, speed=1.5, distance=8.0,
                             max_steps=400, geometry_memory=1)
    settings = task_settings(stage, family, generation_version)
    sim = Sim(cfg, 32, raptor=raptor, physics=physics, actor_obs=184)
    try:
        sim.set_runtime(task_runtime(amplitude))
        sim.set_tasks(settings)
        sim.reset()
        sim.set("actor", actor)
        initial = sim.get("task_states")
        plants = sim.get("environment_physics")
        if not np.all((initial["valid"] == 1) & (initial["generation_status"] == abi.TASK_READY)):
            raise RuntimeError("task generation rejected an env")
        if not np.all(np.isfinite(plants["mass"]) & (plants["mass"] > 0)):
            raise RuntimeError("episode dynamics sample rejected")
        sim.collect(400)
        sim.sync()
        runs, states, final = sim.get("runs"), sim.get("states"), sim.get("task_states")
    finally:
        sim.close()
    if not np.all(runs["episodes"] == 1):
        raise RuntimeError("evaluation must complete exactly one task per environment")
    d = initial["goal_position"] - states["position"]
    error = np.sqrt(((d.astype(np.float32)) ** 2).sum(axis=1, dtype=np.float32))
    speed = np.sqrt((states["linear_velocity"] ** 2).sum(axis=1, dtype=np.float32))
    rows = dict(family=initial["family"], start=initial["start_position"], start_yaw=initial["start_yaw_rad"],
                initial_velocity=initial["start_velocity_world"], goal=initial["goal_position"],
                initial_distance=initial["initial_distance_m"],
                direct_clearance=initial["direct_segment_clearance_m"], witness_length=initial["witness_length_m"],
                mass=plants["mass"], success=runs["successes"], collision=runs["collisions"],
                timeout=runs["timeouts"], time=runs["elapsed"], path=runs["path"], goal_error=error,
                final_speed=speed, hold=final["stable_time_s"], peak_speed=runs["peak_speed"],
                min_clearance=runs["min_clearance"])
    n = float(len(runs))
    successes = float(runs["successes"].sum())
    score = dict(success=successes / n, collision=float(runs["collisions"].sum()) / n,
                 timeout=float(runs["timeouts"].sum()) / n,
                 arrival_time=float(runs["success_time"].astype(np.float64).sum()) / successes if successes else 0.0)
    return score, rows


# ---------------------------------------------------------------- challenge banks
BANK_ENV_STRIDE, BANK_ENV_OFFSET = 747796405, 2891336453  # the reset seed of sim.metal:56


def load_bank(path, split):
    """The levels of one split of a challenge bank (JSONL, schema 1), parsed
    and checked as challenge_evaluation::parse_level does
    (challenge_evaluation.hpp:163-283): families 14-16, the environment seed
    derivation, room bounds, at most 16 obstacles.  Each level carries its
    WWorld record (obstacles, count, family, seed, goal, wind)."""
    import json
    levels = []
    for number, line in enumerate(open(path), 1):
        rec = json.loads(line)
        where = "JSONL line %d" % number
        if rec.get("record_type") != "challenge" or rec.get("schema_version") != 1:
            raise ValueError(where + ": unsupported record")
        if rec["split"] not in ("train", "dev", "final"):
            raise ValueError(where + ": invalid split")
        if rec["split"] != split:
            continue
        family = int(rec["family"])
        if not 14 <= family <= 16:
            raise ValueError(where + ": family must be 14, 15 or 16")
        cfg = rec["sim_config"]
        if int(cfg["family"]) != family or int(cfg["environment_index"]) != int(rec["environment_index"]):
            raise ValueError(where + ": sim_config does not match the record")
        base, index = int(cfg["seed"]), int(rec["environment_index"])
        state = (base + index * BANK_ENV_STRIDE + BANK_ENV_OFFSET) & MASK
        state ^= (state << 13) & MASK
        state ^= state >> 17
        state ^= (state << 5) & MASK
        if state != int(rec["seed"]):
            raise ValueError(where + ": seed does not match the environment seed derivation")
        obstacles = rec["obstacles"]
        if len(obstacles) > 16:
            raise ValueError(where + ": more than 16 obstacles")
        w = np.zeros((), abi.WORLD)
        w["family"] = family
        w["seed"] = int(rec["seed"])
        w["goal"] = np.array(rec["goal"], np.float32)
        w["wind"] = np.array(rec["wind"], np.float32)
        w["count"] = len(obstacles)
        for i, o in enumerate(obstacles):
            if int(o["kind"]) > 2 or min(o["half_extent"]) < 0:
                raise ValueError(where + ": invalid obstacle")
            w["obstacles"][i]["kind"] = int(o["kind"])
            w["obstacles"][i]["center"] = np.array(o["center"], np.float32)
            w["obstacles"][i]["size"] = np.array(o["half_extent"], np.float32)
            w["obstacles"][i]["velocity"] = np.array(o["velocity"], np.float32)
        levels.append(dict(failure_id=rec["failure_id"], family=family, seed=int(rec["seed"]), base_seed=base,
                           environment_index=index, distance=F32(cfg["distance"]), world=w))
    return levels


def bank_evaluate(actor, levels, mode=17, speed=1.5, max_steps=400, velocity_contract=1, geometry_memory=1,
                  raptor=None, physics=None):
    """challenge_evaluation::run (challenge_evaluation.hpp:353-500): batches
    of up to 128 levels, one episode each; the bank's world replaces the
    reset's before any observation, with the level's own reset seed,
    initial distance and reference point.  Returns per-level outcome rows."""
    if mode not in (2, 13, 17):
        raise ValueError("mode must be 2, 13 or 17")
    if not (np.isfinite(speed) and 0 < speed <= 3.0) or not 1 <= max_steps <= 400:
        raise ValueError("speed in (0, 3] and max_steps in 1..400")
    actor = np.ascontiguousarray(actor, np.float32).reshape(-1)
    sizes = {abi.policy_shape(obs=d)["actor_count"]: d for d in (181, 184)}
    if actor.size not in sizes or (mode >= 13 and sizes[actor.size] != 184):
        raise ValueError("guided modes require the 184-input actor")
    rows = []
    for begin in range(0, len(levels), 128):
        batch = levels[begin:begin + 128]
        cfg = abi.default_config(n=len(batch), family=0, mode=mode, seed=batch[0]["seed"], eval=1, speed=speed,
                                 distance=batch[0]["distance"], max_steps=max_steps,
                                 velocity_contract=velocity_contract, geometry_memory=geometry_memory)
        sim = Sim(cfg, 32, raptor=raptor, physics=physics, actor_obs=sizes[actor.size])
        try:
            sim.set("actor", actor)
            worlds, runs = sim.get("worlds"), sim.get("runs")
            for n, lv in enumerate(batch):
                worlds[n] = lv["world"]
                runs[n]["rng"] = (lv["base_seed"] + lv["environment_index"] * BANK_ENV_STRIDE + BANK_ENV_OFFSET) & MASK
                runs[n]["steps"] = 0
                g = lv["world"]["goal"].astype(np.float32)
                dz = F32(g[2] - F32(1.5))
                runs[n]["initial_distance"] = np.sqrt(F32(F32(g[0] * g[0]) + F32(g[1] * g[1])) + F32(dz * dz),
                                                      dtype=np.float32)
                runs[n]["reference_position"] = (0.0, 0.0, 1.5)
            sim.set("worlds", worlds)
            sim.set("runs", runs)
            sim.collect(max_steps)
            sim.sync()
            r = sim.get("runs")
        finally:
            sim.close()
        for n, lv in enumerate(batch):
            if r[n]["episodes"] != 1 or r[n]["successes"] + r[n]["collisions"] + r[n]["timeouts"] != 1:
                raise RuntimeError("level did not produce exactly one terminal outcome: " + lv["failure_id"])
            rows.append(dict(failure_id=lv["failure_id"], success=int(r[n]["successes"]),
                             collision=int(r[n]["collisions"]), timeout=int(r[n]["timeouts"]),
                             progress=float(r[n]["final_progress"]), path=float(r[n]["path"]),
                             elapsed=float(r[n]["elapsed"]), goal_time=float(r[n]["success_time"]),
                             peak_speed=float(r[n]["peak_speed"]), min_clearance=float(r[n]["min_clearance"])))
    return rows


# ---------------------------------------------------------------- controlled threats
F32 = np.float32
MASK = 0xFFFFFFFF


def _urand(state):
    """xorshift32 (13, 17, 5) and its 24-bit uniform (world.hpp:30-31)."""
    state ^= (state << 13) & MASK
    state ^= state >> 17
    state ^= (state << 5) & MASK
    return state, F32(state >> 8) * F32(1.0 / 16777216.0)


def _inside_room(p, margin):
    """threat_inside_room (threat_evaluation.hpp:9-13)."""
    return (p[0] - margin >= F32(-2.0) and p[0] + margin <= F32(14.0) and p[1] - margin >= F32(-5.0) and
            p[1] + margin <= F32(5.0) and p[2] - margin >= F32(0.0) and p[2] + margin <= F32(5.0))


def add_threat_spheres(worlds, seed, kind, drone_speed, threat_speed, nominal_ttc):
    """add_threat_sphere (threat_evaluation.hpp:20-70) for every env n with seed
    seed + n * 747796405: one 0.35 m sphere on a nominal approach (kind 0) or
    lateral-crossing (kind 1) course and the goal moved to (4, 0, 1.5).  The
    clearance checks run on the GPU (ops.clearance = wclearance).  Raises if
    any env's scene starts overlapped or its sphere path leaves the room or
    meets geometry, as the reference's require() does."""
    from . import ops
    worlds = np.array(worlds, abi.WORLD).copy()
    n = len(worlds)
    drone_radius, sphere_radius = F32(0.18), F32(0.35)
    combined = drone_radius + sphere_radius
    drone_speed, threat_speed, nominal_ttc = F32(drone_speed), F32(threat_speed), F32(nominal_ttc)
    if kind not in (0, 1) or drone_speed <= 0 or threat_speed <= 0 or nominal_ttc <= 0 or np.any(worlds["count"] >= 16):
        raise ValueError("invalid threat kind, speeds or time to collision, or a full world")
    candidates = worlds.copy()
    candidates["goal"] = [4.0, 0.0, 1.5]
    start = np.array([0.0, 0.0, 1.5], F32)
    ok = ops.clearance(candidates, np.tile(start, (n, 1)), np.zeros(n, F32)) > 0
    centers, velocities = np.zeros((n, 3), F32), np.zeros((n, 3), F32)
    for e in range(n):
        rng = ((seed + e * 747796405) & MASK) ^ 0x9E3779B9
        if rng == 0:
            rng = 1
        rng, u = _urand(rng)
        lateral = (u - F32(0.5)) * F32(0.20)
        rng, u = _urand(rng)
        vertical = (u - F32(0.5)) * F32(0.16)
        if kind == 0:
            centers[e] = [(drone_speed + threat_speed) * nominal_ttc + combined, lateral, F32(1.5) + vertical]
            velocities[e, 0] = -threat_speed
        else:
            centers[e] = [drone_speed * nominal_ttc, -threat_speed * nominal_ttc + lateral, F32(1.5) + vertical]
            velocities[e, 1] = threat_speed
        c = centers[e]
        d = c - start
        ok[e] &= _inside_room(c, combined) and bool(np.sqrt(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]) > combined)
    for sample in range(9):  # the nominal path against the room and existing geometry
        t = nominal_ttc * (F32(sample) / F32(8.0))
        p = (centers + velocities * t).astype(F32)
        clear = ops.clearance(candidates, p, np.full(n, t, F32))
        for e in range(n):
            ok[e] &= _inside_room(p[e], combined) and bool(clear[e] > sphere_radius)
    if not np.all(ok):
        raise RuntimeError("invalid or overlapping threat scene (envs %s)" % np.flatnonzero(~ok)[:8].tolist())
    for e in range(n):
        i = int(candidates[e]["count"])
        o = candidates[e]["obstacles"][i]
        o["kind"], o["center"], o["size"], o["velocity"] = 1, centers[e], [sphere_radius] * 3, velocities[e]
        candidates[e]["obstacles"][i] = o
        candidates[e]["count"] = i + 1
    return candidates


def evaluate_threat(actor, mode, kind, threat_speed, nominal_ttc, seed=800001, sensor_delay=0, command_delay=0,
                    velocity_contract=1, memory=1, raptor=None, physics=None):
    """evaluate_threat (main.mm:2711-2728): 128 one-episode runs in family-0
    worlds with one controlled threat sphere each, the drone starting at
    1.5 m/s towards a goal 4 m ahead.  Returns the Sim::report dict."""
    if kind not in (0, 1) or sensor_delay > 6 or command_delay > 7:
        raise ValueError("invalid threat kind or delay")
    actor = np.ascontiguousarray(actor, np.float32).reshape(-1)
    sizes = {abi.policy_shape(obs=d)["actor_count"]: d for d in (181, 184)}
    if actor.size not in sizes:
        raise ValueError("threat actor dimensions")
    cfg = abi.default_config(n=128, family=0, mode=mode, eval=1, seed=seed, speed=1.5, distance=4.0,
                             sensor_delay=sensor_delay, command_delay=command_delay,
                             velocity_contract=velocity_contract, geometry_memory=1 if (memory or mode >= 13) else 0)
    sim = Sim(cfg, 32, raptor=raptor, physics=physics, actor_obs=sizes[actor.size])
    sim.set("actor", actor)
    sim.set("worlds", add_threat_spheres(sim.get("worlds"), seed, kind, 1.5, threat_speed, nominal_ttc))
    states, runs = sim.get("states"), sim.get("runs")
    states["linear_velocity"][:, 0] = cfg["speed"]
    runs["desired_velocity"][:, 0] = cfg["speed"]
    runs["previous_nav"][:, 0] = 1.0
    sim.set("states", states)
    sim.set("runs", runs)
    start = time.perf_counter()
    sim.collect(int(cfg["max_steps"]))
    gpu = sim.sync()
    report = sim.report("eval family=0 mode=%d" % mode, time.perf_counter() - start)
    sim.close()
    return dict(report, gpu_s=gpu)
