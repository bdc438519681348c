"""Benchmark: env-steps/sec of the full rollout + PPO update on one MI355X.

Workload (default): 8,192 environments x 128 ticks per iteration, the static
box world of the reference (family 1: 8 boxes per env), its 20x16 depth
camera (12 m range, 2x2-pooled 181-input actor 181->64->4 with 4 log-stds,
32->64->1 critic), RAPTOR + L2F RK4 at 100 Hz with 5 substeps per 20 Hz
action, GAE(0.99, 0.95), then one PPO epoch of 4 minibatches (262,144 rows
each), clip 0.2, Adam 3e-4.  fp32 throughout.  A step is one iteration:
collect all ticks, GAE, normalisation, every minibatch update.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Prints one JSON line.  ``value`` is env-steps/s with every buffer resident in
HBM.  ``roofline`` is for the dominant kernel (the fused rollout kernel),
from HIP-event timing on its own stream; ``cpu_baseline`` times the CPU oracle
(a port of the reference's CPU trainer) on this host on a bounded sample.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "metal-drone-nav_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

# Algorithmic work per env-step (the per-unit figures of the measurement
# plan): env step (5 substeps of RAPTOR + RK4 + clearance, one 320-ray depth
# frame over 8 boxes + room, observation) 117 kFLOP; rollout actor forward
# 24.2 kFLOP; critic at s and s' 8.7 kFLOP.  Bytes: SoA state/run read+write,
# world, one depth frame written, observation rows written: 4.34 KB.
FLOP_ENV_STEP = 117e3 + 24.2e3 + 8.7e3
# The guided (184-input) actor adds the geometry-prior hint: per pooled cell
# goal alignment, 3x3 nearest range and the 3x3 closing-speed risk (~130
# FLOP x 80 cells), and 3 more first-layer inputs (384 FLOP): 10.8 kFLOP.
FLOP_GUIDANCE = 10.8e3
# Geometry-memory hint per env-step: 640 remembered points built (~45 FLOP
# each), 85 candidate sweeps x 640 points (~10 FLOP per pair: along, lateral,
# contact), 85 candidate scores (~60 FLOP): 0.58 MFLOP.
FLOP_MEMORY = 640 * 45 + 85 * 640 * 10 + 85 * 60
BYTES_ENV_STEP = 4.34e3
# The moving-threat mix (4 bounded movers on 8 boxes, or a 10-obstacle
# course) averages 11.5 obstacles per world: 2.5 more per-ray tests (~30 FLOP
# each) over 320 rays, and 2 ring frames re-read per tick with the 100 ms
# sensor delay (SURVEY-style count: R (15 + 30 (K + 1)) per frame).
FLOP_C3_EXTRA = 320 * 30 * 2.5
BYTES_C3_EXTRA = 4 * 320 + 40 * 3.5
# GAE + normalisation: 14 B in + 8 B out (GAE) + 3 passes over advantages.
BYTES_GAE = 22.0
BYTES_NORM = 16.0
PEAK_FP32 = 157.3e12
PEAK_HBM = 8.0e12


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg_kw, horizon, actor_obs=181, target_s=10.0, envs_all=2048, envs_one=256):
    """Bounded sample of the CPU oracle on this host: the workload's world,
    policy, horizon and PPO schedule shape (1 epoch x 4 minibatches) at a
    smaller env count (env-steps/s does not depend on it).  All cores: one
    untimed iteration, then iterations until `target_s` has passed; one
    core: one iteration at `envs_one` envs."""
    from oracle_lib import OracleTrainer, oracle, raptor_fixture
    from mdnav import abi
    lib = oracle()
    all_threads = int(lib.orc_num_threads())

    def run(envs, timed_min_s, warm):
        cfg = abi.default_config(**dict(cfg_kw, n=envs))
        t = OracleTrainer(cfg, horizon, raptor_fixture()[0], epochs=1, minibatch=envs * horizon // 4)
        if actor_obs != 181:
            t.set_actor_obs(actor_obs)
        it = 0
        for _ in range(warm):
            t.iteration(it)
            it += 1
        done, start = 0, time.perf_counter()
        while True:
            t.iteration(it)
            it += 1
            done += 1
            el = time.perf_counter() - start
            if el >= timed_min_s or done >= 16:
                return envs * horizon * done / el, done, el

    value, done, el = run(envs_all, target_s, 1)
    lib.orc_set_num_threads(1)
    try:
        single, done1, el1 = run(envs_one, 0.0, 0)
    finally:
        lib.orc_set_num_threads(all_threads)
    return {"value": value, "unit": "env-steps/s", "cores": all_threads, "kind": "port",
            "single_thread_value": single, "cpu_model": cpu_model(), "host_cpus": os.cpu_count(),
            "sample": "all %d OpenMP threads: %d envs x %d ticks x %d timed iterations after one untimed "
                      "(rollout + GAE + normalisation + 1 epoch x 4 minibatches), %.1f s; one thread: %d envs x "
                      "%d ticks x %d iteration, %.1f s" % (all_threads, envs_all, horizon, done, el, envs_one,
                                                          horizon, done1, el1)}


def calib_copy(nbytes, repeats=3):
    import ctypes
    from mdnav import native
    lib = native.lib()
    lib.mdn_calib_copy.restype = ctypes.c_int
    lib.mdn_calib_copy.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.POINTER(ctypes.c_double)]
    ms = ctypes.c_double()
    rc = lib.mdn_calib_copy(nbytes, repeats, ctypes.byref(ms))
    if rc:
        raise SystemExit("mdn_calib_copy failed: %d" % rc)
    print(json.dumps({"calib_copy_bytes": nbytes, "launches": repeats + 1, "avg_ms": ms.value,
                      "GBps": 2 * nbytes / (ms.value * 1e-3) / 1e9}), flush=True)


TRAFFIC_PROFILE = "profiles/rollout_kernel_pmc_8192x128.md"
MFMA_PROFILES = ("profiles/rollout_chunk_kernels_sq_mfma_8192x128.md",
                 "profiles/wide_policy_kernels_mfma_8192x256_h5120.md")


def profile_values(relpath, prefix):
    """Machine-readable 'prefix<name>: value' lines of a committed rocprofv3
    summary, as {name: value}."""
    out = {}
    try:
        with open(os.path.join(ROOT, relpath)) as f:
            for line in f:
                if line.startswith(prefix) and ":" in line:
                    name, value = line[len(prefix):].split(":", 1)
                    out[name.strip()] = float(value)
    except OSError:
        pass
    return out


def traffic_from_profile():
    """HBM bytes per rollout launch from the committed PMC summary (the line
    'traffic_bytes_per_launch: N'), or None when it is absent."""
    return profile_values(TRAFFIC_PROFILE, "traffic_").get("bytes_per_launch")


def mfma_util(kernels):
    """Matrix-core utilisation per kernel from the committed rocprofv3
    counter summaries (lines 'mfma_util_<kernel>: fraction')."""
    out = {}
    for path in MFMA_PROFILES:
        for name, v in profile_values(path, "mfma_util_").items():
            if name in kernels:
                out[name] = v
    if out:
        out["source"] = ("rocprofv3 MfmaUtil = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 1,024 SIMDs), "
                         "per dispatch of this workload, read from " + " and ".join(MFMA_PROFILES))
    return out


def large_workload(args, hidden=5120, envs=8192, horizon=256, epochs=4, minibatch=32768):
    """Closed-loop rollout with the wide actor choosing every action (split
    ticks: env kernel, wide forward of the tick's rows, env kernel) and wide
    critic values, then the wide-policy PPO update; roofline of the
    wide-policy GEMMs against the dense bf16 matrix-core peak.  The actor is
    the reference's capacity actor: 184 inputs (geometry-prior hint
    included), 5120 hidden units, 967,688 parameters."""
    from mdnav import LargePPOTrainer, Sim, abi
    N, T, D = envs, horizon, args.actor_obs if args.actor_obs_set else 184
    cfg = abi.default_config(n=N, family=1, speed=1.0, distance=3.0)
    log("bench: large workload N=%d T=%d actor %d-%d-4" % (N, T, D, hidden))
    sim = Sim(cfg, T, lanes=args.lanes, actor_obs=D)
    lp = LargePPOTrainer(sim, hidden, epochs, minibatch)
    it = 0
    for _ in range(args.warmup):
        lp.collect()
        lp.rollout_update(it)
        it += 1
    sim.sync()
    sim.set_timing(True)
    sim.reset_timing()
    sim.sync()
    steps = max(1, min(args.steps, 3))
    t0 = time.perf_counter()
    for _ in range(steps):
        lp.collect()
        lp.rollout_update(it)
        it += 1
    gpu_s = sim.sync()
    wall = time.perf_counter() - t0
    kernels = {}
    for name in ("rollout", "gae", "normalize", "lp_forward", "lp_backward", "lp_adam"):
        ms, n = sim.kernel_time(name)
        kernels[name] = {"total_ms": round(ms, 3), "launches": n}
    rows = N * T
    PA = D * hidden + hidden + 4 * hidden + 8
    P = PA + (32 * hidden + 2 * hidden + 1)
    # algorithmic FLOP: rollout 2P per row (actor and critic at s; the critic at s' is the next row's value
    # at s wherever the inputs are equal, and the few rows evaluated on their own, the last tick and resets,
    # are not counted); update per row per epoch: forward 2P, first/second-layer weight gradients 2P (the
    # backward's recomputed forward is not counted)
    flop_eval = 2.0 * rows * P
    flop_fwd = 2.0 * rows * epochs * P
    flop_bwd = 2.0 * rows * epochs * P
    t_fwd = kernels["lp_forward"]["total_ms"] * 1e-3 / steps
    t_bwd = kernels["lp_backward"]["total_ms"] * 1e-3 / steps
    achieved = (flop_eval + flop_fwd + flop_bwd) / (t_fwd + t_bwd)
    out = {
        "metric": "env-steps/sec (rollout+PPO update), wide-policy configuration",
        "value": round(rows * steps / wall, 1), "unit": "env-steps/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": round(wall / steps * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 GEMMs, fp32 weights/Adam",
        "data": "synthetic: seeded procedural worlds (family 1), random-init policies (seed 1789)",
        "config": {"workload": "large actor: %d envs x %d ticks, actor %d-%d-4 (%d parameters) and critic "
                               "32-%d-1, %d epochs x %d minibatches of %d"
                               % (N, T, D, hidden, PA, hidden, epochs, rows // minibatch, minibatch),
                   "behaviour_actions": "wide actor in the loop every tick; wide critic values at s and s'"},
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(achieved / 2.5e15, 4), "traffic": None,
                     "kernel": "wide-policy forward + backward GEMM kernels (bf16 dense peak 2.5 PFLOP/s)",
                     "algorithmic_tflop_per_iteration": round((flop_eval + flop_fwd + flop_bwd) / 1e12, 2)},
        "kernels": kernels, "gpu_seconds": round(gpu_s, 4),
        "mfma_util": mfma_util(("lp_actor_backward", "lp_actor_forward", "lp_critic_backward", "lp_critic_forward")),
        "cpu_baseline": None,
        "cpu_baseline_note": "not run: the CPU update of this workload is about 1e14 FLOP per iteration",
    }
    print(json.dumps(out), flush=True)


def reference_schedule(iters=3):
    """The reference's own GPU benchmark schedule (docs/BENCHMARKS.md:56-67,
    `gpu-bench 8192 3 1`): 8,192 envs x 32 ticks, then 2 epochs of 256-row
    minibatches (2,048 Adam steps per iteration, main.mm:1321-1384), here with
    the pooled 181-input actor.  Wall clock of `iters` iterations after one
    warmup, without per-kernel timing events."""
    from mdnav import PPOTrainer, Sim, abi
    N, T = 8192, 32
    cfg = abi.default_config(n=N, family=1, speed=1.0, distance=3.0)
    sim = Sim(cfg, T, lanes=8, actor_obs=181)
    ppo = PPOTrainer(sim, 2, 256)
    sim.collect()
    ppo.rollout_update(0)
    sim.sync()
    t0 = time.perf_counter()
    for it in range(iters):
        sim.collect()
        ppo.rollout_update(1 + it)
    sim.sync()
    wall = time.perf_counter() - t0
    return {"workload": "8192 envs x 32 ticks, then 2 epochs x 256-row minibatches (2048 Adam steps per iteration), "
                        "actor 181-64-4", "value": round(N * T * iters / wall, 1), "unit": "env-steps/s",
            "ms_per_step": round(wall / iters * 1e3, 3), "iterations": iters,
            "reference_published": {"value": 290.5e3, "unit": "env-steps/s", "hardware": "Apple M3 GPU (Metal)",
                                    "actor": "661-input raw-depth actor", "source": "docs/BENCHMARKS.md:56-67"},
            "note": "the reference's benchmark schedule; the reference's figure is for its 661-input actor, which "
                    "this build does not run, so it is context, not a like-for-like baseline"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--envs", type=int, default=8192)
    ap.add_argument("--horizon", type=int, default=128)
    ap.add_argument("--schedule", choices=["baseline", "reference"], default="baseline",
                    help="baseline: 1 epoch x 4 minibatches; reference: 2 epochs x 256-row minibatches")
    ap.add_argument("--lanes", type=int, default=8)
    ap.add_argument("--actor-obs", type=int, choices=[181, 184], default=None,
                    help="actor inputs: 181 (pooled depth + context) or 184 (plus the geometry-prior hint, "
                         "computed in the env step and added to the first three means); default 181 for the "
                         "small actor, 184 for the large one")
    ap.add_argument("--geometry-memory", action="store_true",
                    help="with the 184-input actor: the history-aware hint (8-frame range and pose rings, 85 "
                         "candidate sweeps) from the memory kernel, one env launch and one memory launch per tick")
    ap.add_argument("--task-training", action="store_true",
                    help="the reference's task training loop (navigation_training.hpp:117-131): stage-2 clutter "
                         "tasks of family 12 with per-episode plants at amplitude 1, mode 22, guided actor with the "
                         "geometry memory, one tick per launch with the per-episode kernel")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-reference-schedule", action="store_true",
                    help="skip the reference-schedule line (its thousands of small launches; for counter passes)")
    ap.add_argument("--workload", choices=["small", "large", "stress", "threats", "c3"], default="small",
                    help="small: 8,192 envs x 128 ticks, 181-64-4 actor (the headline metric); large: 8,192 envs x "
                         "256 ticks, 184-5120-4 actor (967,688 parameters) and 32-5120-1 critic on bf16 matrix cores, "
                         "4 epochs x 64 "
                         "minibatches of 32,768; stress: 65,536 envs x 128 ticks, small actor; threats: 8,192 envs "
                         "x 256 ticks of the reference's moving-threat rehearsal mix (family 13: doorways, tables, "
                         "random families and the two moving-sphere threat families, clean even lanes) with "
                         "100 ms sensor and command delays, small actor; c3: 8,192 envs x 256 ticks of the "
                         "moving-threat mix (env lanes n %% 4: 0-1 eight boxes + four kind-3 bounded movers, 2 the "
                         "same with a long 8-13 m goal, 3 a combined course with a bounded crossing sphere) with "
                         "100 ms sensor and command delays, small actor")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="BYTES",
                    help="run only the plain copy kernel over BYTES (reads BYTES, writes BYTES per launch); "
                         "its FETCH_SIZE/WRITE_SIZE readings scale the rollout kernel's counters to bytes")
    args = ap.parse_args()
    if args.task_training:
        args.actor_obs, args.geometry_memory, args.no_cpu_baseline = 184, True, True
    args.actor_obs_set = args.actor_obs is not None
    if args.actor_obs is None:
        args.actor_obs = 184 if args.geometry_memory else 181
    if args.geometry_memory and args.actor_obs != 184:
        sys.exit("--geometry-memory needs the 184-input actor")
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each GPU box holds one MI355X); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.calib_copy:
        calib_copy(args.calib_copy)
        return
    if args.workload == "large":
        large_workload(args)
        return

    from mdnav import PPOTrainer, Sim, abi
    if args.workload == "stress":
        args.envs, args.horizon, args.no_cpu_baseline = 65536, 128, True
    if args.workload in ("threats", "c3"):
        args.envs, args.horizon = 8192, 256
    N, T = args.envs, args.horizon
    headline = (N, T) == (8192, 128) and args.actor_obs == 181 and not args.geometry_memory and \
        args.workload == "small" and not args.task_training
    epochs, minibatch = (1, N * T // 4) if args.schedule == "baseline" else (2, 256)
    cfg_kw = dict(family=1, speed=1.0, distance=3.0, geometry_memory=1 if args.geometry_memory else 0)
    if args.workload == "threats":  # the reference's threat rehearsal with 100 ms delays (2 ticks at 20 Hz)
        cfg_kw = dict(family=13, speed=1.5, distance=4.0, sensor_delay=2, command_delay=2)
    if args.workload == "c3":  # moving-threat mix: kind-3 movers, long goals, courses; 100 ms delays
        cfg_kw = dict(family=abi.FAMILY_C3_MIX, speed=1.5, distance=4.0, sensor_delay=2, command_delay=2)
    if args.task_training:  # navigation_training.hpp:119-123
        cfg_kw = dict(family=12, mode=22, speed=1.5, distance=8.0, max_steps=400, geometry_memory=1,
                      entropy_coef=0.001, learning_rate=0.0001)
    cfg = abi.default_config(n=N, **cfg_kw)
    log("bench: creating sim N=%d T=%d schedule=%s" % (N, T, args.schedule))
    sim = Sim(cfg, T, lanes=args.lanes, actor_obs=args.actor_obs)
    if args.task_training:
        from mdnav import task_runtime, task_settings
        sim.set_runtime(task_runtime(1.0))
        sim.set_tasks(task_settings(2, 12))
        sim.reset()
    ppo = PPOTrainer(sim, epochs, minibatch)
    it = 0
    for _ in range(args.warmup):
        sim.collect()
        ppo.rollout_update(it)
        it += 1
    sim.sync()
    log("bench: warmup done (%d iterations)" % args.warmup)
    sim.set_timing(True)
    sim.reset_timing()
    sim.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        sim.collect()
        if args.task_training:  # navigation_training.hpp:149-150: reject bad draws before the update
            sim.validate_rollout()
        ppo.rollout_update(it)
        it += 1
    gpu_s = sim.sync()
    t1 = time.perf_counter()
    wall = t1 - t0
    log("bench: timed %d iterations in %.3f s (GPU %.3f s)" % (args.steps, wall, gpu_s))

    kernels = {}
    for name in ("rollout", "memory", "episode", "gae", "normalize", "rows", "grads", "adam"):
        ms, n = sim.kernel_time(name)
        kernels[name] = {"total_ms": round(ms, 4), "launches": n, "avg_ms": round(ms / n, 5) if n else None}
    roll = kernels["rollout"]
    env_steps_launch = N * T
    # one launch per iteration (with the geometry memory: one per tick, timed
    # here per iteration)
    avg_s = roll["total_ms"] * 1e-3 / args.steps
    flop_env_step = FLOP_ENV_STEP + (FLOP_GUIDANCE if args.actor_obs == 184 else 0.0) + \
        (FLOP_C3_EXTRA if args.workload == "c3" else 0.0)
    bytes_env_step = BYTES_ENV_STEP + (BYTES_C3_EXTRA if args.workload == "c3" else 0.0)
    achieved = flop_env_step * env_steps_launch / avg_s
    # VALU-issue bound (SQ counters: VALU busy 53 % of wave cycles, matrix
    # cores 8 %); the fp32 vector and fp32 matrix peaks are both 157.3 TFLOP/s
    roofline = {"bound": "valu", "achieved": round(achieved / 1e12, 3), "peak": 157.3, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP32, 4), "traffic": traffic_from_profile() if headline else None,
                "traffic_unit": ("HBM bytes per launch, from %s (rocprofv3 FETCH_SIZE + WRITE_SIZE of this workload, "
                                 "copy-kernel scaled), not measured in this run" % TRAFFIC_PROFILE),
                "kernel": ("rollout_kernel (fused env step + rollout actor/critic, %d ticks per launch)" % T
                           if not args.geometry_memory else
                           "rollout_kernel (env step + rollout actor/critic, split at the hint: %d ticks in %d "
                           "launches per iteration)" % (T, roll["launches"] // args.steps)),
                "roof_note": "fp32 compute roof: env step on the VALU, policy/critic layers and RAPTOR dense/GRU "
                             "on fp32 MFMA; algorithmic %.1f kFLOP and %.2f KB per env-step x %d env-steps per "
                             "launch" % (flop_env_step / 1e3, bytes_env_step / 1e3, env_steps_launch),
                "hbm_frac_algorithmic": round(bytes_env_step * env_steps_launch / avg_s / PEAK_HBM, 5)}
    secondary = {}
    if kernels["memory"]["launches"]:
        mem_s = kernels["memory"]["total_ms"] * 1e-3 / args.steps
        secondary["memory"] = {"bound": "valu", "achieved_TFLOPs": round(FLOP_MEMORY * N * T / mem_s / 1e12, 3),
                               "frac": round(FLOP_MEMORY * N * T / mem_s / PEAK_FP32, 4),
                               "ms_per_iteration": round(mem_s * 1e3, 3),
                               "note": "%.0f kFLOP per env-step" % (FLOP_MEMORY / 1e3)}
    if kernels["gae"]["launches"]:
        gae_s = kernels["gae"]["avg_ms"] * 1e-3
        secondary["gae"] = {"bound": "hbm", "achieved_GBps": round(BYTES_GAE * N * T / gae_s / 1e9, 1),
                            "frac": round(BYTES_GAE * N * T / gae_s / PEAK_HBM, 4)}
    if kernels["normalize"]["launches"]:
        ns = kernels["normalize"]["avg_ms"] * 1e-3
        secondary["normalize"] = {"bound": "hbm", "achieved_GBps": round(BYTES_NORM * N * T / ns / 1e9, 1),
                                  "frac": round(BYTES_NORM * N * T / ns / PEAK_HBM, 4)}

    value = N * T * args.steps / wall
    family = cfg_kw["family"]
    if args.task_training:
        data = ("synthetic: navigation tasks generated per episode (stage 2 clutter goals, family 12 worlds) with "
                "per-episode plants at amplitude 1, random-init guided policy (seed 1789)")
        workload = ("task training: stage-2 clutter tasks (family 12) with per-episode plants, mode 22, %d envs x "
                    "%d ticks, guided actor 184-64-4 with the geometry-memory hint, %s PPO schedule, "
                    "validate_rollout after every collect" % (N, T, args.schedule))
    elif args.workload == "threats":
        data = ("synthetic: seeded procedural worlds of the reference's threat rehearsal family 13 (per episode: "
                "doorway, table, a random family 0-6, or a moving-sphere threat, families 10/11), random-init policy")
        workload = ("moving-threat rehearsal mix, %d envs x %d ticks, 100 ms sensor and command delays (even envs "
                    "clean), small actor 181-64-4, %s PPO schedule" % (N, T, args.schedule))
    elif args.workload == "c3":
        data = ("synthetic: seeded moving-threat mix per env lane n % 4 (lanes 0-1: family-1 boxes + 4 kind-3 "
                "bounded spheres, r 0.2-0.5 m, peak speed 0.3-1.5 m/s; lane 2: the same with an 8-13 m goal; "
                "lane 3: a combined corridor course with a bounded crossing sphere), random-init policy")
        workload = ("moving-threat mix (kind-3 bounded movers, static/long/course lanes 50/25/25), %d envs x %d "
                    "ticks, 100 ms sensor and command delays, small actor 181-64-4, %s PPO schedule"
                    % (N, T, args.schedule))
    else:
        data = "synthetic: seeded procedural worlds (reference family 1), random-init policy (seed 1789)"
        workload = ("static-box world, %d envs x %d ticks, %s actor %d-64-4%s, %s PPO schedule"
                    % (N, T, "small" if args.actor_obs == 181 else "guided", args.actor_obs,
                       " with the geometry-memory hint" if args.geometry_memory else "", args.schedule))
    out = {
        "metric": ("env-steps/sec (rollout+PPO update) at 8,192 envs; HBM GB/s and MFMA util %" if headline else
                   "env-steps/sec (rollout+PPO update) at %d envs x %d ticks" % (N, T)),
        "value": round(value, 1), "unit": "env-steps/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall / args.steps * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": data,
        "config": {"workload": workload,
                   "envs": N, "horizon": T, "family": family, "rays": 320, "actor": "%d-64-4" % args.actor_obs,
                   "critic": "32-64-1",
                   "epochs": epochs, "minibatch": minibatch, "lanes_per_env": args.lanes,
                   "shapes": "the reference's own: 20x16 = 320 rays, 2x2-pooled %d-input actor, 32-input critic "
                             "(BASELINE's literal 192-ray / 208-input / 64-64 shapes are not a configuration the "
                             "reference builds)" % args.actor_obs,
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "kernels": kernels,
        "secondary_roofline": secondary,
        "mfma_util": mfma_util(("rollout_kernel", "chunk_kernel")) if headline else {},
        "gpu_seconds": round(gpu_s, 4),
    }
    if headline and not args.no_reference_schedule:
        log("bench: reference schedule")
        out["reference_schedule"] = reference_schedule()
    if not args.no_cpu_baseline:
        log("bench: cpu baseline")
        out["cpu_baseline"] = cpu_baseline(cfg_kw, T, actor_obs=args.actor_obs)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
