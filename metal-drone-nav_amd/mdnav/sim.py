"""Host classes mirroring the reference's API over the HIP library.

* ``Sim``        — main.mm:516-603 (``Sim(Metal&, SimConfig, horizon)``,
  ``set_config``, ``reset``, ``collect``, ``report`` and the shared buffers).
* ``PPOTrainer`` — main.mm:1110-1474 (``PPOTrainer(Sim&, epochs)``,
  ``rollout_update``, ``metric_mean``, ``optimizer_step``).
* ``Trainer``    — cpu_reference.hpp:112-615 (``Trainer(cfg, horizon, raptor,
  physics)``, ``run(rollouts) -> Metrics``, public buffers), here running on
  the GPU: a drop-in for callers of the CPU trainer's interface.

The reference reads buffers through ``MTLBuffer.contents``; here ``get``/``set``
copy them in the reference's host layouts.  Errors raise ``MdnError`` where
the reference's ``require`` throws ``std::runtime_error``.
"""
import ctypes
import os
import time

import numpy as np

from . import abi
from .native import KERNELS, MdnError, P, check, contiguous, lib, ptr

ASSETS = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "assets")


def load_raptor(path=None):
    """The frozen RAPTOR controller (raptor.hpp:25-40; main.mm:126)."""
    return abi.load_raptor(path or os.path.join(ASSETS, "raptor.bin"))


def crazyflie_params():
    """rl_physics_crazyflie_default (physics.hpp:184-219)."""
    p = np.zeros((), abi.PHYSICS_PARAMS)
    pos = [.028, -.028, 0, -.028, -.028, 0, -.028, .028, 0, .028, .028, 0]
    tz = [-1, 1, -1, 1]
    for r in range(4):
        i = 3 * r
        p["rotor_positions"][i:i + 2] = pos[i:i + 2]
        p["rotor_thrust_directions"][i + 2] = 1.0
        p["rotor_torque_directions"][i + 2] = tz[r]
        p["rotor_thrust_coefficients"][i:i + 3] = [0.00352526, 0.01437313, 0.09223048]
        p["rotor_torque_constants"][r] = 4.665e-3
        p["rotor_time_constants_rising"][r] = 0.05545454545454546
        p["rotor_time_constants_falling"][r] = 0.24939393939393945
    diag = [9.416556729130406e-6, 9.644051701582312e-6, 1.745951732253285e-5]
    inv = [106195.93007988465, 103690.85846314249, 57275.35197719487]
    for i in range(3):
        p["inertia"][4 * i] = diag[i]
        p["inertia_inverse"][4 * i] = inv[i]
    p["gravity_world"][2] = -9.81
    p["mass"] = np.float32(np.float32(np.float32(np.float32(0.027) + np.float32(0.0017)) + np.float32(0.0003))
                           + np.float32(0.0016))
    p["action_min"], p["action_max"], p["dt"] = 0.0, 1.0, 0.01
    p["position_limit"] = p["velocity_limit"] = p["angular_velocity_limit"] = 100000.0
    return p


class Sim:
    """Batched simulator handle (Sim, main.mm:516-603)."""

    def __init__(self, cfg, horizon, raptor=None, physics=None, lanes=8, actor_obs=181):
        L = lib()
        self.cfg = np.array(cfg, abi.SIM_CONFIG)
        self.horizon = int(horizon)
        self._raptor = np.array(load_raptor() if raptor is None else raptor, abi.RAPTOR_WEIGHTS)
        self._physics = np.array(crazyflie_params() if physics is None else physics, abi.PHYSICS_PARAMS)
        h = ctypes.c_void_p()
        check(L.mdn_sim_create(ptr(self.cfg), self.horizon, ptr(self._raptor), ptr(self._physics),
                               ctypes.byref(h)))
        self.h = h
        self.ppo = None
        if lanes != 8:
            check(L.mdn_sim_set_lanes(self.h, lanes))
        if actor_obs != 181:
            self.set_actor_obs(actor_obs)

    @property
    def n(self):
        return int(self.cfg["n"])

    def close(self):
        if getattr(self, "h", None):
            lib().mdn_sim_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def set_config(self, cfg):
        c = np.array(cfg, abi.SIM_CONFIG)
        check(lib().mdn_sim_set_config(self.h, ptr(c)))
        self.cfg = c

    def set_lanes(self, lanes):
        check(lib().mdn_sim_set_lanes(self.h, lanes))

    def set_actor_obs(self, d):
        """Actor inputs: 181, or 184 with the geometry-prior hint
        (FIXED_PPO_ACTOR_OBS_DIM, ppo.hpp:11-34).  Fresh policy."""
        check(lib().mdn_sim_set_actor_obs(self.h, d))

    @property
    def actor_obs(self):
        d = ctypes.c_uint32()
        check(lib().mdn_sim_get_actor_obs(self.h, ctypes.byref(d)))
        return d.value

    def set_camera(self, profile):
        """Camera profile: abi.CAMERA_LEGACY (1) or abi.CAMERA_NATIVE (2)
        (sensor_profile.hpp:16-25, 111-126)."""
        check(lib().mdn_sim_set_camera(self.h, int(profile)))

    @property
    def camera(self):
        c = np.zeros((), abi.CAMERA_PROFILE)
        check(lib().mdn_sim_get_camera(self.h, c.ctypes.data_as(ctypes.c_void_p)))
        return c

    def set_runtime(self, runtime):
        """Episode dynamics variation (NavigationRuntimeConfig,
        navigation_runtime.hpp:9-14); takes effect at the next reset."""
        r = np.array(runtime, abi.RUNTIME_CONFIG)
        check(lib().mdn_sim_set_runtime(self.h, r.ctypes.data_as(ctypes.c_void_p)))

    def set_tasks(self, tasks):
        """Goal-conditioned navigation tasks (NavigationTaskControl,
        navigation_tasks.hpp:93-95); take effect at the next reset."""
        t = np.array(tasks, abi.TASK_CONTROL)
        check(lib().mdn_sim_set_tasks(self.h, t.ctypes.data_as(ctypes.c_void_p)))

    def set_bank(self, worlds, schedule):
        """Frozen challenge bank (main.mm:2175-2178): WORLD records and an
        env-major schedule [N][stride] of level ids (abi.BANK_REHEARSAL for
        a generated rehearsal world); an empty bank disables it."""
        w = np.ascontiguousarray(worlds, abi.WORLD).reshape(-1)
        sch = np.ascontiguousarray(schedule, np.uint32)
        if w.size and (sch.ndim != 2 or sch.shape[0] != int(self.cfg["n"])):
            raise MdnError("bank schedule must be [n_envs][stride], got shape %s" % (sch.shape,))
        stride = int(sch.shape[-1]) if sch.size else 0
        check(lib().mdn_sim_set_bank(self.h, w.ctypes.data_as(ctypes.c_void_p), w.size,
                                     sch.ctypes.data_as(ctypes.c_void_p), stride))

    def reset(self):
        check(lib().mdn_sim_reset(self.h))
        return self.sync()

    def validate_rollout(self):
        """navigation_training::validate_rollout (navigation_training.hpp:27-35):
        raises MdnError naming the first env whose task is not valid and
        ready or whose plant mass is not finite and positive."""
        check(lib().mdn_sim_validate_rollout(self.h))

    def collect(self, count=0):
        """Enqueue ``count`` ticks (0 = horizon); returns immediately."""
        check(lib().mdn_sim_collect(self.h, count))

    def sync(self):
        """Metal::finish: wait, return GPU seconds since the previous sync."""
        s = ctypes.c_double()
        check(lib().mdn_sim_sync(self.h, ctypes.byref(s)))
        return s.value

    def _bytes(self, bid):
        b = ctypes.c_uint64()
        check(lib().mdn_sim_buffer_bytes(self.h, bid, ctypes.byref(b)))
        return b.value

    def get(self, name):
        bid, dtype = abi.BUFFERS[name]
        nbytes = self._bytes(bid)
        out = np.zeros(nbytes // np.dtype(dtype).itemsize, dtype)
        check(lib().mdn_sim_download(self.h, bid, ptr(out), nbytes))
        return out

    def set(self, name, values):
        bid, dtype = abi.BUFFERS[name]
        nbytes = self._bytes(bid)
        arr = contiguous(values, dtype).reshape(-1)
        if arr.nbytes != nbytes:
            raise MdnError("upload of %s needs %d bytes, got %d" % (name, nbytes, arr.nbytes))
        check(lib().mdn_sim_upload(self.h, bid, ptr(arr), nbytes))

    # timing of individual kernels (HIP events on the sim's stream)
    def set_timing(self, on=True):
        check(lib().mdn_sim_set_timing(self.h, 1 if on else 0))

    def reset_timing(self):
        check(lib().mdn_sim_reset_timing(self.h))

    def kernel_time(self, name):
        ms, n = ctypes.c_double(), ctypes.c_uint64()
        check(lib().mdn_sim_kernel_time(self.h, KERNELS[name], ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value

    def report(self, label="", wall=0.0):
        """Sim::report (main.mm:599-602) as a dict of episode statistics."""
        r = self.get("runs")
        ep = int(r["episodes"].sum())
        succ = int(r["successes"].sum())
        tot = float(r["total_elapsed"].astype(np.float64).sum())
        return dict(label=label, episodes=ep, success=succ / ep if ep else 0.0,
                    collision=int(r["collisions"].sum()) / ep if ep else 0.0,
                    timeout=int(r["timeouts"].sum()) / ep if ep else 0.0,
                    progress=float(r["final_progress"].astype(np.float64).sum()) / ep if ep else 0.0,
                    mean_goal_time=float(r["success_time"].astype(np.float64).sum()) / succ if succ else 0.0,
                    mean_speed=float(r["total_path"].astype(np.float64).sum()) / tot if tot else 0.0,
                    peak_speed=float(r["peak_speed"].max()), min_clearance=float(r["min_clearance"].min()),
                    wall_s=wall)


class PPOTrainer:
    """Optimiser over a Sim's rollout (PPOTrainer, main.mm:1110-1474)."""

    def __init__(self, sim, epochs=2, minibatch=256):
        h = ctypes.c_void_p()
        check(lib().mdn_ppo_create(sim.h, epochs, minibatch, ctypes.byref(h)))
        self.h = h
        self.sim = sim
        sim.ppo = self
        self.epochs = epochs
        self.minibatch = minibatch

    def close(self):
        if getattr(self, "h", None):
            lib().mdn_ppo_destroy(self.h)
            self.h = None

    def __del__(self):
        # the Sim destroys its trainer with itself; only free if still attached
        if getattr(self, "h", None) and getattr(self.sim, "h", None):
            self.close()

    def rollout_update(self, rollout_index):
        check(lib().mdn_ppo_rollout_update(self.h, rollout_index))

    def gae(self):
        check(lib().mdn_ppo_gae(self.h))

    def normalize(self):
        check(lib().mdn_ppo_normalize(self.h))

    def update(self, rollout_index):
        check(lib().mdn_ppo_update(self.h, rollout_index))

    def metric_mean(self):
        out = np.zeros(4, np.float32)
        check(lib().mdn_ppo_metric_mean(self.h, ptr(out)))
        return out

    def grad_norm_summary(self):
        """PPOTrainer::grad_norm_summary (main.mm:1443-1465): mean, max and
        clipped fraction of the last update's pre-clip gradient norms; raises
        on a non-finite norm."""
        out = abi.GradNormSummary()
        check(lib().mdn_ppo_grad_norm_summary(self.h, ctypes.byref(out)))
        return out

    @property
    def optimizer_step(self):
        s = ctypes.c_uint64()
        check(lib().mdn_ppo_optimizer_step(self.h, ctypes.byref(s)))
        return s.value

    @property
    def updates_per_rollout(self):
        u = ctypes.c_uint32()
        check(lib().mdn_ppo_updates_per_rollout(self.h, ctypes.byref(u)))
        return u.value

    def save_checkpoint(self, path, family, seed, completed_rollouts):
        """PPOTrainer::save_checkpoint (main.mm:1285-1317): PPOFIX1 version 6, 8
        with the dynamics/task blocks when per-episode plants or tasks are on,
        10 with the native camera."""
        check(lib().mdn_ppo_save_checkpoint(self.h, str(path).encode(), family, seed, completed_rollouts))

    def load_checkpoint(self, path, family, horizon, n, seed):
        """PPOTrainer::load_checkpoint (main.mm:1218-1284), versions 3-10 (a
        shaping block must be the disabled one; version 10's camera contract
        must be this simulator's).  Returns the completed rollouts (0 when the
        file is absent)."""
        done = ctypes.c_uint32()
        check(lib().mdn_ppo_load_checkpoint(self.h, str(path).encode(), family, horizon, n, seed, ctypes.byref(done)))
        return done.value


class LargePPOTrainer:
    """PPO with the hidden width raised to `hidden` (ppo.hpp FIXED_PPO_HIDDEN_DIM;
    5120 gives the reference's capacity actor): bf16 matrix-core GEMMs with
    fp32 master weights and Adam, on the rollout buffers of `sim`."""

    PARAMS = {"actor": 0, "critic": 1, "actor_m": 2, "actor_v": 3, "critic_m": 4, "critic_v": 5}

    def __init__(self, sim, hidden=5120, epochs=4, minibatch=32768):
        self.sim = sim
        self.hidden = hidden
        h = P()
        check(lib().mdn_lppo_create(sim.h, hidden, epochs, minibatch, ctypes.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().mdn_lppo_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def evaluate(self):
        """logp of the stored actions and values at s and s' under this policy."""
        check(lib().mdn_lppo_evaluate(self.h))

    def collect(self, count=0):
        """Sim::collect with this policy acting every tick (0 = horizon ticks);
        values at s and s' from this critic."""
        check(lib().mdn_lppo_collect(self.h, count))

    def means(self):
        """Actor means [rows][4] of the last collect or evaluate."""
        out = np.zeros(self.sim.horizon * self.sim.n * 4, np.float32)
        check(lib().mdn_lppo_means(self.h, ptr(out), out.size))
        return out

    def rollout_update(self, rollout_index):
        check(lib().mdn_lppo_rollout_update(self.h, rollout_index))

    def get(self, name):
        which = self.PARAMS[name]
        n = ctypes.c_uint64()
        check(lib().mdn_lppo_param_count(self.h, which, ctypes.byref(n)))
        out = np.zeros(n.value, np.float32)
        check(lib().mdn_lppo_get_params(self.h, which, ptr(out), n.value))
        return out

    def set(self, name, values):
        which = self.PARAMS[name]
        v = contiguous(values, np.float32)
        check(lib().mdn_lppo_set_params(self.h, which, ptr(v), v.size))

    def metric_mean(self):
        out = np.zeros(4, np.float32)
        check(lib().mdn_lppo_metric_mean(self.h, ptr(out)))
        return out

    def grad_norm_summary(self):
        """PPOTrainer::grad_norm_summary (main.mm:1443-1465) of the wide policy."""
        out = abi.GradNormSummary()
        check(lib().mdn_lppo_grad_norm_summary(self.h, ctypes.byref(out)))
        return out

    @property
    def optimizer_step(self):
        s = ctypes.c_uint64()
        check(lib().mdn_lppo_optimizer_step(self.h, ctypes.byref(s)))
        return s.value


class Trainer:
    """cpu_reference::Trainer interface (cpu_reference.hpp:112-615) on the GPU."""

    def __init__(self, cfg, horizon, raptor=None, physics=None, epochs=2, minibatch=256, lanes=8, actor_obs=181):
        self.sim = Sim(cfg, horizon, raptor, physics, lanes=lanes, actor_obs=actor_obs)
        self.ppo = PPOTrainer(self.sim, epochs, minibatch)
        self.horizon = horizon

    def run(self, rollouts):
        """Trainer::run (cpu_reference.hpp:163-185): rollout + GAE + update."""
        start = time.perf_counter()
        for r in range(rollouts):
            self.sim.collect()
            self.ppo.rollout_update(r)
        self.sim.sync()
        wall = time.perf_counter() - start
        runs = self.sim.get("runs")
        m = self.ppo.metric_mean()
        metrics = abi.Metrics()
        metrics.wall_seconds = wall
        metrics.updates = self.ppo.optimizer_step
        for f in ("episodes", "successes", "collisions", "timeouts"):
            setattr(metrics, f, int(runs[f].sum()))
        for f in ("final_progress", "total_path", "total_elapsed", "success_time"):
            setattr(metrics, f, float(runs[f].astype(np.float64).sum()))
        metrics.policy_loss, metrics.value_loss, metrics.entropy_loss, metrics.ratio = (float(x) for x in m)
        return metrics

    def validate_batched_forward(self, tolerance=2.0e-5):
        """Trainer::validate_batched_forward (cpu_reference.hpp:187-208): the
        batched GPU forward of the current actor and critic over three
        synthetic rows (obs[i] = 0.2 sin(0.0037 i), critic obs[i] =
        0.3 cos(0.17 i)) against a row-by-row evaluation of ppo.hpp:65-93
        (float64 here); True when every hidden activation, mean and value
        agrees within `tolerance`."""
        from . import ops
        d = int(self.sim.actor_obs)
        actor = self.sim.get("actor").astype(np.float64)
        critic = self.sim.get("critic").astype(np.float64)
        obs = (0.2 * np.sin(np.arange(3 * d, dtype=np.float32) * np.float32(0.0037))).astype(np.float32)
        co = (0.3 * np.cos(np.arange(3 * 32, dtype=np.float32) * np.float32(0.17))).astype(np.float32)
        obs, co = obs.reshape(3, d), co.reshape(3, 32)
        ah, am = ops.actor_forward(actor.astype(np.float32), obs)
        ch, cv = ops.critic_forward(critic.astype(np.float32), co)
        H = 64
        w1, b1 = actor[:H * d].reshape(H, d), actor[H * d:H * d + H]
        w2, b2 = actor[H * d + H:H * d + 5 * H].reshape(4, H), actor[H * d + 5 * H:H * d + 5 * H + 4]
        h = np.tanh(obs.astype(np.float64) @ w1.T + b1)
        mean = h @ w2.T + b2
        if d == 184:  # the geometry-prior hint of the 184-input actor (ppo.hpp:77)
            mean[:, :3] += obs[:, d - 3:]
        cw1, cb1 = critic[:H * 32].reshape(H, 32), critic[H * 32:H * 33]
        cw2, cb2 = critic[H * 33:H * 34], critic[H * 34]
        hc = np.tanh(co.astype(np.float64) @ cw1.T + cb1)
        value = hc @ cw2 + cb2
        err = max(np.abs(h - ah).max(), np.abs(mean - am).max(), np.abs(hc - ch).max(), np.abs(value - cv).max())
        return bool(err <= tolerance)

    def get(self, name):
        return self.sim.get(name)

    def set(self, name, values):
        self.sim.set(name, values)
