"""ctypes bindings of the CPU oracle (oracle/_build/liboracle.so) and of the
reference's own header code compiled into oracle/_ref/libmdnref.so.

Test infrastructure: only tests, __graft_entry__.smoke() and bench.py's
cpu_baseline leg load these libraries, and only as the checker.
"""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "metal-drone-nav_amd"))
from mdnav import abi  # noqa: E402

ORACLE_SO = os.path.join(ROOT, "oracle", "_build", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libmdnref.so")
# the same headers built with FIXED_PPO_ACTOR_OBS_DIM=184 (the guided actor)
REF184_SO = os.path.join(ROOT, "oracle", "_ref", "libmdnref184.so")
GOLDEN = os.path.join(ROOT, "tests", "golden")

P = ctypes.c_void_p
U32, U64, F32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _sig(lib, name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)
    return f


_oracle = None


def oracle():
    global _oracle
    if _oracle is None:
        lib = ctypes.CDLL(ORACLE_SO)
        _sig(lib, "orc_trainer_create", P, P, U32, P, P, U32, U32)
        _sig(lib, "orc_trainer_destroy", None, P)
        _sig(lib, "orc_trainer_collect", None, P, U32)
        _sig(lib, "orc_trainer_gae", None, P)
        _sig(lib, "orc_trainer_normalize", None, P)
        _sig(lib, "orc_trainer_update", None, P, U32)
        _sig(lib, "orc_trainer_iteration", None, P, U32)
        _sig(lib, "orc_trainer_set_config", None, P, P)
        _sig(lib, "orc_trainer_set_hidden", None, P, U32)
        _sig(lib, "orc_trainer_evaluate", None, P)
        _sig(lib, "orc_trainer_set_ext_means", None, P, P)
        _sig(lib, "orc_trainer_set_actor_obs", None, P, U32)
        _sig(lib, "orc_trainer_set_camera", None, P, U32)
        _sig(lib, "orc_camera_rays_tan", None, F32, P)
        _sig(lib, "orc_guidance", None, P, P, P, F32, P, F32, P)
        _sig(lib, "orc_guidance_memory", None, P, P, P, F32, P, F32, P, P, P, U32, U32, P)
        _sig(lib, "orc_memory_clearance", None, P, P, P, P, U32, U32, F32, P)
        _sig(lib, "orc_trainer_minibatch_grads", None, P, U32, U32, P, P, P, P, P, P)
        _sig(lib, "orc_trainer_optimizer_step", U64, P)
        _sig(lib, "orc_trainer_set_optimizer_step", None, P, U64)
        _sig(lib, "orc_trainer_metric_mean", None, P, P)
        _sig(lib, "orc_trainer_buffer", P, P, U32, ctypes.POINTER(U64))
        _sig(lib, "orc_physics_step_batch", None, P, P, P, P, P, U64)
        _sig(lib, "orc_raptor_sequence", None, P, P, U32, P, P)
        _sig(lib, "orc_generate_world", None, P, U32, U32, F32)
        _sig(lib, "orc_ray_world_batch", None, P, P, P, U32, P, U64)
        _sig(lib, "orc_clearance_batch", None, P, P, P, P, U64)
        _sig(lib, "orc_obstacle_center", None, P, U32, F32, P)
        _sig(lib, "orc_atan2_batch", None, P, P, P, U64)
        _sig(lib, "orc_guided_mode_means", None, U32, P, P)
        _sig(lib, "orc_ray_box", F32, P, P, P, P)
        _sig(lib, "orc_ray_sphere", F32, P, P, P, F32)
        _sig(lib, "orc_ray_cylinder", F32, P, P, P, F32, F32)
        _sig(lib, "orc_camera_rays", None, P)
        _sig(lib, "orc_math_batch", None, U32, P, P, U64)
        _sig(lib, "orc_compute_gae", None, U32, U32, P, P, P, P, P, F32, F32, P, P)
        _sig(lib, "orc_normalize_advantages", None, P, U64, F32)
        _sig(lib, "orc_squared_norm", F32, P, U64)
        _sig(lib, "orc_sample_loss_and_grad", None, P, P, P, F32, F32, F32, F32, F32, F32, F32, F32,
             P, P, P, P)
        _sig(lib, "orc_actor_forward_batch", None, P, P, U32, U32, U64, P, P)
        _sig(lib, "orc_critic_forward_batch", None, P, P, U64, P, P)
        _sig(lib, "orc_init_policy", None, P, P)
        _sig(lib, "orc_minibatch_schedule", None, U32, U32, U32, U32, P)
        _sig(lib, "orc_step_reward", F32, F32, F32, F32, F32, ctypes.c_int, ctypes.c_int)
        _sig(lib, "orc_adam_update", None, P, P, P, P, U64, U64, F32, F32, F32, F32, F32)
        _sig(lib, "orc_critic_observation", None, P, P, P, P)
        _sig(lib, "orc_crazyflie_params", None, P)
        _sig(lib, "orc_default_config", None, P)
        _sig(lib, "orc_num_threads", ctypes.c_int)
        _sig(lib, "orc_set_num_threads", None, ctypes.c_int)
        _sig(lib, "orc_trainer_set_runtime", None, P, P)
        _sig(lib, "orc_trainer_set_tasks", None, P, P)
        _sig(lib, "orc_trainer_reset", None, P)
        _sig(lib, "orc_trainer_set_bank", None, P, P, U32, P, U32)
        _sig(lib, "orc_sample_domain", ctypes.c_int, P, ctypes.POINTER(U32), F32, P, P, P)
        _sig(lib, "orc_domain_episode_seed", U32, P, U32, U32, U32)
        _sig(lib, "orc_domain_stress_range", None, P)
        _sig(lib, "orc_task_default_config", ctypes.c_int, P, U32, U32, F32)
        _sig(lib, "orc_task_settings", ctypes.c_int, P, U32, U32)
        _sig(lib, "orc_generate_task", U32, P, P, ctypes.POINTER(U32), P)
        _sig(lib, "orc_task_step", None, P, P, P, P, P, U32, U32, P)
        _oracle = lib
    return _oracle


# the same headers built with clang++ (left-to-right argument evaluation, as
# the reference's Metal compiler)
REFCLANG_SO = os.path.join(ROOT, "oracle", "_ref", "libmdnref_clang.so")


def ref_available(actor_obs=181):
    if actor_obs == "clang":
        return os.path.exists(REFCLANG_SO)
    return os.path.exists(REF_SO if actor_obs == 181 else REF184_SO)


_refs = {}


def ref(actor_obs=181):
    """The reference's headers built for an actor of `actor_obs` inputs."""
    if actor_obs not in _refs:
        lib = ctypes.CDLL(REFCLANG_SO if actor_obs == "clang" else REF_SO if actor_obs == 181 else REF184_SO)
        _sig(lib, "ref_generate_world", None, P, U32, U32, F32)
        _sig(lib, "ref_ray_world_batch", None, P, P, P, U32, P, U64)
        _sig(lib, "ref_clearance_batch", None, P, P, P, P, U64)
        _sig(lib, "ref_obstacle_center", None, P, U32, F32, P)
        _sig(lib, "ref_camera_rays", None, P)
        _sig(lib, "ref_camera_rays_native", None, P)
        _sig(lib, "ref_camera_profile", None, U32, P)
        _sig(lib, "ref_physics_step_batch", None, P, P, P, P, P, U64)
        _sig(lib, "ref_crazyflie_params", None, P)
        _sig(lib, "ref_raptor_sequence", None, P, P, U32, P, P)
        _sig(lib, "ref_raptor_forward", None, P, P, P, P)
        _sig(lib, "ref_raptor_pack_observation", None, P, P, P, P, P, P, P, P, P)
        _sig(lib, "ref_quaternion_matrix", None, P, P)
        _sig(lib, "ref_ppo_self_tests", ctypes.c_int, F32)
        _sig(lib, "ref_actor_param_count", U32)
        _sig(lib, "ref_critic_param_count", U32)
        _sig(lib, "ref_actor_forward", None, P, P, P, P)
        _sig(lib, "ref_critic_forward", F32, P, P, P)
        _sig(lib, "ref_gaussian_log_prob", F32, P, P, P)
        _sig(lib, "ref_compute_gae", None, U32, U32, P, P, P, P, P, F32, F32, P, P)
        _sig(lib, "ref_normalize_advantages", None, P, U64, F32)
        _sig(lib, "ref_sample_loss_and_grad", None, P, P, P, F32, F32, F32, F32, F32, F32, F32, F32, F32,
             P, P, P, P)
        _sig(lib, "ref_actor_critic_grads", None, P, P, P, P, P, P, P, U32, P, P)
        _sig(lib, "ref_adam_update", None, P, P, P, P, U64, U64, F32, F32, F32, F32, F32)
        _sig(lib, "ref_urand", F32, ctypes.POINTER(U32))
        _sig(lib, "ref_guidance", None, P, P, P, F32, P, F32, P)
        _sig(lib, "ref_guidance_memory", None, P, P, P, F32, P, F32, P, P, P, U32, U32, P)
        _sig(lib, "ref_memory_clearance", None, P, P, P, P, U32, U32, F32, P)
        _sig(lib, "ref_sample_domain", ctypes.c_int, P, ctypes.POINTER(U32), F32, P, P, P)
        _sig(lib, "ref_domain_stress_range", None, P)
        _sig(lib, "ref_task_default_config", ctypes.c_int, P, U32, U32, F32)
        _sig(lib, "ref_generate_task", U32, P, P, ctypes.POINTER(U32), P)
        _sig(lib, "ref_task_apply_start", None, P, P)
        _sig(lib, "ref_task_step", None, P, P, P, P, P, U32, U32, P)
        _sig(lib, "ref_navwid_load", ctypes.c_int, ctypes.c_char_p, P, P, ctypes.POINTER(U64), P, U32, P)
        _refs[actor_obs] = lib
    return _refs[actor_obs]


# ---------------------------------------------------------------- fixtures
def physics_fixture():
    """assets/physics.bin (reference.cpp:83-155): params + 512 transitions."""
    data = open(os.path.join(GOLDEN, "physics.bin"), "rb").read()
    assert data[:8] == b"RLPHYS1\x00"
    version, cases, horizon = np.frombuffer(data[8:20], np.uint32)
    assert version == 1
    params = np.frombuffer(data[20:372], abi.PHYSICS_PARAMS)[0].copy()
    rec = np.dtype([("state", abi.PHYSICS_STATE), ("action", np.float32, 4),
                    ("wind", np.float32, 3), ("next", abi.PHYSICS_STATE)])
    n = int(cases) * int(horizon)
    recs = np.frombuffer(data[372:372 + n * rec.itemsize], rec).copy()
    assert 372 + n * rec.itemsize == len(data)
    return params, recs, int(cases), int(horizon)


def raptor_fixture():
    """assets/raptor.bin (export_raptor.py:86-105): weights + official sequence."""
    path = os.path.join(GOLDEN, "raptor.bin")
    weights = abi.load_raptor(path)
    data = open(path, "rb").read()
    off = 16 + 8336
    assert data[off:off + 8] == b"RPFIX1\x00\x00"
    steps, obs_dim, act_dim = np.frombuffer(data[off + 8:off + 20], np.uint32)
    off += 20
    obs = np.frombuffer(data[off:off + 4 * steps * obs_dim], np.float32).reshape(steps, obs_dim).copy()
    off += 4 * steps * obs_dim
    actions = np.frombuffer(data[off:off + 4 * steps * act_dim], np.float32).reshape(steps, act_dim).copy()
    return weights, obs, actions


def crazyflie():
    p = np.zeros((), abi.PHYSICS_PARAMS)
    oracle().orc_crazyflie_params(ptr(p))
    return p


class OracleTrainer:
    """Python face of the oracle's Trainer (cpu_reference::Trainer shape)."""

    def __init__(self, cfg, horizon, raptor, physics=None, epochs=2, minibatch=256):
        self.lib = oracle()
        self.cfg = np.array(cfg, abi.SIM_CONFIG)
        self.raptor = np.array(raptor, abi.RAPTOR_WEIGHTS)
        self.physics = np.array(crazyflie() if physics is None else physics, abi.PHYSICS_PARAMS)
        self.h = self.lib.orc_trainer_create(ptr(self.cfg), horizon, ptr(self.raptor), ptr(self.physics),
                                             epochs, minibatch)
        self.horizon = horizon

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.orc_trainer_destroy(self.h)
            self.h = None

    def buffer(self, name):
        bid, dtype = abi.BUFFERS[name]
        nbytes = U64(0)
        p = self.lib.orc_trainer_buffer(self.h, bid, ctypes.byref(nbytes))
        count = nbytes.value // np.dtype(dtype).itemsize
        if count == 0:
            return np.zeros(0, dtype)
        arr = np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint8)), (nbytes.value,))
        return arr.view(dtype)

    def get(self, name):
        return self.buffer(name).copy()

    def set_runtime(self, runtime):
        self._runtime = np.array(runtime, abi.RUNTIME_CONFIG)
        self.lib.orc_trainer_set_runtime(self.h, ptr(self._runtime))

    def set_tasks(self, tasks):
        self._tasks = np.array(tasks, abi.TASK_CONTROL)
        self.lib.orc_trainer_set_tasks(self.h, ptr(self._tasks))

    def reset(self):
        self.lib.orc_trainer_reset(self.h)

    def set_bank(self, worlds, schedule):
        self._bank_w = np.ascontiguousarray(worlds, abi.WORLD).reshape(-1)
        self._bank_s = np.ascontiguousarray(schedule, np.uint32)
        self.lib.orc_trainer_set_bank(self.h, ptr(self._bank_w), self._bank_w.size, ptr(self._bank_s),
                                      int(self._bank_s.shape[-1]) if self._bank_s.size else 0)

    def set(self, name, values):
        b = self.buffer(name)
        b[...] = np.asarray(values, b.dtype).reshape(b.shape)

    def collect(self, count=0):
        self.lib.orc_trainer_collect(self.h, count)

    def gae(self):
        self.lib.orc_trainer_gae(self.h)

    def normalize(self):
        self.lib.orc_trainer_normalize(self.h)

    def update(self, rollout_index):
        self.lib.orc_trainer_update(self.h, rollout_index)

    def set_hidden(self, hidden):
        """Replace the policy by one of hidden width `hidden` (fresh init)."""
        self.lib.orc_trainer_set_hidden(self.h, hidden)

    def evaluate(self):
        """logp / values / next_values of the stored rollout under the policy."""
        self.lib.orc_trainer_evaluate(self.h)

    def set_camera(self, profile):
        """Camera profile 1 (legacy) or 2 (native), sensor_profile.hpp:111-126."""
        self.lib.orc_trainer_set_camera(self.h, int(profile))

    def set_actor_obs(self, d):
        """Actor input width: 181, or 184 with the geometry-prior hint (fresh policy)."""
        self.lib.orc_trainer_set_actor_obs(self.h, d)

    def set_ext_means(self, means):
        """Means [T*N*4] used by act() in place of the actor (None: the actor)."""
        self._ext_means = None if means is None else np.ascontiguousarray(means, np.float32)
        self.lib.orc_trainer_set_ext_means(self.h, None if means is None else ptr(self._ext_means))

    def iteration(self, rollout_index):
        self.lib.orc_trainer_iteration(self.h, rollout_index)

    def minibatch_grads(self, begin, b):
        ag = np.zeros(self.buffer("actor").size, np.float32)
        cg = np.zeros(self.buffer("critic").size, np.float32)
        row = np.zeros(4, np.float32)
        dm = np.zeros((b, 4), np.float32)
        dls = np.zeros((b, 4), np.float32)
        dv = np.zeros(b, np.float32)
        self.lib.orc_trainer_minibatch_grads(self.h, begin, b, ptr(ag), ptr(cg), ptr(row), ptr(dm), ptr(dls),
                                             ptr(dv))
        return ag, cg, row, dm, dls, dv

    def metric_mean(self):
        out = np.zeros(4, np.float32)
        self.lib.orc_trainer_metric_mean(self.h, ptr(out))
        return out

    @property
    def optimizer_step(self):
        return int(self.lib.orc_trainer_optimizer_step(self.h))

    @optimizer_step.setter
    def optimizer_step(self, step):
        self.lib.orc_trainer_set_optimizer_step(self.h, step)

    def set_config(self, cfg):
        self.cfg = np.array(cfg, abi.SIM_CONFIG)
        self.lib.orc_trainer_set_config(self.h, ptr(self.cfg))

    def load_checkpoint(self, path):
        """A PPOFIX1 version-6 body (main.mm:1302-1306) into the oracle's
        buffers: parsed here with numpy, independently of the library's reader."""
        data = np.fromfile(path, np.uint8)
        h = data[:136].view(abi.CHECKPOINT_HEADER)[0]
        assert h["magic"] == b"PPOFIX1" and h["version"] in (6, 8), (h["magic"], h["version"])
        off = 136
        for name in ("actor", "critic", "actor_m", "actor_v", "critic_m", "critic_v", "states", "runs", "worlds",
                     "sensors", "poses", "commands"):
            buf = self.buffer(name)
            buf.view(np.uint8)[...] = data[off:off + buf.nbytes]
            off += buf.nbytes
        if h["version"] == 8:  # main.mm:1303-1307: runtime, tasks, plants, task states, nominal plant, RAPTOR
            self.set_runtime(data[off:off + 56].view(abi.RUNTIME_CONFIG)[0])
            self.set_tasks(data[off + 56:off + 204].view(abi.TASK_CONTROL)[0])
            off += 204
            for name in ("environment_physics", "task_states"):
                buf = self.buffer(name)
                buf.view(np.uint8)[...] = data[off:off + buf.nbytes]
                off += buf.nbytes
            off += abi.PHYSICS_PARAMS.itemsize + abi.RAPTOR_WEIGHTS.itemsize
        assert off == data.size
        self.set_config(h["config"])
        self.optimizer_step = int(h["optimizer_step"])
        return h


def math_batch(fn, x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros_like(x)
    oracle().orc_math_batch({"exp": 0, "log": 1, "sin": 2, "cos": 3, "tanh": 4, "expm1": 5,
                             "sigmoid": 6}[fn], ptr(x), ptr(y), x.size)
    return y


def task_runtime(amplitude, enabled=1):
    """NavigationRuntimeConfig of the reference's task training and evaluation
    (navigation_training.hpp:20-22): the stress range, seed 0x3f84d5b5."""
    r = np.zeros((), abi.RUNTIME_CONFIG)
    r["enabled"] = enabled
    r["domain_amplitude"] = amplitude
    r["domain_seed"] = abi.TASK_DOMAIN_SEED
    rng = np.zeros((), abi.DOMAIN_RANGE)
    oracle().orc_domain_stress_range(ptr(rng))
    r["domain_range"] = rng
    return r


def task_settings(stage, family):
    """task_settings of navigation_training.hpp:7-14."""
    t = np.zeros((), abi.TASK_CONTROL)
    assert oracle().orc_task_settings(ptr(t), stage, family) == 1
    return t


def task_eval_config(seed, family, mode=17, n=128):
    """SimConfig of navigation_training::evaluate (navigation_training.hpp:68-71)."""
    return abi.default_config(n=n, eval=1, mode=mode, seed=seed, family=family, speed=1.5, distance=8.0,
                              max_steps=400, geometry_memory=1)
