"""Stateless operators of the C ABI over numpy arrays: the device versions of
the reference's fixture kernels (main.mm:29-43, 74-81) and ppo_gae /
ppo_normalize_advantages (ppo.metal:279-332)."""
import ctypes

import numpy as np

from . import abi
from .native import check, contiguous, lib, ptr


def physics_step(states, actions, winds, params):
    s = contiguous(states, abi.PHYSICS_STATE).reshape(-1)
    a = contiguous(actions, np.float32).reshape(-1, 4)
    w = contiguous(winds, np.float32).reshape(-1, 3)
    p = np.array(params, abi.PHYSICS_PARAMS)
    out = np.zeros(len(s), abi.PHYSICS_STATE)
    check(lib().mdn_op_physics_step(ptr(s), ptr(a), ptr(w), ptr(p), ptr(out), len(s)))
    return out


def raptor_sequence(weights, obs, copies=1):
    w = np.array(weights, abi.RAPTOR_WEIGHTS)
    o = contiguous(obs, np.float32).reshape(-1, 22)
    steps = o.shape[0]
    actions = np.zeros((copies, steps, 4), np.float32)
    hidden = np.zeros((copies, 16), np.float32)
    check(lib().mdn_op_raptor_sequence(ptr(w), ptr(o), steps, copies, ptr(actions), ptr(hidden)))
    return actions, hidden


def ray_world(worlds, rays, times, rays_per_world):
    w = contiguous(worlds, abi.WORLD).reshape(-1)
    r = contiguous(rays, np.float32).reshape(-1, 6)
    t = contiguous(times, np.float32).reshape(-1)
    out = np.zeros(len(r), np.float32)
    check(lib().mdn_op_ray_world(ptr(w), ptr(r), ptr(t), rays_per_world, ptr(out), len(r)))
    return out


def clearance(worlds, points, times):
    w = contiguous(worlds, abi.WORLD).reshape(-1)
    p = contiguous(points, np.float32).reshape(-1, 3)
    t = contiguous(times, np.float32).reshape(-1)
    out = np.zeros(len(w), np.float32)
    check(lib().mdn_op_clearance(ptr(w), ptr(p), ptr(t), ptr(out), len(w)))
    return out


def gae(horizon, n, rewards, values, next_values, terminated, truncated, gamma=0.99, lam=0.95):
    r, v, nv = (contiguous(x, np.float32).reshape(-1) for x in (rewards, values, next_values))
    te, tr = (contiguous(x, np.uint8).reshape(-1) for x in (terminated, truncated))
    adv = np.zeros(horizon * n, np.float32)
    ret = np.zeros(horizon * n, np.float32)
    check(lib().mdn_op_gae(horizon, n, ptr(r), ptr(v), ptr(nv), ptr(te), ptr(tr), ctypes.c_float(gamma),
                           ctypes.c_float(lam), ptr(adv), ptr(ret)))
    return adv, ret


def normalize(advantages, eps=1e-8):
    a = contiguous(advantages, np.float32).reshape(-1).copy()
    check(lib().mdn_op_normalize(ptr(a), len(a), ctypes.c_float(eps)))
    return a
