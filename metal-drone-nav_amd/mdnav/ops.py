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


# ---------------------------------------------------------------- fixed_ppo operators (ppo.hpp:65-324)
def _need(name, arr, size):
    """The C call reads exactly `size` floats of `arr`: refuse any other size
    before it reads past a numpy buffer."""
    if arr.size != size:
        raise ValueError("%s has %d values, expected %d" % (name, arr.size, size))


def actor_forward(params, obs, hidden_dim=64):
    """fixed_ppo::actor_forward over rows of obs[batch][D]: (hidden, means)."""
    x = contiguous(obs, np.float32)
    x = x.reshape(-1, x.shape[-1])
    w = contiguous(params, np.float32).reshape(-1)
    _need("actor params", w, hidden_dim * x.shape[1] + 5 * hidden_dim + 8)
    h = np.zeros((len(x), hidden_dim), np.float32)
    m = np.zeros((len(x), 4), np.float32)
    check(lib().mdn_op_actor_forward(ptr(w), x.shape[1], hidden_dim, ptr(x), len(x), ptr(h), ptr(m)))
    return h, m


def critic_forward(params, obs, hidden_dim=64):
    """fixed_ppo::critic_forward over rows of obs[batch][D]: (hidden, values)."""
    x = contiguous(obs, np.float32)
    x = x.reshape(-1, x.shape[-1])
    w = contiguous(params, np.float32).reshape(-1)
    _need("critic params", w, hidden_dim * x.shape[1] + 2 * hidden_dim + 1)
    h = np.zeros((len(x), hidden_dim), np.float32)
    v = np.zeros(len(x), np.float32)
    check(lib().mdn_op_critic_forward(ptr(w), x.shape[1], hidden_dim, ptr(x), len(x), ptr(h), ptr(v)))
    return h, v


def _log_std(log_std, rows):
    """A shared [4] log-std (stride 0) or one per row [rows][4] (stride 4)."""
    ls = contiguous(log_std, np.float32)
    if ls.size != 4 and ls.size != 4 * rows:
        raise ValueError("log_std has %d values, expected 4 or %d" % (ls.size, 4 * rows))
    return ls.reshape(-1), (0 if ls.size == 4 else 4)


def gaussian_log_prob(actions, means, log_std):
    a = contiguous(actions, np.float32).reshape(-1, 4)
    m = contiguous(means, np.float32).reshape(-1, 4)
    _need("means", m, a.size)
    ls, stride = _log_std(log_std, len(a))
    out = np.zeros(len(a), np.float32)
    check(lib().mdn_op_gaussian_log_prob(ptr(a), ptr(m), ptr(ls), stride, len(a), ptr(out)))
    return out


def sample_loss_and_grad(actions, means, log_std, old_logp, values, advantages, returns, batch_size,
                         clip=0.2, value_coef=0.5, entropy_coef=0.005, old_values=None):
    """fixed_ppo::sample_loss_and_grad per row: (d_mean, d_log_std, d_value,
    losses[policy, value, entropy, ratio])."""
    a = contiguous(actions, np.float32).reshape(-1, 4)
    b = len(a)
    m = contiguous(means, np.float32).reshape(-1, 4)
    _need("means", m, a.size)
    ls, stride = _log_std(log_std, b)
    ol, v, adv, ret = (contiguous(x, np.float32).reshape(-1) for x in (old_logp, values, advantages, returns))
    ov = v if old_values is None else contiguous(old_values, np.float32).reshape(-1)
    for name, x in (("old_logp", ol), ("values", v), ("advantages", adv), ("returns", ret), ("old_values", ov)):
        _need(name, x, b)
    dm, dl = np.zeros((b, 4), np.float32), np.zeros((b, 4), np.float32)
    dv, loss = np.zeros(b, np.float32), np.zeros((b, 4), np.float32)
    check(lib().mdn_op_sample_loss_and_grad(ptr(a), ptr(m), ptr(ls), stride, ptr(ol), ptr(ov), ptr(v), ptr(adv),
                                            ptr(ret), b, batch_size, clip, value_coef, entropy_coef, ptr(dm),
                                            ptr(dl), ptr(dv), ptr(loss)))
    return dm, dl, dv, loss


def adam_update(params, grad, first, second, step, lr, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0):
    """fixed_ppo::adam_update; returns updated (params, first, second) copies."""
    p, g, m, v = (contiguous(x, np.float32).reshape(-1).copy() for x in (params, grad, first, second))
    for name, x in (("grad", g), ("first", m), ("second", v)):
        _need(name, x, p.size)
    check(lib().mdn_op_adam_update(ptr(p), ptr(g), ptr(m), ptr(v), len(p), step, lr, beta1, beta2, eps,
                                   weight_decay))
    return p, m, v


def ppo_self_tests(tolerance=2e-3):
    """fixed_ppo::run_cpu_self_tests through the GPU operators."""
    ok = ctypes.c_int(0)
    check(lib().mdn_op_ppo_self_tests(tolerance, ctypes.byref(ok)))
    return bool(ok.value)
