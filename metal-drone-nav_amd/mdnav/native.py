"""ctypes binding of lib/libmdnav.so (include/mdnav.h).

Loading fails loudly: there is no CPU fallback behind this module.
"""
import ctypes
import os

import numpy as np

from . import abi

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG, "lib", "libmdnav.so")
EXPORTS = [
    "mdn_last_error", "mdn_version", "mdn_sim_create", "mdn_sim_destroy", "mdn_sim_set_config",
    "mdn_sim_get_config", "mdn_sim_reset", "mdn_sim_collect", "mdn_sim_sync", "mdn_sim_buffer_bytes",
    "mdn_sim_download", "mdn_sim_upload", "mdn_sim_set_timing", "mdn_sim_kernel_time",
    "mdn_sim_reset_timing", "mdn_sim_set_lanes", "mdn_sim_set_actor_obs", "mdn_sim_get_actor_obs",
    "mdn_ppo_create", "mdn_ppo_destroy",
    "mdn_ppo_rollout_update", "mdn_ppo_gae", "mdn_ppo_normalize", "mdn_ppo_update",
    "mdn_ppo_metric_mean", "mdn_ppo_optimizer_step", "mdn_ppo_updates_per_rollout",
    "mdn_op_physics_step", "mdn_op_raptor_sequence", "mdn_op_ray_world", "mdn_op_clearance",
    "mdn_op_gae", "mdn_op_normalize", "mdn_lppo_create", "mdn_lppo_destroy", "mdn_lppo_evaluate",
    "mdn_lppo_rollout_update", "mdn_lppo_param_count", "mdn_lppo_get_params", "mdn_lppo_set_params",
    "mdn_lppo_metric_mean", "mdn_lppo_optimizer_step", "mdn_lppo_collect", "mdn_lppo_means",
    "mdn_op_check_division", "mdn_ppo_save_checkpoint", "mdn_ppo_load_checkpoint", "mdn_checkpoint_read",
    "mdn_navpol_read", "mdn_navpol_write", "mdn_fnv1a64_file", "mdn_sim_set_runtime", "mdn_sim_get_runtime",
    "mdn_sim_set_tasks", "mdn_sim_get_tasks", "mdn_task_default_config", "mdn_domain_stress_range", "mdn_sim_set_bank", "mdn_navwid_read",
    "mdn_navwid_write", "mdn_op_actor_forward", "mdn_op_critic_forward", "mdn_op_gaussian_log_prob",
    "mdn_op_sample_loss_and_grad", "mdn_op_adam_update", "mdn_op_ppo_self_tests", "mdn_sim_validate_rollout",
    "mdn_checkpoint_read_params", "mdn_op_normalize_noalloc", "mdn_sim_get_bank", "mdn_sim_set_camera",
    "mdn_sim_get_camera", "mdn_ppo_grad_norm_summary", "mdn_lppo_grad_norm_summary",
]

P = ctypes.c_void_p
U32, U64, F32, I32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_int
KERNELS = {"rollout": 0, "gae": 1, "normalize": 2, "rows": 3, "grads": 4, "adam": 5, "lp_forward": 6,
           "lp_backward": 7, "lp_adam": 8, "memory": 9, "episode": 10}

_lib = None


class MdnError(RuntimeError):
    """A non-zero status of the C ABI (the reference's require() failures)."""


def _sig(lib, name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError("libmdnav.so is not built (%s); run __graft_entry__.build()" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        _sig(L, "mdn_last_error", ctypes.c_char_p)
        _sig(L, "mdn_version", ctypes.c_char_p)
        _sig(L, "mdn_sim_create", I32, P, U32, P, P, ctypes.POINTER(P))
        _sig(L, "mdn_sim_destroy", None, P)
        _sig(L, "mdn_sim_set_config", I32, P, P)
        _sig(L, "mdn_sim_get_config", I32, P, P, ctypes.POINTER(U32))
        _sig(L, "mdn_sim_reset", I32, P)
        _sig(L, "mdn_sim_collect", I32, P, U32)
        _sig(L, "mdn_sim_sync", I32, P, ctypes.POINTER(ctypes.c_double))
        _sig(L, "mdn_sim_buffer_bytes", I32, P, U32, ctypes.POINTER(U64))
        _sig(L, "mdn_sim_download", I32, P, U32, P, U64)
        _sig(L, "mdn_sim_upload", I32, P, U32, P, U64)
        _sig(L, "mdn_sim_set_timing", I32, P, I32)
        _sig(L, "mdn_sim_kernel_time", I32, P, U32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(U64))
        _sig(L, "mdn_sim_reset_timing", I32, P)
        _sig(L, "mdn_sim_set_lanes", I32, P, U32)
        _sig(L, "mdn_sim_set_actor_obs", I32, P, U32)
        _sig(L, "mdn_ppo_save_checkpoint", I32, P, ctypes.c_char_p, U32, U32, U32)
        _sig(L, "mdn_ppo_load_checkpoint", I32, P, ctypes.c_char_p, U32, U32, U32, U32, ctypes.POINTER(U32))
        _sig(L, "mdn_checkpoint_read", I32, ctypes.c_char_p, P, P, U64)
        _sig(L, "mdn_navpol_read", I32, ctypes.c_char_p, P, P, U64, ctypes.POINTER(U64))
        _sig(L, "mdn_navpol_write", I32, ctypes.c_char_p, P, P, U64, U64)
        _sig(L, "mdn_fnv1a64_file", I32, ctypes.c_char_p, ctypes.POINTER(U64))
        _sig(L, "mdn_sim_get_actor_obs", I32, P, ctypes.POINTER(U32))
        _sig(L, "mdn_sim_set_camera", I32, P, U32)
        _sig(L, "mdn_sim_get_camera", I32, P, P)
        _sig(L, "mdn_sim_set_runtime", I32, P, P)
        _sig(L, "mdn_sim_get_runtime", I32, P, P)
        _sig(L, "mdn_sim_set_tasks", I32, P, P)
        _sig(L, "mdn_sim_get_tasks", I32, P, P)
        _sig(L, "mdn_task_default_config", I32, U32, U32, F32, P)
        _sig(L, "mdn_domain_stress_range", I32, P)
        _sig(L, "mdn_sim_set_bank", I32, P, P, U32, P, U32)
        _sig(L, "mdn_navwid_read", I32, ctypes.c_char_p, P, P, P, U64, ctypes.POINTER(U64))
        _sig(L, "mdn_navwid_write", I32, ctypes.c_char_p, P, P, P, U64, U64)
        _sig(L, "mdn_ppo_create", I32, P, U32, U32, ctypes.POINTER(P))
        _sig(L, "mdn_ppo_destroy", None, P)
        _sig(L, "mdn_ppo_rollout_update", I32, P, U32)
        _sig(L, "mdn_ppo_gae", I32, P)
        _sig(L, "mdn_ppo_normalize", I32, P)
        _sig(L, "mdn_ppo_update", I32, P, U32)
        _sig(L, "mdn_ppo_metric_mean", I32, P, P)
        _sig(L, "mdn_ppo_optimizer_step", I32, P, ctypes.POINTER(U64))
        _sig(L, "mdn_ppo_updates_per_rollout", I32, P, ctypes.POINTER(U32))
        _sig(L, "mdn_lppo_create", I32, P, U32, U32, U32, ctypes.POINTER(P))
        _sig(L, "mdn_lppo_destroy", None, P)
        _sig(L, "mdn_lppo_evaluate", I32, P)
        _sig(L, "mdn_lppo_collect", I32, P, U32)
        _sig(L, "mdn_op_check_division", I32, P, U32, P)
        _sig(L, "mdn_lppo_means", I32, P, P, U64)
        _sig(L, "mdn_lppo_rollout_update", I32, P, U32)
        _sig(L, "mdn_lppo_param_count", I32, P, U32, ctypes.POINTER(U64))
        _sig(L, "mdn_lppo_get_params", I32, P, U32, P, U64)
        _sig(L, "mdn_lppo_set_params", I32, P, U32, P, U64)
        _sig(L, "mdn_lppo_metric_mean", I32, P, P)
        _sig(L, "mdn_lppo_optimizer_step", I32, P, ctypes.POINTER(U64))
        _sig(L, "mdn_op_physics_step", I32, P, P, P, P, P, U64)
        _sig(L, "mdn_op_raptor_sequence", I32, P, P, U32, U32, P, P)
        _sig(L, "mdn_op_ray_world", I32, P, P, P, U32, P, U64)
        _sig(L, "mdn_op_clearance", I32, P, P, P, P, U64)
        _sig(L, "mdn_op_gae", I32, U32, U32, P, P, P, P, P, F32, F32, P, P)
        _sig(L, "mdn_op_normalize", I32, P, U64, F32)
        _sig(L, "mdn_op_actor_forward", I32, P, U32, U32, P, U64, P, P)
        _sig(L, "mdn_op_critic_forward", I32, P, U32, U32, P, U64, P, P)
        _sig(L, "mdn_op_gaussian_log_prob", I32, P, P, P, U32, U64, P)
        _sig(L, "mdn_op_sample_loss_and_grad", I32, P, P, P, U32, P, P, P, P, P, U64, F32, F32, F32, F32,
             P, P, P, P)
        _sig(L, "mdn_op_adam_update", I32, P, P, P, P, U64, U64, F32, F32, F32, F32, F32)
        _sig(L, "mdn_op_ppo_self_tests", I32, F32, ctypes.POINTER(I32))
        _sig(L, "mdn_sim_validate_rollout", I32, P)
        _sig(L, "mdn_checkpoint_read_params", I32, ctypes.c_char_p, P, P, U64, P, U64)
        _sig(L, "mdn_op_normalize_noalloc", I32, P, U64, F32, P)
        _sig(L, "mdn_sim_get_bank", I32, P, P)
        _sig(L, "mdn_ppo_grad_norm_summary", I32, P, P)
        _sig(L, "mdn_lppo_grad_norm_summary", I32, P, P)
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise MdnError(lib().mdn_last_error().decode() or ("status %d" % rc))


def ptr(a):
    return a.ctypes.data_as(P)


def contiguous(a, dtype):
    return np.ascontiguousarray(np.asarray(a, dtype))
