"""On-disk formats of the reference: PPOFIX1 trainer checkpoints
(main.mm:978-994, 1218-1317) and NAVPOL1 deployed policies
(deployment.hpp:142-205), read and written by the C library."""
import ctypes

import numpy as np

from . import abi
from .native import check, lib, ptr

NAV_POLICY_WEIGHTS = 184 * 64 + 64 + 4 * 64 + 4 + 4  # the 184-64-4 actor (deployment.hpp:26-38)


def _path(path):
    return str(path).encode()


def fnv1a64_file(path):
    """FNV-1a 64 of a file (deployment.hpp:122-136), the NAVPOL1 provenance hash."""
    h = ctypes.c_uint64()
    check(lib().mdn_fnv1a64_file(_path(path), ctypes.byref(h)))
    return h.value


def read_navigation_policy(path):
    """NavigationPolicy::load: (metadata, weights[12104], source_hash)."""
    meta = np.zeros((), abi.NAV_POLICY_META)
    w = np.zeros(NAV_POLICY_WEIGHTS, np.float32)
    h = ctypes.c_uint64()
    check(lib().mdn_navpol_read(_path(path), ptr(meta), ptr(w), w.size, ctypes.byref(h)))
    return meta, w, h.value


def default_navigation_metadata(max_speed=1.5):
    """The metadata the reference's export writes (deployment.hpp:72-86)."""
    m = np.zeros((), abi.NAV_POLICY_META)
    vals = dict(version=1, observation_count=184, hidden_count=64, action_count=4, policy_mode=17,
                weight_count=NAV_POLICY_WEIGHTS, max_speed_mps=max_speed, sensor_rows=16, sensor_columns=20,
                range_max_m=12.0, navigation_period_s=0.05, native_period_s=0.01, memory_frames=8,
                body_frame=0x00554c46)
    for k, v in vals.items():
        m[k] = v
    return m


def write_navigation_policy(path, weights, meta=None, source_hash=0):
    """NavigationPolicy::write_file with the source checkpoint's hash given."""
    meta = default_navigation_metadata() if meta is None else np.array(meta, abi.NAV_POLICY_META)
    w = np.ascontiguousarray(weights, np.float32).reshape(-1)
    check(lib().mdn_navpol_write(_path(path), ptr(meta), ptr(w), w.size, ctypes.c_uint64(source_hash)))


def read_checkpoint(path, actor=True):
    """(header, actor parameters or None) of a PPOFIX1 file, versions 3-10."""
    h = np.zeros((), abi.CHECKPOINT_HEADER)
    check(lib().mdn_checkpoint_read(_path(path), ptr(h), None, 0))
    if not actor:
        return h, None
    a = np.zeros(int(h["actor_count"]), np.float32)
    check(lib().mdn_checkpoint_read(_path(path), ptr(h), ptr(a), a.size))
    return h, a
