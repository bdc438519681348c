"""On-disk formats of the reference: PPOFIX1 trainer checkpoints
(main.mm:978-994, 1218-1317) and NAVPOL1 deployed policies
(deployment.hpp:142-205), read and written by the C library."""
import ctypes
import os

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


def read_wide_policy(path):
    """WideNavigationPolicy::load (navigation_wide_deployment.hpp:15-40):
    (metadata, camera contract, weights[189 H + 8], source_hash)."""
    meta = np.zeros((), abi.NAV_POLICY_META)
    cam = np.zeros((), abi.SENSOR_CONTRACT)
    check(lib().mdn_navwid_read(_path(path), ptr(meta), ptr(cam), None, 0, None))
    w = np.zeros(int(meta["weight_count"]), np.float32)
    h = ctypes.c_uint64()
    check(lib().mdn_navwid_read(_path(path), ptr(meta), ptr(cam), ptr(w), w.size, ctypes.byref(h)))
    return meta, cam, w, h.value


def export_wide_policy(checkpoint, destination):
    """navigation_export_wide.py:11-69: the 184-H-4 actor of a guided PPOFIX1
    checkpoint (versions 6, 8, 9, 10; mode 17 or 22; 5 substeps, sensor period
    1; body-velocity contract 1 with the geometry memory; the whole actor and
    critic payload present; finite actor weights; an optional
    ``<checkpoint>.train.json`` sidecar must name 184 inputs, width H and the
    camera) as NAVWID4, with the legacy camera (native for version 10) and the
    checkpoint's FNV-1a 64, plus the ``<destination>.json`` provenance record.
    Returns that record."""
    import hashlib
    import json
    import math
    data = open(checkpoint, "rb").read()
    if len(data) < 136 or data[:8] != b"PPOFIX1\0":
        raise ValueError("Expected a PPOFIX1 checkpoint")
    h = np.frombuffer(data[:136], abi.CHECKPOINT_HEADER)[0]
    version, actor_count = int(h["version"]), int(h["actor_count"])
    width, rem = divmod(actor_count - 8, 189)
    if version not in (6, 8, 9, 10) or rem or width not in (64, 256, 768, 2560, 5120):
        raise ValueError("Unsupported guided 184/H/4 actor or checkpoint version")
    c = h["config"]
    if int(c["mode"]) not in (17, 22) or int(c["substeps"]) != 5 or int(c["sensor_period"]) != 1:
        raise ValueError("Unsupported action map or control cadence")
    speed = float(c["speed"])
    if int(c["velocity_contract"]) != 1 or int(c["geometry_memory"]) != 1 or not (math.isfinite(speed) and
                                                                                      0 < speed <= 10):
        raise ValueError("Unsupported body-velocity or geometry-memory contract")
    critic_count = int(h["critic_count"])
    if len(data) < 136 + 4 * (actor_count + critic_count):
        raise ValueError("Truncated actor/critic parameter payload")
    weights = np.frombuffer(data[136:136 + 4 * actor_count], np.float32)
    if not np.all(np.isfinite(weights)):
        raise ValueError("Non-finite actor parameter")
    native = version == 10
    sidecar = str(checkpoint) + ".train.json"
    if os.path.exists(sidecar):
        with open(sidecar) as f:
            contract = json.load(f)
        if contract.get("actor_obs_dim") != 184 or contract.get("actor_hidden_dim") != width:
            raise ValueError("Source architecture sidecar differs")
        if contract.get("sensor_profile") != ("native" if native else "legacy"):
            raise ValueError("Source camera sidecar differs")
    meta = default_navigation_metadata(speed)
    meta["version"], meta["hidden_count"], meta["weight_count"] = 4, width, actor_count
    cam = np.zeros((), abi.SENSOR_CONTRACT)
    cam["profile_id"], cam["tan_h"], cam["tan_v"] = (2 if native else 1), 1.0, (0.8 if native else 0.75)
    cam["mount_x_m"], cam["min_range_m"], cam["max_range_m"] = (0.08 if native else 0.0), 0.03, 12.0
    w = np.ascontiguousarray(weights)
    source_hash = fnv1a64_file(checkpoint)
    check(lib().mdn_navwid_write(_path(destination), ptr(meta), ptr(cam), ptr(w), w.size,
                                 ctypes.c_uint64(source_hash)))
    payload = open(destination, "rb").read()
    record = {
        "schema": "wide-guided-nav-v4", "source": str(checkpoint),
        "source_sha256": hashlib.sha256(data).hexdigest(), "source_fnv1a64": source_hash,
        "source_version": version, "actor_inputs": 184, "actor_hidden": width, "actor_parameters": actor_count,
        "source_critic_parameters": critic_count, "serialized_critic_parameters": 0,
        "sensor_profile": 2 if native else 1, "max_speed_mps": speed,
        "weights_sha256": hashlib.sha256(w.tobytes()).hexdigest(),
        "nav_sha256": hashlib.sha256(payload).hexdigest(), "bytes": len(payload),
        "scope": "Frozen deterministic mode17 actor export; not independent flight proof.",
    }
    with open(str(destination) + ".json", "w") as f:
        f.write(json.dumps(record, indent=2) + "\n")
    return record


def read_checkpoint(path, actor=True):
    """(header, actor parameters or None) of a PPOFIX1 file, versions 3-10."""
    h = np.zeros((), abi.CHECKPOINT_HEADER)
    check(lib().mdn_checkpoint_read(_path(path), ptr(h), None, 0))
    if not actor:
        return h, None
    a = np.zeros(int(h["actor_count"]), np.float32)
    check(lib().mdn_checkpoint_read(_path(path), ptr(h), ptr(a), a.size))
    return h, a


def read_checkpoint_params(path):
    """(header, actor, critic) of a PPOFIX1 file: the vectors that follow the
    header, as navigation_training::load_actor reads them
    (navigation_training.hpp:37-62)."""
    h = np.zeros((), abi.CHECKPOINT_HEADER)
    check(lib().mdn_checkpoint_read_params(_path(path), ptr(h), None, 0, None, 0))
    a = np.zeros(int(h["actor_count"]), np.float32)
    c = np.zeros(int(h["critic_count"]), np.float32)
    check(lib().mdn_checkpoint_read_params(_path(path), ptr(h), ptr(a), a.size, ptr(c), c.size))
    return h, a, c
