"""The C-ABI library loads on a machine without a GPU and exports every
entry point include/mdnav.h declares (no compute calls here)."""
import ctypes
import os
import re

import numpy as np
import pytest

from mdnav import abi, native
from oracle_lib import crazyflie, oracle, ptr

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header="mdnav.h"):
    text = open(os.path.join(ROOT, "include", header)).read()
    return sorted(set(re.findall(r"\b(mdn_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared()
    assert len(names) >= 30
    lib = ctypes.CDLL(native.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(native.EXPORTS)
    for n in declared("mdnav_calib.h"):
        assert hasattr(lib, n), n
    assert native.lib().mdn_version().decode().startswith("mdnav")


def test_struct_sizes_match_reference_layouts():
    for dt, size in [(abi.PHYSICS_STATE, 68), (abi.PHYSICS_PARAMS, 352), (abi.RAPTOR_WEIGHTS, 8336),
                     (abi.WORLD, 676), (abi.SIM_RUN, 184), (abi.SIM_CONFIG, 84)]:
        assert dt.itemsize == size


def test_python_host_constants_match_oracle():
    from mdnav.sim import crazyflie_params
    assert crazyflie_params().tobytes() == crazyflie().tobytes()
    c = np.zeros((), abi.SIM_CONFIG)
    oracle().orc_default_config(ptr(c))
    assert c.tobytes() == abi.default_config().tobytes()


def test_error_path_without_gpu_call():
    """Argument validation fails before any device work and reports text."""
    lib = native.lib()
    out = ctypes.c_void_p()
    rc = lib.mdn_sim_create(None, 4, None, None, ctypes.byref(out))
    assert rc == -1 and b"null" in lib.mdn_last_error()
    rc = lib.mdn_ppo_create(None, 2, 256, ctypes.byref(out))
    assert rc == -1


def test_operator_wrappers_refuse_wrong_sizes():
    """The fixed_ppo wrappers check every array against the shape the C call
    reads, before any call (no GPU needed): a params vector of another
    layout, a log_std neither shared nor per row, short per-row arrays."""
    import numpy as np
    from mdnav import ops
    obs = np.zeros((3, 181), np.float32)
    with pytest.raises(ValueError, match="actor params"):
        ops.actor_forward(np.zeros(64 * 181 + 5 * 64 + 7, np.float32), obs)
    with pytest.raises(ValueError, match="critic params"):
        ops.critic_forward(np.zeros(64 * 32 + 2 * 64, np.float32), np.zeros((3, 32), np.float32))
    a = np.zeros((5, 4), np.float32)
    with pytest.raises(ValueError, match="log_std"):
        ops.gaussian_log_prob(a, a, np.zeros(6, np.float32))
    with pytest.raises(ValueError, match="means"):
        ops.gaussian_log_prob(a, np.zeros((4, 4), np.float32), np.zeros(4, np.float32))
    with pytest.raises(ValueError, match="advantages"):
        ops.sample_loss_and_grad(a, a, np.zeros(4, np.float32), np.zeros(5), np.zeros(5), np.zeros(4),
                                 np.zeros(5), 5)
    with pytest.raises(ValueError, match="second"):
        ops.adam_update(np.zeros(10), np.zeros(10), np.zeros(10), np.zeros(9), 1, 1e-3)
