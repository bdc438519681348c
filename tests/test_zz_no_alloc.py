"""mdn_op_normalize_noalloc, the entry point that allocates nothing: on
device memory it gives mdn_op_normalize's result bit for bit, on two calls
in a row (the second smaller, so stale scratch from the first would show),
and it refuses a count beyond its scratch limit before touching the GPU.

The device buffers are the caller's, made here with the HIP runtime the
library itself links (so one runtime serves the whole process)."""
import ctypes

import numpy as np
import pytest

from mdnav import native, ops

MAX = 1 << 26


def test_noalloc_rejects_oversize():
    lib = native.lib()
    rc = lib.mdn_op_normalize_noalloc(ctypes.c_void_p(16), MAX + 1, 1e-8, None)
    assert rc == -1 and b"scratch limit" in lib.mdn_last_error()
    assert lib.mdn_op_normalize_noalloc(None, 10, 1e-8, None) == -1


def loaded_hip_runtime():
    """Path of the HIP runtime this process mapped when it loaded libmdnav.so
    (from /proc/self/maps), so the test's own HIP calls go to that runtime
    whatever its version suffix."""
    native.lib()
    with open("/proc/self/maps") as f:
        paths = {line.split()[-1] for line in f if "libamdhip64.so" in line}
    assert len(paths) == 1, paths
    return paths.pop()


def hip_runtime():
    hip = ctypes.CDLL(loaded_hip_runtime(), mode=ctypes.RTLD_GLOBAL)
    for name, args in (("hipMalloc", [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]),
                       ("hipFree", [ctypes.c_void_p]),
                       ("hipMemcpy", [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]),
                       ("hipDeviceSynchronize", [])):
        getattr(hip, name).restype = ctypes.c_int
        getattr(hip, name).argtypes = args
    return hip


@pytest.mark.gpu
def test_noalloc_matches_normalize():
    lib = native.lib()
    hip = hip_runtime()
    H2D, D2H = 1, 2
    rng = np.random.default_rng(23)
    for n in (1_048_576 + 77, 30_001):  # the second call is smaller
        print("case: normalize without allocation, %d rows" % n, flush=True)
        a = (rng.normal(0.3, 2.0, n) * rng.uniform(0.1, 3.0, n)).astype(np.float32)
        want = ops.normalize(a)
        dev = ctypes.c_void_p()
        assert hip.hipMalloc(ctypes.byref(dev), a.nbytes) == 0
        try:
            assert hip.hipMemcpy(dev, a.ctypes.data_as(ctypes.c_void_p), a.nbytes, H2D) == 0
            rc = lib.mdn_op_normalize_noalloc(dev, n, ctypes.c_float(1e-8), None)
            assert rc == 0, lib.mdn_last_error()
            assert hip.hipDeviceSynchronize() == 0
            got = np.empty_like(a)
            assert hip.hipMemcpy(got.ctypes.data_as(ctypes.c_void_p), dev, a.nbytes, D2H) == 0
        finally:
            hip.hipFree(dev)
        assert np.array_equal(got, want)
        assert abs(float(got.astype(np.float64).mean())) < 1e-5
