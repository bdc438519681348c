"""The C++ façade (include/mdnav.hpp) compiles against the C ABI and links
libmdnav.so; error codes surface as std::runtime_error."""
import os
import subprocess

import pytest

from mdnav import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "cpp", "facade_example.cpp")
EXE = os.path.join(ROOT, "tests", "cpp", "facade_example")


def build_example():
    libdir = os.path.dirname(native.LIB_PATH)
    cmd = ["g++", "-std=c++17", "-O2", "-ffp-contract=off", "-I" + os.path.join(ROOT, "include"), SRC,
           "-L" + libdir, "-lmdnav", "-Wl,-rpath," + libdir, "-o", EXE]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return EXE


def test_facade_compiles_and_reports_usage():
    exe = build_example()
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 2 and "usage" in r.stderr


def test_facade_loads_deployed_policy():
    exe = build_example()
    r = subprocess.run([exe, "--policy", os.path.join(ROOT, "tests", "golden", "navigation.bin")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert "mode=17 observations=184 weights=12104 max_speed=1.50 source=1d991b0048dec80a" in r.stdout, r.stdout
    r = subprocess.run([exe, "--policy", os.path.join(ROOT, "tests", "golden", "raptor.bin")],
                       capture_output=True, text=True)
    assert r.returncode == 1 and "magic mismatch" in r.stderr, r.stderr


@pytest.mark.gpu
def test_facade_trains_on_gpu():
    exe = build_example()
    print("case: facade example 256 envs x 2 rollouts", flush=True)
    r = subprocess.run([exe, os.path.join(ROOT, "tests", "golden", "raptor.bin"), "256", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "updates=128" in r.stdout, r.stdout  # 2 rollouts x 2 epochs x 32 minibatches
