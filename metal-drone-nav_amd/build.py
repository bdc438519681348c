"""Build lib/libmdnav.so (HIP kernels + C ABI) for gfx950 with hipcc.

    python metal-drone-nav_amd/build.py [--jobs J]

Each source compiles to an object in _build/ in parallel, then one shared
library links them.  Contraction stays off (-ffp-contract=off) so device
arithmetic rounds like the CPU oracle; packed FP32 instructions are
disabled.
"""
import argparse
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = ["rollout.hip", "memory.hip", "ppo.hip", "large.hip", "fixtures.hip", "fixed_ppo.hip", "capi.hip"]
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(HERE, "csrc")]
LIB = os.path.join(HERE, "lib", "libmdnav.so")


def _compile(src):
    obj = os.path.join(HERE, "_build", src.replace(".hip", ".o"))
    cmd = [HIPCC] + FLAGS + ["-c", os.path.join(HERE, "csrc", src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s" % (src, r.stderr[-4000:]))
    return obj


def build(jobs=4):
    os.makedirs(os.path.join(HERE, "_build"), exist_ok=True)
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr[-4000:])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    print(build(ap.parse_args().jobs))
    sys.exit(0)
