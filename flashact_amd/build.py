"""Builds libflashact_mi355x.so (HIP kernels + C ABI) in-tree with hipcc for gfx950."""
from __future__ import annotations

import concurrent.futures
import glob
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libflashact_mi355x.so")
# C++ host program that calls the C ABI directly (tests/cabi_driver.cpp), run by the GPU tests
DRIVER_SRC = os.path.join(ROOT, "tests", "cabi_driver.cpp")
DRIVER_PATH = os.path.join(ROOT, "tests", "bin", "cabi_driver")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # keep the compiler from forming packed-fp32 VALU ops (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


# hipcc (ROCm 7.2) evaluates __builtin_bit_cast(T, v[i]) on an ext_vector element as a cast of
# element 0; kernels use as_f32/as_u32 (fa_device.h) instead, and the build rejects the direct form.
BAD_BITCAST = re.compile(r"__builtin_bit_cast\(\s*[\w:]+\s*,\s*[^(),]*\[")


def check_sources() -> None:
    for src in sources() + sorted(glob.glob(os.path.join(HERE, "csrc", "*.h"))):
        for no, line in enumerate(open(src), 1):
            if BAD_BITCAST.search(line.split("//", 1)[0]):
                raise RuntimeError(f"{src}:{no}: __builtin_bit_cast of a vector element is mis-compiled; "
                                   f"use as_f32/as_u32: {line.strip()}")


def sources():
    return sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")))


def _compile(hipcc: str, src: str, obj: str) -> tuple[str, int, str]:
    cmd = [hipcc, *HIPCC_FLAGS, "-c", "-I", os.path.join(ROOT, "include"), src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l)
    return src, res.returncode, out


def build(verbose: bool = False) -> str:
    """Compiles every csrc/*.hip to an object in parallel, then links the shared library."""
    check_sources()
    os.makedirs(LIB_DIR, exist_ok=True)
    obj_dir = os.path.join(LIB_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    srcs = sources()
    objs = [os.path.join(obj_dir, os.path.basename(s) + ".o") for s in srcs]
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16))
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(lambda so: _compile(hipcc, *so), zip(srcs, objs)))
    for src, rc, out in results:
        if rc != 0:
            raise RuntimeError(f"hipcc failed on {src} ({rc}):\n{out}")
        if verbose and out.strip():
            print(out, file=sys.stderr)
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, *HIPCC_FLAGS, "-shared", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc link failed ({res.returncode}):\n{out}")
    os.replace(tmp, LIB_PATH)
    build_driver(hipcc)
    return LIB_PATH


def build_driver(hipcc: str) -> str:
    """Links tests/cabi_driver.cpp against the library (rpath relative to the binary, so the tree can
    move to another machine)."""
    os.makedirs(os.path.dirname(DRIVER_PATH), exist_ok=True)
    rpath = "-Wl,-rpath,$ORIGIN/" + os.path.relpath(LIB_DIR, os.path.dirname(DRIVER_PATH))
    tmp = DRIVER_PATH + ".tmp"
    cmd = [hipcc, "-O2", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"), DRIVER_SRC,
           "-L", LIB_DIR, "-lflashact_mi355x", rpath, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {DRIVER_SRC} ({res.returncode}):\n{res.stdout}{res.stderr}")
    os.replace(tmp, DRIVER_PATH)
    return DRIVER_PATH


if __name__ == "__main__":
    print(build(verbose=True))
