"""Builds libflashact_mi355x.so (HIP kernels + C ABI) in-tree with hipcc for gfx950."""
from __future__ import annotations

import glob
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libflashact_mi355x.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
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


def build(verbose: bool = False) -> str:
    check_sources()
    os.makedirs(LIB_DIR, exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), *sources(), "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{out}")
    if verbose and out.strip():
        print(out, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
