"""Builds libflashact_mi355x.so (HIP kernels + C ABI) in-tree with hipcc for gfx950."""
from __future__ import annotations

import concurrent.futures
import glob
import json
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
# litmus tests of the cross-CU / cross-XCD message passing the kernels rely on (tests/litmus_xcd.hip)
LITMUS_SRC = os.path.join(ROOT, "tests", "litmus_xcd.hip")
LITMUS_PATH = os.path.join(ROOT, "tests", "bin", "litmus_xcd")
FABRIC_SRC = os.path.join(ROOT, "tests", "fabric_probe.hip")
FABRIC_PATH = os.path.join(ROOT, "tests", "bin", "fabric_probe")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # keep the compiler from forming packed-fp32 VALU ops (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


# Per-kernel register budget: the build fails when a kernel spills more VGPRs (or uses more scratch
# bytes per lane) than listed here, so a change that pushes a hot loop into scratch is caught at
# build time. Kernels not listed must not spill at all.
RESOURCE_BUDGET = os.path.join(HERE, "resource_budget.json")
RESOURCE_REPORT = os.path.join(LIB_DIR, "resource_usage.json")
_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|VGPRs Spill|SGPRs Spill):\s+(\S+)")


def parse_resource_usage(text: str) -> dict:
    """{kernel symbol: {"vgpr", "agpr", "scratch", "vgpr_spill", "sgpr_spill"}} from the compiler's
    -Rpass-analysis=kernel-resource-usage remarks."""
    keys = {"VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch", "VGPRs Spill": "vgpr_spill",
            "SGPRs Spill": "sgpr_spill"}
    out, cur = {}, None
    for m in _REMARK.finditer(text):
        k, v = m.group(1), m.group(2)
        if k == "Function Name":
            cur = out.setdefault(v, {})
        elif cur is not None:
            cur[keys[k]] = int(v)
    return out


def check_resources(usage: dict) -> list:
    budget = json.load(open(RESOURCE_BUDGET)) if os.path.exists(RESOURCE_BUDGET) else {}
    bad = []
    for name, u in sorted(usage.items()):
        b = budget.get(name, {"vgpr_spill": 0, "scratch": 0})
        if u.get("vgpr_spill", 0) > b["vgpr_spill"] or u.get("scratch", 0) > b["scratch"]:
            bad.append(f"{name}: {u.get('vgpr_spill', 0)} spilled VGPRs / {u.get('scratch', 0)} B scratch per lane "
                       f"> budget {b['vgpr_spill']} / {b['scratch']}")
    return bad


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
    cmd = [hipcc, *HIPCC_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", "-I", os.path.join(ROOT, "include"),
           src, "-o", obj]
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
    usage = {}
    for src, rc, out in results:
        if rc != 0:
            raise RuntimeError(f"hipcc failed on {src} ({rc}):\n{out}")
        usage.update(parse_resource_usage(out))
        rest = "\n".join(l for l in out.splitlines() if "kernel-resource-usage" not in l and not l.startswith(" "))
        if verbose and rest.strip():
            print(rest, file=sys.stderr)
    with open(RESOURCE_REPORT, "w") as f:
        json.dump(usage, f, indent=1, sort_keys=True)
    if verbose:
        for name, u in sorted(usage.items()):
            print(f"{name}: {u.get('vgpr')} VGPR + {u.get('agpr')} AGPR, {u.get('vgpr_spill')} spilled VGPRs, "
                  f"{u.get('scratch')} B scratch per lane, {u.get('sgpr_spill')} spilled SGPRs", file=sys.stderr)
    bad = check_resources(usage)
    if bad:
        raise RuntimeError("register spills above the budget in " + RESOURCE_BUDGET + ":\n  " + "\n  ".join(bad))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, *HIPCC_FLAGS, "-shared", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc link failed ({res.returncode}):\n{out}")
    os.replace(tmp, LIB_PATH)
    build_driver(hipcc)
    build_litmus(hipcc)
    build_probe(hipcc, FABRIC_SRC, FABRIC_PATH)
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


def build_litmus(hipcc: str) -> str:
    return build_probe(hipcc, LITMUS_SRC, LITMUS_PATH)


def build_probe(hipcc: str, src: str, path: str) -> str:
    """A standalone test program (one .hip file, no library) -> tests/bin."""
    os.makedirs(os.path.dirname(path), exist_ok=True)
    tmp = path + ".tmp"
    cmd = [hipcc, *HIPCC_FLAGS, src, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src} ({res.returncode}):\n{res.stdout}{res.stderr}")
    os.replace(tmp, path)
    return path


if __name__ == "__main__":
    print(build(verbose=True))
