"""C++ host code calling the engine through its C ABI alone (tests/cabi_driver.cpp, built by
``flashact_amd.build``): no Python binding and no torch between the caller and the kernels.

The test writes a seeded case as raw files, runs the driver as a child process, and compares the
x_t it writes back with the CPU oracle at the acceptance tolerance (max-abs <= 2e-2, mean-abs <= 2e-3);
for pi0.5 it also checks the suffix cache rows against a launch of the same case through ctypes.
"""
import os
import subprocess

import numpy as np
import pytest
import torch

from flashact_amd.build import DRIVER_PATH
from tests import ma2_case as M
from tests import pi05_case as P

MAX_ABS, MEAN_ABS = 2e-2, 2e-3

pytestmark = pytest.mark.gpu


def _write(d, name, t):
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    t.numpy().tofile(os.path.join(d, name + ".bin"))


def _run(args):
    if not os.path.exists(DRIVER_PATH):
        pytest.fail(f"{DRIVER_PATH} is missing: run __graft_entry__.build() first")
    print("cabi_driver", " ".join(str(a) for a in args), flush=True)
    res = subprocess.run([DRIVER_PATH, *map(str, args)], capture_output=True, text=True, timeout=120)
    print(res.stdout.strip(), res.stderr.strip(), flush=True)
    assert res.returncode == 0, res.stderr
    return res.stdout


PI05 = dict(NL=2, Lp=300, Tv=50, S=2, rows=56, seed=31)
MA2 = dict(NL=2, Lk=493, Tv=30, S=2, adim=6, rows=32, seed=32)


def _pi05_files(d):
    c = P.make_case(NL=PI05["NL"], Lp=PI05["Lp"], Tv=PI05["Tv"], S=PI05["S"], seed=PI05["seed"])
    g = P.gpu_tensors(c, "cpu")
    for k in ("w1", "wo", "w2", "w3"):
        _write(d, k, g["packed"][k])
    kc, vc = g["caches"][0]
    x_t = torch.zeros(PI05["rows"], 32)
    x_t[:PI05["Tv"]] = c["inp"]["noise"][0]
    for k, t in (("mods", g["mods"]), ("mod_final", g["mod_final"]), ("rope_cos", g["cos"]), ("rope_sin", g["sin"]),
                 ("w_ain", g["w_ain"]), ("b_ain", g["b_ain"]), ("w_aout", g["w_aout"]), ("b_aout", g["b_aout"]),
                 ("kcache", kc), ("vtcache", vc), ("x_t", x_t)):
        _write(d, k, t)
    return c, g, ["pi05", d, PI05["NL"], PI05["Lp"], PI05["Tv"], PI05["S"], g["Lmax"], PI05["rows"]]


def _ma2_files(d):
    c = M.make_case(NL=MA2["NL"], Lk=MA2["Lk"], Tv=MA2["Tv"], S=MA2["S"], adim=MA2["adim"], seed=MA2["seed"])
    g = M.gpu_tensors(c, "cpu")
    for k, t in zip(("w_qkv", "w_so", "w_cq", "w_co", "w_gu", "w_dn"), g["ws"]):
        _write(d, k, t)
    for k, t in zip(("b_qkv", "b_so", "b_cq", "b_co", "b_gu", "b_dn"), g["bs"]):
        _write(d, k, t)
    x_t = torch.zeros(MA2["rows"], 32)
    x_t[:MA2["Tv"]] = c["inp"]["noise"][0]
    for k, t in (("mods", g["mods"]), ("mod_final", g["mod_final"]), ("rope_cos", g["cos"]), ("rope_sin", g["sin"]),
                 ("w_ain", g["w_ain"]), ("b_ain", g["b_ain"]), ("w_aout", g["w_aout"]), ("b_aout", g["b_aout"]),
                 ("kctx", g["kc"][0]), ("vtctx", g["vt"][0]), ("x_t", x_t)):
        _write(d, k, t)
    return c, g, ["ma2", d, MA2["NL"], MA2["Lk"], g["Lkmax"], MA2["Tv"], MA2["adim"], MA2["S"], MA2["rows"]]


@pytest.fixture(scope="module")
def drivers(tmp_path_factory):
    """Both driver processes run here, before any launch of this test process: a child process's
    cooperative launch is refused by the runtime (hipErrorIllegalState) once its parent process has
    made cooperative launches of its own, so tests/conftest.py also runs this module first. The GPU
    is not touched by this process until both children have finished."""
    import torch as _t
    if _t.cuda.device_count() == 0:
        pytest.skip("no GPU visible (GPU tests run on the MI355X box)")
    out = {}
    for name, make in (("pi05", _pi05_files), ("ma2", _ma2_files)):
        d = str(tmp_path_factory.mktemp(name))
        c, g, args = make(d)
        out[name] = (c, g, d, _run(args))
    return out


def test_cpp_driver_pi05(drivers, gpu):
    c, g, d, stdout = drivers["pi05"]
    Tv, rows, NL = PI05["Tv"], PI05["rows"], PI05["NL"]
    assert "cus=256" in stdout and "coop_max_blocks=256" in stdout
    xo = np.fromfile(os.path.join(d, "x_t.out"), dtype=np.float32).reshape(rows, 32)
    ref = P.run_oracle(c)[0]
    st = P.parity(xo[:Tv], ref)
    print(f"C++ driver pi05 {PI05}: {st}", flush=True)
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st
    assert np.all(xo[Tv:] == 0.0)
    # the same case through the Python binding: identical actions and suffix cache rows
    xg, kg, vg = P.run_gpu(c, gpu, xt_rows=rows)
    assert np.array_equal(xg, xo)
    ko = np.fromfile(os.path.join(d, "kcache.out"), dtype=np.uint16).reshape(NL, g["Lmax"], 256)
    vo = np.fromfile(os.path.join(d, "vtcache.out"), dtype=np.uint16).reshape(NL, 256, g["Lmax"])
    assert np.array_equal(ko, P.u16(kg)) and np.array_equal(vo, P.u16(vg))


def test_cpp_driver_ma2(drivers):
    c, g, d, _ = drivers["ma2"]
    Tv, rows, adim = MA2["Tv"], MA2["rows"], MA2["adim"]
    xo = np.fromfile(os.path.join(d, "x_t.out"), dtype=np.float32).reshape(rows, 32)
    ref = M.run_oracle(c)[0]
    st = M.parity(xo[:Tv], ref, adim)
    print(f"C++ driver ma2 {MA2}: {st}", flush=True)
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st
    assert np.all(xo[Tv:] == 0.0)
    assert np.array_equal(xo[:Tv, adim:], c["inp"]["noise"][0, :, adim:].numpy())


def test_child_after_parent_launch_is_refused_with_a_clear_error(tmp_path, gpu):
    """A child process started after this process has made cooperative launches (every earlier GPU
    test did): where the runtime refuses the child's cooperative launch (hipErrorIllegalState, seen on
    these boxes), fa_last_error() must say why and what to do instead of a bare launch failure. Where
    the runtime allows it, the child simply succeeds. No kernel runs in the refused case."""
    c = P.make_case(NL=1, Lp=40, Tv=10, S=1, seed=3)
    P.run_gpu(c, gpu)  # this process's own cooperative launch, in case this test runs alone
    d = str(tmp_path)
    _, _, args = _pi05_files(d)
    res = subprocess.run([DRIVER_PATH, *map(str, args)], capture_output=True, text=True, timeout=120)
    print("child rc", res.returncode, res.stderr.strip()[-400:], flush=True)
    if res.returncode != 0:
        assert "refused the cooperative launch" in res.stderr and "parent" in res.stderr, res.stderr
