"""The C-ABI library on the CPU: it loads, exports every symbol include/flashact_mi355x.h declares,
and its argument validation rejects bad requests before touching a device (no kernel launches)."""
import ctypes
import os
import re

import pytest

from flashact_amd import _lib
from flashact_amd.build import LIB_PATH

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flashact_mi355x.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*[A-Za-z_][\w \*]*?\b(fa_\w+)\s*\(", src, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB_PATH):
        from flashact_amd import build
        build.build()
    return _lib.lib()


def test_exports_every_declared_symbol(lib):
    names = _declared()
    assert "fa_pi05_denoise" in names and len(names) >= 8
    so = ctypes.CDLL(LIB_PATH)
    for n in names:
        assert hasattr(so, n), f"{n} declared in the header but not exported"
    assert sorted(n for n, _, _ in _lib.SYMBOLS) == names, "ctypes binding out of sync with the header"


def test_versions_and_sizes(lib):
    assert lib.fa_abi_version() == _lib.ABI_VERSION
    assert lib.fa_pi05_max_batch() >= 1
    ws = lib.fa_pi05_workspace_bytes(1, 50, 1024)
    assert ws > 0 and ws % 256 == 0


def _args(**kw):
    a = _lib.Pi05Args()
    fake = 1 << 20  # aligned dummy addresses: validation must fail before anything is dereferenced
    for f in ("w1", "wo", "w2", "w3", "mods", "mod_final", "rope_cos", "rope_sin", "w_ain", "b_ain", "w_aout",
              "b_aout", "kcache", "vtcache", "x_t", "workspace"):
        setattr(a, f, fake)
    a.Lp, a.Lmax, a.num_steps, a.Tv, a.num_layers, a.batch, a.xt_rows = 968, 1024, 10, 50, 18, 1, 50
    a.workspace_bytes = 1 << 30
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code,text", [
    (dict(Tv=65, xt_rows=65), 1, "Tv"),
    (dict(Tv=0), 1, "Tv"),
    (dict(Lmax=1000), 1, "Lmax"),
    (dict(Lmax=1008), 1, "Lmax"),
    (dict(xt_rows=10), 1, "xt_rows"),
    (dict(workspace_bytes=4096), 1, "workspace"),
    (dict(w2=None), 1, "w2 is NULL"),
    (dict(kcache=(1 << 20) + 8), 1, "kcache is not 16-byte aligned"),
    (dict(srows=4), 1, "kvsrc_k"),
    (dict(srows=900, kvsrc_k=1 << 20, kvsrc_v=1 << 20), 1, "srows=900 < Lp=968"),
    (dict(srows=968, kvsrc_k=(1 << 20) + 2, kvsrc_v=1 << 20), 1, "not 16-byte aligned"),
    (dict(srows=-1), 1, "srows"),
    (dict(weight_dtype=1), 1, "row scales"),
    (dict(weight_dtype=1, s1=1 << 20, so=1 << 20, s2=1 << 20, s3=(1 << 20) + 4), 1, "16-byte aligned"),
    (dict(weight_dtype=1, s1=1 << 20, so=1 << 20, s2=1 << 20, s3=1 << 20, batch=2), 2, "batch 1"),
    (dict(weight_dtype=7), 1, "weight_dtype"),
    (dict(s2=1 << 20), 1, "must be NULL for bf16"),
    (dict(batch=65), 1, "batch"),
    (dict(batch=0), 1, "batch"),
    (dict(batch=16, workspace_bytes=4096), 1, "workspace"),
    (dict(batch=16, trace=1 << 20), 2, "batch 1"),
])
def test_denoise_rejects_bad_requests(lib, kw, code, text):
    rc = lib.fa_pi05_denoise(ctypes.byref(_args(**kw)), None)
    assert rc == code
    assert text in lib.fa_last_error().decode()


def test_denoise_null_args(lib):
    assert lib.fa_pi05_denoise(None, None) == 1
    assert "NULL" in lib.fa_last_error().decode()


def test_denoise_without_device(lib):
    """A valid request on a host without an MI355X fails with FA_ERR_DEVICE and launches nothing."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert lib.fa_pi05_denoise(ctypes.byref(_args()), None) == 3
    assert lib.fa_pi05_denoise(ctypes.byref(_args(batch=16)), None) == 3
    fp8 = _args(weight_dtype=1, s1=1 << 20, so=1 << 20, s2=1 << 20, s3=1 << 20)
    assert lib.fa_pi05_denoise(ctypes.byref(fp8), None) == 3


def test_batched_workspace_sizes(lib):
    """bs >= 2 selects the batched kernel: its workspace grows with batch x Tv and the key range."""
    one = lib.fa_pi05_workspace_bytes(1, 50, 1024)
    b2 = lib.fa_pi05_workspace_bytes(2, 50, 1024)
    b16 = lib.fa_pi05_workspace_bytes(16, 50, 1024)
    assert 0 < b2 < b16 and b16 % 256 == 0 and one > 0
    assert lib.fa_pi05_workspace_bytes(16, 50, 2048) > b16
    assert lib.fa_pi05_workspace_bytes(lib.fa_pi05_max_batch() + 1, 50, 1024) == 0


def _ma2_args(**kw):
    a = _lib.Ma2Args()
    fake = 1 << 20
    for f in ("w_qkv", "w_so", "w_cq", "w_co", "w_gu", "w_dn", "b_qkv", "b_so", "b_cq", "b_co", "b_gu", "b_dn",
              "mods", "mod_final", "rope_cos", "rope_sin", "w_ain", "b_ain", "w_aout", "b_aout", "kctx", "vtctx",
              "x_t", "workspace"):
        setattr(a, f, fake)
    a.Lk, a.Lkmax, a.Tv, a.adim, a.num_steps, a.num_layers, a.batch, a.xt_rows = 493, 496, 30, 6, 10, 36, 1, 32
    a.workspace_bytes = 1 << 30
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code,text", [
    (dict(Tv=65, xt_rows=65), 1, "Tv"),
    (dict(adim=33), 1, "adim"),
    (dict(Lkmax=490), 1, "Lkmax"),
    (dict(Lkmax=500), 1, "Lkmax"),
    (dict(xt_rows=10), 1, "xt_rows"),
    (dict(workspace_bytes=4096), 1, "workspace"),
    (dict(w_gu=None), 1, "w_gu is NULL"),
    (dict(vtctx=(1 << 20) + 4), 1, "vtctx is not 16-byte aligned"),
    (dict(weight_dtype=1), 2, "bf16"),
    (dict(batch=70), 1, "tokens"),
])
def test_ma2_rejects_bad_requests(lib, kw, code, text):
    rc = lib.fa_ma2_flow(ctypes.byref(_ma2_args(**kw)), None)
    assert rc == code
    assert text in lib.fa_last_error().decode()


def test_ma2_without_device(lib):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert lib.fa_ma2_flow(ctypes.byref(_ma2_args()), None) == 3
    assert lib.fa_ma2_flow(ctypes.byref(_ma2_args(batch=16)), None) == 3
    assert lib.fa_ma2_workspace_bytes(1, 30, 496) > 0
    assert lib.fa_ma2_workspace_bytes(16, 30, 496) > lib.fa_ma2_workspace_bytes(1, 30, 496)


def _pf_args(**kw):
    a = _lib.PrefillArgs()
    fake = 1 << 20
    for f in ("wqkv", "wo", "wgu", "wdn", "ln_in", "ln_post", "rope_cos", "rope_sin", "x", "kcache", "vtcache",
              "workspace"):
        setattr(a, f, fake)
    a.Lp, a.Lmax, a.num_layers, a.batch = 968, 1024, 18, 1
    a.workspace_bytes = 1 << 30
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code,text", [
    (dict(Lp=0), 1, "Lp>=1"),
    (dict(Lmax=960), 1, "Lmax"),
    (dict(Lmax=1000), 1, "Lmax"),
    (dict(batch=17), 1, "tokens"),
    (dict(num_layers=0), 1, "num_layers"),
    (dict(workspace_bytes=4096), 1, "workspace"),
    (dict(wgu=None), 1, "wgu is NULL"),
    (dict(x=(1 << 20) + 8), 1, "x is not 16-byte aligned"),
    (dict(workspace=(1 << 20) + 16), 1, "workspace is not 256-byte aligned"),
    (dict(weight_dtype=1), 2, "bf16"),
])
def test_prefill_rejects_bad_requests(lib, kw, code, text):
    rc = lib.fa_pi05_prefill(ctypes.byref(_pf_args(**kw)), None)
    assert rc == code
    assert text in lib.fa_last_error().decode()


def test_prefill_without_device(lib):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert lib.fa_pi05_prefill(ctypes.byref(_pf_args()), None) == 3
    one = lib.fa_pi05_prefill_workspace_bytes(1, 968, 1024)
    assert one > 0 and one % 256 == 0
    assert lib.fa_pi05_prefill_workspace_bytes(4, 968, 1024) > one
    assert lib.fa_pi05_prefill_workspace_bytes(1, 968, 960) == 0
    assert lib.fa_pi05_prefill_workspace_bytes(17, 968, 1024) == 0


def test_resource_report_parses_and_budget_holds():
    """build.py reads each kernel's register use from the compiler's remarks and refuses spills above
    flashact_amd/resource_budget.json; the report of the library built here is within it."""
    import json
    from flashact_amd import build
    text = ("x.hip:1:1: remark: Function Name: _Zk [-Rpass-analysis=kernel-resource-usage]\n"
            "x.hip:1:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]\n"
            "x.hip:1:1: remark:     AGPRs: 12 [-Rpass-analysis=kernel-resource-usage]\n"
            "x.hip:1:1: remark:     ScratchSize [bytes/lane]: 8 [-Rpass-analysis=kernel-resource-usage]\n"
            "x.hip:1:1: remark:     SGPRs Spill: 3 [-Rpass-analysis=kernel-resource-usage]\n"
            "x.hip:1:1: remark:     VGPRs Spill: 2 [-Rpass-analysis=kernel-resource-usage]\n")
    u = build.parse_resource_usage(text)
    assert u == {"_Zk": {"vgpr": 256, "agpr": 12, "scratch": 8, "sgpr_spill": 3, "vgpr_spill": 2}}
    assert build.check_resources(u)  # an unlisted kernel may not spill
    if os.path.exists(build.RESOURCE_REPORT):
        rep = json.load(open(build.RESOURCE_REPORT))
        assert any("pi05_denoise_bs1" in k for k in rep)
        assert build.check_resources(rep) == []
