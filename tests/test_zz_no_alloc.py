"""fa_pi05_denoise_noalloc (the entry point that allocates nothing) against fa_pi05_denoise.

Both run the same kernels; the no-allocation one on the library's static device scratch instead of
a caller workspace. Two calls in a row (the second with a smaller input: fewer prefix keys, fewer
action tokens), each compared with fa_pi05_denoise on the same inputs at the acceptance tolerance
(max-abs <= 2e-2, mean-abs <= 2e-3; in practice the two agree to a few ulp, the exchange parity
bit of each workspace's launch history being the only difference), plus the kernel status read
from the scratch address the call reports, and the size limit.
"""
import ctypes

import numpy as np
import pytest
import torch

from flashact_amd import _lib, pi05
from tests import pi05_case as P

MAX_ABS, MEAN_ABS = 2e-2, 2e-3

pytestmark = pytest.mark.gpu


def _args(c, g, x_t):
    p = g["packed"]
    kc, vc = g["caches"][0]
    a = _lib.Pi05Args()
    a.weight_dtype = _lib.FA_DTYPE_BF16
    a.w1, a.wo, a.w2, a.w3 = (p[k].data_ptr() for k in ("w1", "wo", "w2", "w3"))
    a.mods, a.mod_final = g["mods"].data_ptr(), g["mod_final"].data_ptr()
    a.rope_cos, a.rope_sin = g["cos"].data_ptr(), g["sin"].data_ptr()
    a.w_ain, a.b_ain = g["w_ain"].data_ptr(), g["b_ain"].data_ptr()
    a.w_aout, a.b_aout = g["w_aout"].data_ptr(), g["b_aout"].data_ptr()
    a.kcache, a.vtcache = kc.data_ptr(), vc.data_ptr()
    a.Lp, a.Lmax, a.num_steps, a.Tv = c["Lp"], g["Lmax"], c["S"], c["Tv"]
    a.num_layers, a.batch = c["NL"], 1
    a.x_t, a.xt_rows = x_t.data_ptr(), int(x_t.shape[0])
    return a


def _noalloc(c, g, gpu):
    L = _lib.lib()
    x_t = c["inp"]["noise"][0].to(gpu).clone()
    a = _args(c, g, x_t)
    scratch = ctypes.c_void_p(0)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    _lib.check(L.fa_pi05_denoise_noalloc(ctypes.byref(a), ctypes.c_void_p(stream), ctypes.byref(scratch)),
               "fa_pi05_denoise_noalloc")
    torch.cuda.synchronize(gpu)
    st = ctypes.c_uint(7)
    _lib.check(L.fa_pi05_read_status(scratch, ctypes.byref(st)), "fa_pi05_read_status")
    return x_t.cpu().numpy(), scratch.value, st.value


def test_noalloc_matches_workspace_entry_point(gpu):
    seen = []
    for NL, Lp, Tv, S, seed in ((2, 968, 50, 2, 51), (2, 300, 10, 2, 52)):  # the second call is smaller
        c = P.make_case(NL=NL, Lp=Lp, Tv=Tv, S=S, seed=seed)
        g = P.gpu_tensors(c, gpu)
        out, scratch, status = _noalloc(c, g, gpu)
        ref = P.run_gpu(c, gpu, g)[0]  # fa_pi05_denoise with the cached caller workspace
        st = P.parity(out[:Tv], ref[:Tv])
        print(f"noalloc vs fa_pi05_denoise NL={NL} Lp={Lp} Tv={Tv} S={S}: {st} status={status}", flush=True)
        assert status == 0 and scratch != 0
        assert np.isfinite(out).all()
        assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st
        seen.append(scratch)
    assert seen[0] == seen[1], "one scratch per device"


def test_noalloc_on_fp16_caches(gpu):
    """The reference's cache type at batch 1 (cache_dtype F16): no shadow is needed, so the entry point
    that allocates nothing serves it; output and suffix cache rows equal fa_pi05_denoise's on copies of
    the same fp16 caches (two calls, the second smaller)."""
    L = _lib.lib()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    for NL, Lp, Tv, S, seed in ((2, 968, 50, 2, 61), (1, 200, 10, 2, 62)):
        c = P.make_case(NL=NL, Lp=Lp, Tv=Tv, S=S, seed=seed)
        g = P.gpu_tensors(c, gpu)
        kb, vb = g["caches"][0]
        runs = []
        for noalloc in (True, False):
            kh, vh = kb.to(torch.float16).contiguous(), vb.to(torch.float16).contiguous()
            x_t = c["inp"]["noise"][0].to(gpu).clone()
            a = _args(c, g, x_t)
            a.kcache, a.vtcache = kh.data_ptr(), vh.data_ptr()
            a.cache_dtype = _lib.FA_DTYPE_F16
            if noalloc:
                scratch = ctypes.c_void_p(0)
                _lib.check(L.fa_pi05_denoise_noalloc(ctypes.byref(a), ctypes.c_void_p(stream), ctypes.byref(scratch)),
                           "fa_pi05_denoise_noalloc")
            else:
                ws = pi05.workspace(gpu)
                a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
                _lib.check(L.fa_pi05_denoise(ctypes.byref(a), ctypes.c_void_p(stream)), "fa_pi05_denoise")
            torch.cuda.synchronize(gpu)
            if noalloc:
                st = ctypes.c_uint(7)
                _lib.check(L.fa_pi05_read_status(scratch, ctypes.byref(st)), "fa_pi05_read_status")
                assert st.value == 0
            runs.append((x_t.cpu().numpy(), kh.cpu(), vh.cpu()))
        (o1, k1, v1), (o2, k2, v2) = runs
        st = P.parity(o1[:Tv], o2[:Tv])
        print(f"noalloc vs fa_pi05_denoise on fp16 caches NL={NL} Lp={Lp} Tv={Tv} S={S}: {st}", flush=True)
        assert np.isfinite(o1).all()
        assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st
        assert torch.equal(k1[:, :Lp], k2[:, :Lp]) and torch.equal(v1[:, :, :Lp], v2[:, :, :Lp])
        for a1, a2 in ((k1[:, Lp:Lp + Tv].float(), k2[:, Lp:Lp + Tv].float()),
                       (v1[:, :, Lp:Lp + Tv].float(), v2[:, :, Lp:Lp + Tv].float())):
            assert torch.count_nonzero(a1) == a1.numel()
            assert float((a1 - a2).abs().max()) <= 0.02 * float(a2.abs().max()) + 1e-3


def test_noalloc_rejects_requests_beyond_its_scratch(gpu):
    L = _lib.lib()
    c = P.make_case(NL=1, Lp=50, Tv=50, S=1, seed=1)
    g = P.gpu_tensors(c, gpu)
    x_t = torch.zeros(16, 50, 32, device=gpu)
    a = _args(c, g, x_t[0])
    a.batch, a.Lmax = 16, 1024  # a batch-16 workspace is ~58 MiB
    rc = L.fa_pi05_denoise_noalloc(ctypes.byref(a), None, None)
    assert rc == 1 and b"static scratch holds" in L.fa_last_error()
    a = _args(c, g, x_t[0])
    a.workspace, a.workspace_bytes = 1 << 20, 1 << 20
    rc = L.fa_pi05_denoise_noalloc(ctypes.byref(a), None, None)
    assert rc == 1 and b"workspace must be NULL" in L.fa_last_error()
