"""pi0.5 denoise loop on the MI355X vs the CPU fp32 oracle (parity gate).

Tolerance (the acceptance tolerance for bf16 operands with fp32 accumulation vs the fp32 oracle, on
the final actions): max-abs <= 2e-2 and mean-abs <= 2e-3.
"""
import numpy as np
import pytest
import torch

from tests import pi05_case as P
from flashact_amd import pi05

MAX_ABS, MEAN_ABS = 2e-2, 2e-3

pytestmark = pytest.mark.gpu


def _check(c, gpu, **kw):
    ref = P.run_oracle(c)[0]
    out, kc, vc = P.run_gpu(c, gpu, **kw)
    st = P.parity(out[:c["Tv"]], ref)
    print(f"NL={c['NL']} Lp={c['Lp']} Tv={c['Tv']} S={c['S']}: {st}", flush=True)
    ws = pi05.workspace(gpu)
    assert pi05.read_status(ws) == 0
    assert np.isfinite(out).all()
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st
    return out, ref, kc, vc


def test_pi05_small_two_layers(gpu):
    _check(P.make_case(NL=2, Lp=968, Tv=50, S=2), gpu)


def test_pi05_full_baseline_shape(gpu):
    """The batch-1 benchmark workload vs the fp32 oracle: 18 layers, Lp=968, Tv=50, 10 steps."""
    _check(P.make_case(NL=18, Lp=968, Tv=50, S=10), gpu)


@pytest.mark.parametrize("Lp,Tv,S", [(0, 50, 2), (37, 1, 3), (968, 64, 1), (2003, 17, 2), (5, 33, 1)])
def test_pi05_edge_shapes(gpu, Lp, Tv, S):
    _check(P.make_case(NL=2, Lp=Lp, Tv=Tv, S=S, seed=Lp + Tv), gpu)


@pytest.mark.parametrize("Lp,Tv", [(13, 15), (200, 16), (994, 17), (13, 31), (200, 32), (994, 48), (13, 49),
                                   (994, 63)])
def test_pi05_token_tile_boundaries(gpu, Lp, Tv):
    """Tv on either side of the 16-token tiles (the combine skips tiles past Tv, the attention
    partials skip rows past Tv) and Lp with this step's first key inside an 8-key V^T slot (13, 994)
    or on a slot boundary (200); Lp = 994 with Tv = 48 / 63 gives two 32-key blocks per rank."""
    _check(P.make_case(NL=1, Lp=Lp, Tv=Tv, S=2, seed=7 * Lp + Tv), gpu)


def test_pi05_deterministic(gpu):
    c = P.make_case(NL=2, Lp=300, Tv=50, S=2)
    g = P.gpu_tensors(c, gpu)
    a = P.run_gpu(c, gpu, g)[0]
    b = P.run_gpu(c, gpu, g)[0]
    assert np.array_equal(a, b)


def test_pi05_padded_rows_untouched(gpu):
    c = P.make_case(NL=1, Lp=100, Tv=10, S=1)
    out = P.run_gpu(c, gpu, xt_rows=16)[0]
    assert np.all(out[10:] == 0.0)


def test_pi05_suffix_cache_rows(gpu):
    """The launch writes the suffix K (RoPE'd) / V rows of the caller's caches (reference contract)."""
    c = P.make_case(NL=1, Lp=64, Tv=8, S=1)
    out, ref, kc, vc = _check(c, gpu)
    kc = kc.float().cpu()
    vc = vc.float().cpu()
    # recompute step-0 layer-0 suffix k, v on the CPU in fp32
    w = c["w"]
    x = c["inp"]["noise"][0] @ w["w_ain"].T + w["b_ain"]
    m = c["mods"][0, 0, 0]
    h = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6) * (1 + m[:1024]) + m[1024:2048]
    k = h @ w["wk"][0].float().T
    v = h @ w["wv"][0].float().T
    cos, sin = c["cos"], c["sin"]
    k = torch.cat([k[:, :128] * cos - k[:, 128:] * sin, k[:, 128:] * cos + k[:, :128] * sin], -1)
    assert torch.allclose(kc[0, 64:72], k, atol=3e-2, rtol=3e-2)
    assert torch.allclose(vc[0, :, 64:72].T, v, atol=3e-2, rtol=3e-2)
    assert torch.equal(kc[0, :64], c["inp"]["kpre"][0, 0].float())


def test_pi05_stage_cycles(gpu):
    c = P.make_case(NL=1, Lp=100, Tv=20, S=1)
    sc = torch.zeros(16, dtype=torch.int64, device=gpu)
    P.run_gpu(c, gpu, stage_cycles=sc)
    v = sc.cpu().numpy()
    assert (v[:10] > 0).all() and (v[10:] == 0).all()


def test_pi05_rejects_bad_shapes(gpu):
    c = P.make_case(NL=1, Lp=100, Tv=20, S=1)
    g = P.gpu_tensors(c, gpu)
    p = g["packed"]
    kc, vc = g["caches"][0]
    x_t = torch.zeros(65, 32, device=gpu)
    # the shim validates sizes before the C ABI does (the C ABI's own checks: tests/test_abi.py)
    with pytest.raises(ValueError, match="Tv"):
        pi05.launch(p["w1"], p["wo"], p["w2"], p["w3"], None, None, None, None, g["mods"], g["mod_final"],
                    g["cos"], g["sin"], g["w_ain"], g["b_ain"], g["w_aout"], g["b_aout"], None, None, 0,
                    kc, vc, 100, g["Lmax"], 1, 65, x_t)
    with pytest.raises(ValueError, match="Lmax"):
        pi05.launch(p["w1"], p["wo"], p["w2"], p["w3"], None, None, None, None, g["mods"], g["mod_final"],
                    g["cos"], g["sin"], g["w_ain"], g["b_ain"], g["w_aout"], g["b_aout"], None, None, 0,
                    kc, vc, 100, 112, 1, 20, x_t)
    with pytest.raises(ValueError, match="srows"):
        pi05.launch(p["w1"], p["wo"], p["w2"], p["w3"], None, None, None, None, g["mods"], g["mod_final"],
                    g["cos"], g["sin"], g["w_ain"], g["b_ain"], g["w_aout"], g["b_aout"], kc, vc, 10,
                    kc, vc, 100, g["Lmax"], 1, 20, x_t)
