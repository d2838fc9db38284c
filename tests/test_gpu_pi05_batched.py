"""Batched pi0.5 denoise loop (batch >= 2: the MFMA-bound kernel) on the MI355X vs the CPU fp32 oracle.

Tolerance (the acceptance tolerance for bf16 operands with fp32 accumulation vs the fp32 oracle, on the
final actions of every sample): max-abs <= 2e-2 and mean-abs <= 2e-3.
"""
import numpy as np
import pytest
import torch

from tests import pi05_case as P
from flashact_amd import pi05

MAX_ABS, MEAN_ABS = 2e-2, 2e-3

pytestmark = pytest.mark.gpu


def _check(c, gpu, **kw):
    ref = P.run_oracle(c)
    out, kc, vc = P.run_gpu_batched(c, gpu, **kw)
    ws = pi05.workspace(gpu, c["batch"], c["Tv"], pi05.lmax_for(c["Lp"], c["Tv"]))
    assert pi05.read_status(ws) == 0
    assert np.isfinite(out).all()
    for b in range(c["batch"]):
        st = P.parity(out[b, :c["Tv"]], ref[b])
        print(f"B={c['batch']} sample {b} NL={c['NL']} Lp={c['Lp']} Tv={c['Tv']} S={c['S']}: {st}", flush=True)
        assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, (b, st)
    return out, ref, kc, vc


def test_batched_two_samples(gpu):
    _check(P.make_case(NL=2, Lp=968, Tv=50, S=2, batch=2), gpu)


# Lp + Tv: 54, 50, 364, 1109 end inside a 128-key chunk (the last chunk masked, its V^T tail group
# zeroed), 256 fills every chunk exactly (no masking at all)
@pytest.mark.parametrize("B,Lp,Tv,S", [(3, 37, 17, 2), (2, 0, 50, 1), (5, 300, 64, 1), (2, 1100, 9, 2),
                                      (2, 206, 50, 1)])
def test_batched_edge_shapes(gpu, B, Lp, Tv, S):
    _check(P.make_case(NL=2, Lp=Lp, Tv=Tv, S=S, batch=B, seed=B + Lp + Tv), gpu)


def test_batched_baseline_config2(gpu):
    """The batch-16 benchmark workload vs the fp32 oracle: batch 16, 18 layers, Lp=968, Tv=50, 10 steps."""
    _check(P.make_case(NL=18, Lp=968, Tv=50, S=10, batch=16), gpu)


def test_batched_matches_bs1_kernel(gpu):
    """Sample i of a batched launch agrees with the batch-1 kernel run on sample i alone."""
    c = P.make_case(NL=2, Lp=200, Tv=50, S=2, batch=3, seed=7)
    g = P.gpu_tensors(c, gpu)
    outb = P.run_gpu_batched(c, gpu, g)[0]
    for b in range(3):
        g1 = P.gpu_tensors(c, gpu)
        out1 = P.run_gpu(c, gpu, g1, sample=b)[0]
        assert np.abs(out1 - outb[b]).max() <= MAX_ABS


def test_batched_padded_rows_untouched(gpu):
    c = P.make_case(NL=1, Lp=100, Tv=10, S=1, batch=2)
    out = P.run_gpu_batched(c, gpu, xt_rows=16)[0]
    assert np.all(out[:, 10:] == 0.0)


def test_batched_suffix_cache_rows(gpu):
    """Each sample's suffix K/V rows land in its own slice of the stacked caches; the prefix is untouched."""
    c = P.make_case(NL=1, Lp=64, Tv=8, S=1, batch=2)
    out, ref, kc, vc = _check(c, gpu)
    kc = kc.float().cpu()
    vc = vc.float().cpu()
    w = c["w"]
    for b in range(2):
        x = c["inp"]["noise"][b] @ w["w_ain"].T + w["b_ain"]
        m = c["mods"][0, 0, 0]
        h = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6) * (1 + m[:1024]) + m[1024:2048]
        k = h @ w["wk"][0].float().T
        v = h @ w["wv"][0].float().T
        cos, sin = c["cos"], c["sin"]
        k = torch.cat([k[:, :128] * cos - k[:, 128:] * sin, k[:, 128:] * cos + k[:, :128] * sin], -1)
        assert torch.allclose(kc[b, 0, 64:72], k, atol=3e-2, rtol=3e-2)
        assert torch.allclose(vc[b, 0, :, 64:72].T, v, atol=3e-2, rtol=3e-2)
        assert torch.equal(kc[b, 0, :64], c["inp"]["kpre"][b, 0].float())
