"""pi0.5 bs=1 with FP8-W8A16 weights (the reference's numerics, src/pi05/hybrid_model.py:105-110 and
src/pi05/mk6.cu:204-225) on the MI355X vs the oracle's fp8 path on the same e4m3 codes and scales.

The kernel streams e4m3 codes through its LDS ring, converts them exactly to bf16 for the MFMAs
and multiplies each output row by its scale; the oracle computes (sum_k x_k q_nk) s_n in fp32.
Tolerance as for bf16 weights: max-abs <= 2e-2 and mean-abs <= 2e-3 on the final actions.
"""
import numpy as np
import pytest
import torch

from flashact_amd import pi05
from tests import pi05_case as P

MAX_ABS, MEAN_ABS = 2e-2, 2e-3

pytestmark = pytest.mark.gpu


def _run(c, gpu, xt_rows=None):
    w = c["w"]
    nat = {k: w[k] for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")}
    pk = pi05.pack_weights_fp8(*(nat[k].to(gpu) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")))
    g = P.gpu_tensors(c, gpu)
    kc, vc = g["caches"][0]
    rows = xt_rows or c["Tv"]
    x_t = torch.zeros(rows, 32, dtype=torch.float32, device=gpu)
    x_t[:c["Tv"]] = c["inp"]["noise"][0].to(gpu)
    pi05.launch(pk["w1"], pk["wo"], pk["w2"], pk["w3"], pk["s1"], pk["so"], pk["s2"], pk["s3"], g["mods"],
                g["mod_final"], g["cos"], g["sin"], g["w_ain"], g["b_ain"], g["w_aout"], g["b_aout"], None, None, 0,
                kc, vc, c["Lp"], g["Lmax"], c["S"], c["Tv"], x_t)
    torch.cuda.synchronize()
    assert pi05.read_status(pi05.workspace(gpu)) == 0
    # oracle: the same per-row codes / scales in natural layouts
    from oracle import oracle as O
    ow = P.oracle_weights(c)
    for n, k in (("q", "wq"), ("k", "wk"), ("v", "wv"), ("o", "wo"), ("g", "wg"), ("u", "wu"), ("d", "wd")):
        q, s = pi05.quantize_fp8(nat[k])
        ow["q" + n], ow["s" + n] = q.numpy(), s.numpy()
    ref = O.pi05_denoise_fp8(ow, c["inp"]["noise"].numpy(), Lp=c["Lp"], Tv=c["Tv"], S=c["S"], NL=c["NL"])[0]
    return x_t.cpu().numpy(), ref


@pytest.mark.parametrize("NL,Lp,Tv,S", [(2, 200, 50, 2), (18, 968, 50, 10), (18, 968, 10, 10), (1, 0, 1, 1),
                                        (2, 333, 64, 2)])
def test_fp8_matches_oracle(gpu, NL, Lp, Tv, S):
    c = P.make_case(NL=NL, Lp=Lp, Tv=Tv, S=S, seed=NL + Lp + Tv)
    out, ref = _run(c, gpu)
    st = P.parity(out[:Tv], ref)
    print(f"fp8 NL={NL} Lp={Lp} Tv={Tv} S={S}: {st}", flush=True)
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st


def test_fp8_padded_rows_untouched(gpu):
    c = P.make_case(NL=1, Lp=50, Tv=10, S=1, seed=3)
    out, _ = _run(c, gpu, xt_rows=16)
    assert np.all(out[10:] == 0.0)
