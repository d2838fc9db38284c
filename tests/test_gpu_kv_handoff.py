"""K/V hand-off (srows > 0; the reference's prologue at src/pi05/mk6.cu:258-277) on the MI355X.

The source holds the prefix K with RoPE on interleaved pairs (2d, 2d + 1), as a prefill that uses
that pairing leaves it, and V row-major, with srows >= Lp rows per layer. After the hand-off the
caches must equal the split-half / transposed caches built on the host (bit for bit: the hand-off
only moves bf16 values), and the denoise loop must then produce exactly what it produces from
host-built caches.
"""
import numpy as np
import pytest
import torch

from flashact_amd import pi05
from tests import pi05_case as P

pytestmark = pytest.mark.gpu


def _interleaved(kpre):
    """[.., 256] split-half K -> the interleaved-pair layout: out[2d] = k[d], out[2d+1] = k[d+128]."""
    return torch.stack([kpre[..., :128], kpre[..., 128:]], dim=-1).reshape(kpre.shape).contiguous()


def _launch(c, g, kc, vc, x_t, ksrc=None, vsrc=None, srows=0):
    p = g["packed"]
    empty = torch.empty(0, device=x_t.device)
    pi05.launch(p["w1"], p["wo"], p["w2"], p["w3"], empty, empty, empty, empty, g["mods"], g["mod_final"],
                g["cos"], g["sin"], g["w_ain"], g["b_ain"], g["w_aout"], g["b_aout"], ksrc, vsrc, srows,
                kc, vc, c["Lp"], g["Lmax"], c["S"], c["Tv"], x_t)
    torch.cuda.synchronize()


@pytest.mark.parametrize("batch,Lp,extra", [(1, 968, 0), (1, 200, 9), (3, 130, 3)])
def test_handoff_matches_host_built_caches(gpu, batch, Lp, extra):
    c = P.make_case(NL=2, Lp=Lp, Tv=50, S=2, batch=batch, seed=Lp)
    g = P.gpu_tensors(c, gpu)
    kc_ref = torch.stack([k for k, _ in g["caches"]]).contiguous()
    vc_ref = torch.stack([v for _, v in g["caches"]]).contiguous()
    srows = Lp + extra
    ksrc = torch.randn(batch, 2, srows, 256, device=gpu).to(torch.bfloat16)  # rows >= Lp: never read
    vsrc = torch.randn(batch, 2, srows, 256, device=gpu).to(torch.bfloat16)
    ksrc[:, :, :Lp] = _interleaved(c["inp"]["kpre"].to(gpu))
    vsrc[:, :, :Lp] = c["inp"]["vpre"].to(gpu)
    x0 = c["inp"]["noise"].to(gpu)
    shape = (lambda t: t) if batch > 1 else (lambda t: t[0])
    # host-built caches
    xa = shape(x0.clone())
    _launch(c, g, shape(kc_ref.clone()), shape(vc_ref.clone()), xa)
    # hand-off into caches that start as garbage in the prefix rows
    kc = torch.randn_like(kc_ref, dtype=torch.float32).to(torch.bfloat16)
    vc = torch.randn_like(vc_ref, dtype=torch.float32).to(torch.bfloat16)
    xb = shape(x0.clone())
    _launch(c, g, shape(kc), shape(vc), xb, ksrc, vsrc, srows)
    assert torch.equal(kc[:, :, :Lp], kc_ref[:, :, :Lp])
    assert torch.equal(vc[:, :, :, :Lp], vc_ref[:, :, :, :Lp])
    assert torch.equal(xa, xb)
    ref = P.run_oracle(c)
    st = P.parity(np.asarray(xb.cpu()).reshape(batch, c["Tv"], 32), ref)
    print(f"hand-off B={batch} Lp={Lp} srows={srows}: {st}", flush=True)
    assert st["max_abs"] <= 2e-2 and st["mean_abs"] <= 2e-3
