"""Builds seeded MolmoAct2 cases and runs them through the oracle (CPU) or the C ABI (GPU)."""
from __future__ import annotations

import numpy as np
import torch

from flashact_amd import ma2, synthetic


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def make_case(NL=2, Lk=493, Tv=30, S=2, adim=6, batch=1, seed=0, unit_gates=True):
    """Synthetic N(0, 0.02) weights; with ``unit_gates`` the residual gates are shifted to ~1 so
    that every block moves the output (the benchmark keeps the plain N(0, 0.02) draw)."""
    w = synthetic.ma2_weights(seed, "cpu", NL=NL, S=S)
    if unit_gates:
        w["mods"][:, :, :, 2] += 1.0
    inp = synthetic.ma2_inputs(seed + 1, "cpu", batch=batch, NL=NL, Lk=Lk, Tv=Tv, adim=adim)
    cos, sin = ma2.rope_table(Tv)
    return dict(w=w, inp=inp, cos=cos, sin=sin, NL=NL, Lk=Lk, Tv=Tv, S=S, adim=adim, batch=batch)


def run_oracle(c) -> np.ndarray:
    """[batch][Tv][32] after the S-step loop (fp32 CPU oracle)."""
    from oracle import oracle as O
    w, inp = c["w"], c["inp"]
    ow = {k: u16(w[k]) for k in ("w_qkv", "w_so", "w_cq", "w_co", "w_g", "w_u", "w_dn", "w_aout")}
    ow.update({k: w[k].numpy() for k in ("b_qkv", "b_so", "b_cq", "b_co", "b_g", "b_u", "b_dn", "mods", "mod_final",
                                         "w_ain", "b_ain", "b_aout")})
    ow.update(rope_cos=c["cos"].numpy(), rope_sin=c["sin"].numpy(), kctx=u16(inp["kctx"]), vctx=u16(inp["vctx"]))
    return O.ma2_flow(ow, inp["noise"].numpy(), Lk=c["Lk"], Tv=c["Tv"], S=c["S"], NL=c["NL"], adim=c["adim"])


def gpu_tensors(c, device):
    w, inp = c["w"], c["inp"]
    d = lambda k: w[k].to(device)  # noqa: E731
    ws, bs = ma2.pack_weights(d("w_qkv"), d("w_so"), d("w_cq"), d("w_co"), d("w_g"), d("w_u"), d("w_dn"),
                              d("b_qkv"), d("b_so"), d("b_cq"), d("b_co"), d("b_g"), d("b_u"), d("b_dn"))
    Lkmax = ma2.lkmax_for(c["Lk"])
    kc, vt = ma2.make_context(inp["kctx"].to(device), inp["vctx"].to(device), Lkmax)  # [B][NL][..]
    return dict(ws=ws, bs=bs, kc=kc, vt=vt, Lkmax=Lkmax, mods=d("mods"), mod_final=d("mod_final"),
                cos=c["cos"].to(device), sin=c["sin"].to(device), w_ain=d("w_ain"), b_ain=d("b_ain"),
                w_aout=w["w_aout"].to(device).to(torch.bfloat16), b_aout=d("b_aout"))


def run_gpu(c, device, g=None, samples=None, xt_rows=None, stage_cycles=None, ws=None):
    """One launch over ``samples`` (default: all); returns x_t [len(samples)][Tv][32] numpy.
    ``ws``: a caller-owned workspace tensor (default: the per-device cached one)."""
    g = g or gpu_tensors(c, device)
    samples = list(range(c["batch"])) if samples is None else list(samples)
    kc = g["kc"][samples].contiguous()
    vt = g["vt"][samples].contiguous()
    rows = xt_rows or c["Tv"]
    x_t = torch.zeros(len(samples), rows, 32, dtype=torch.float32, device=device)
    x_t[:, :c["Tv"]] = c["inp"]["noise"][samples].to(device)
    ma2.launch(g["ws"], g["bs"], g["mods"], g["mod_final"], g["cos"], g["sin"], g["w_ain"], g["b_ain"], g["w_aout"],
               g["b_aout"], kc, vt, c["Lk"], g["Lkmax"], c["Tv"], c["adim"], c["S"], x_t, stage_cycles=stage_cycles,
               workspace_tensor=ws)
    torch.cuda.synchronize(device)
    return x_t.cpu().numpy()


def parity(gpu_out: np.ndarray, ref: np.ndarray, adim: int) -> dict:
    """Differences over the integrated dims [0, adim) of every row."""
    a = gpu_out[..., :adim].astype(np.float64)
    b = ref[..., :adim].astype(np.float64)
    d = np.abs(a - b)
    cos = float(a.ravel() @ b.ravel() / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30))
    return {"max_abs": float(d.max()), "mean_abs": float(d.mean()), "cos": cos}
