"""Builds seeded pi0.5 cases and runs them through the oracle (CPU) or the C ABI (GPU)."""
from __future__ import annotations

import numpy as np
import torch

from flashact_amd import pi05, synthetic


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def make_case(NL=2, Lp=968, Tv=50, S=2, seed=0, batch=1, device="cpu"):
    w = synthetic.pi05_weights(seed, device, NL=NL)
    inp = synthetic.pi05_inputs(seed + 1, device, batch=batch, NL=NL, Lp=Lp, Tv=Tv)
    mods, modf = pi05.precompute_mods(S, w["w_ti"], w["b_ti"], w["w_to"], w["b_to"], w["w_in"], w["b_in"],
                                      w["w_post"], w["b_post"], w["w_fin"], w["b_fin"])
    cos, sin = pi05.rope_table(Lp, Tv, device=device)
    return dict(w=w, inp=inp, mods=mods, mod_final=modf, cos=cos, sin=sin, NL=NL, Lp=Lp, Tv=Tv, S=S, batch=batch)


def oracle_weights(c) -> dict:
    w = c["w"]
    ow = {k: u16(w[k]) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")}
    ow.update(mods=c["mods"].cpu().numpy(), mod_final=c["mod_final"].cpu().numpy(),
              rope_cos=c["cos"].cpu().numpy(), rope_sin=c["sin"].cpu().numpy(),
              w_ain=w["w_ain"].cpu().numpy(), b_ain=w["b_ain"].cpu().numpy(),
              w_aout=w["w_aout"].cpu().numpy(), b_aout=w["b_aout"].cpu().numpy(),
              kpre=u16(c["inp"]["kpre"]), vpre=u16(c["inp"]["vpre"]))
    return ow


def run_oracle(c) -> np.ndarray:
    from oracle import oracle as O
    return O.pi05_denoise(oracle_weights(c), c["inp"]["noise"].cpu().numpy(), Lp=c["Lp"], Tv=c["Tv"], S=c["S"],
                          NL=c["NL"])


def gpu_tensors(c, device):
    w = c["w"]
    packed = pi05.pack_weights(*(w[k].to(device) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")))
    Lmax = pi05.lmax_for(c["Lp"], c["Tv"])
    caches = []
    for b in range(c["batch"]):
        kv = torch.stack([c["inp"]["kpre"][b], c["inp"]["vpre"][b]], dim=1).to(device)  # [NL][2][Lp][HD]
        caches.append(pi05.make_caches(kv, Lmax))
    return dict(packed=packed, Lmax=Lmax, caches=caches,
                mods=c["mods"].to(device), mod_final=c["mod_final"].to(device),
                cos=c["cos"].to(device), sin=c["sin"].to(device),
                w_ain=w["w_ain"].to(device), b_ain=w["b_ain"].to(device),
                w_aout=w["w_aout"].to(device), b_aout=w["b_aout"].to(device))


def run_gpu(c, device, g=None, stage_cycles=None, xt_rows=None, sample=0, ws=None):
    """One launch for sample ``sample``; returns (x_t [Tv][32] numpy, kcache, vtcache)."""
    g = g or gpu_tensors(c, device)
    p = g["packed"]
    kc, vc = g["caches"][sample]
    rows = xt_rows or c["Tv"]
    x_t = torch.zeros(rows, 32, dtype=torch.float32, device=device)
    x_t[:c["Tv"]] = c["inp"]["noise"][sample].to(device)
    empty = torch.empty(0, device=device)
    pi05.launch(p["w1"], p["wo"], p["w2"], p["w3"], empty, empty, empty, empty, g["mods"], g["mod_final"],
                g["cos"], g["sin"], g["w_ain"], g["b_ain"], g["w_aout"], g["b_aout"], None, None, 0,
                kc, vc, c["Lp"], g["Lmax"], c["S"], c["Tv"], x_t, stage_cycles=stage_cycles,
                workspace_tensor=ws)
    torch.cuda.synchronize(device)
    return x_t.cpu().numpy(), kc, vc


def parity(gpu_out: np.ndarray, ref: np.ndarray) -> dict:
    d = np.abs(gpu_out.astype(np.float64) - ref.astype(np.float64))
    a, b = gpu_out.ravel().astype(np.float64), ref.ravel().astype(np.float64)
    cos = float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30))
    return {"max_abs": float(d.max()), "mean_abs": float(d.mean()), "cos": cos}


def run_gpu_batched(c, device, g=None, xt_rows=None, ws=None):
    """One batched launch over all samples; returns (x_t [B][Tv][32] numpy, kcache, vtcache)."""
    g = g or gpu_tensors(c, device)
    p = g["packed"]
    kc = torch.stack([k for k, _ in g["caches"]]).contiguous()
    vc = torch.stack([v for _, v in g["caches"]]).contiguous()
    rows = xt_rows or c["Tv"]
    x_t = torch.zeros(c["batch"], rows, 32, dtype=torch.float32, device=device)
    x_t[:, :c["Tv"]] = c["inp"]["noise"].to(device)
    empty = torch.empty(0, device=device)
    pi05.launch(p["w1"], p["wo"], p["w2"], p["w3"], empty, empty, empty, empty, g["mods"], g["mod_final"],
                g["cos"], g["sin"], g["w_ain"], g["b_ain"], g["w_aout"], g["b_aout"], None, None, 0,
                kc, vc, c["Lp"], g["Lmax"], c["S"], c["Tv"], x_t, workspace_tensor=ws)
    torch.cuda.synchronize(device)
    return x_t.cpu().numpy(), kc, vc
