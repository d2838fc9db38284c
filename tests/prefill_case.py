"""Seeded backbone-prefill cases (BASELINE config 3 shape) for the oracle (CPU) and the C ABI (GPU)."""
from __future__ import annotations

import numpy as np
import torch

from flashact_amd import pi05, synthetic
from tests.pi05_case import u16


def make_case(NL=2, Lp=200, batch=1, seed=0, device="cpu"):
    w = synthetic.backbone_weights(seed + 20, device, NL=NL)
    x = synthetic.prefix_inputs(seed + 21, device, batch=batch, Lp=Lp)
    cos, sin = pi05.rope_table(0, Lp)
    return dict(w=w, x=x, cos=cos, sin=sin, NL=NL, Lp=Lp, batch=batch)


def run_oracle(c):
    """(K, V) fp32, each [batch][NL][Lp][256]."""
    from oracle import oracle as O
    w = c["w"]
    ow = {k: u16(w[k]) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")}
    ow.update(ln_in=w["ln_in"].cpu().numpy(), ln_post=w["ln_post"].cpu().numpy(), rope_cos=c["cos"].numpy(),
              rope_sin=c["sin"].numpy())
    return O.gemma_prefill(ow, c["x"].cpu().numpy(), NL=c["NL"])


def gpu_weights(c, device):
    w = c["w"]
    packed = pi05.pack_weights(*(w[k].to(device) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")))
    packed = {"wqkv": packed["w1"], "wo": packed["wo"], "wgu": packed["w2"], "wdn": packed["w3"]}
    return dict(packed=packed, ln_in=w["ln_in"].to(device), ln_post=w["ln_post"].to(device))


def run_gpu(c, device, g=None, Lmax=None, ws=None, samples=None, stage_cycles=None):
    """One prefill launch; returns (kcache [B][NL][Lmax][256], vtcache [B][NL][256][Lmax]) on the GPU."""
    from flashact_amd import prefill
    g = g or gpu_weights(c, device)
    samples = list(range(c["batch"])) if samples is None else list(samples)
    Lmax = Lmax or (c["Lp"] + 15) // 16 * 16
    B = len(samples)
    kc = torch.zeros(B, c["NL"], Lmax, 256, dtype=torch.bfloat16, device=device)
    vt = torch.zeros(B, c["NL"], 256, Lmax, dtype=torch.bfloat16, device=device)
    x = c["x"][samples].to(device).contiguous()
    prefill.prefill(g["packed"], g["ln_in"], g["ln_post"], x, kc, vt, c["cos"].to(device), c["sin"].to(device),
                    stage_cycles=stage_cycles, workspace_tensor=ws)
    torch.cuda.synchronize(device)
    return kc, vt


def kv_diff(kc, vt, K, V, Lp):
    """Per-layer max / mean |GPU - oracle| of K and V over the Lp prefix rows, and the largest |oracle|."""
    kg = kc[:, :, :Lp].float().cpu().numpy()
    vg = vt[:, :, :, :Lp].float().cpu().numpy().transpose(0, 1, 3, 2)
    dk, dv = np.abs(kg - K), np.abs(vg - V)
    return {"k_max": float(dk.max()), "k_mean": float(dk.mean()), "v_max": float(dv.max()),
            "v_mean": float(dv.mean()), "ref_max": float(max(np.abs(K).max(), np.abs(V).max()))}
