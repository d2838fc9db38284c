"""Seeded backbone-prefill cases (the benchmark prefill shape) for the oracle (CPU) and the C ABI (GPU)."""
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


def run_bf16_floor(c):
    """(K, V) [batch][NL][Lp][256] of a torch restatement of the prefill in fp32 arithmetic that
    rounds to bf16 exactly where the kernel does: the matmul operands bf16 MFMAs take (the normed rows,
    q, k, v, the softmax weights of each 128-key chunk and that chunk's normalised output, the
    combined attention output, the MLP activation) and the K-split partial sums the kernel stores in
    bf16 (the O projection in 2 K ranges of 1024, the down projection in 8 of 2048, each partial
    rounded once before the next norm adds them to the fp32 residual). Its distance to the fp32
    oracle is the error those roundings alone produce (the floor a bf16 kernel is held to); it is
    not the oracle."""
    w = c["w"]
    bf = lambda t: t.to(torch.bfloat16).float()  # noqa: E731
    cos, sin = c["cos"].float(), c["sin"].float()

    def rms(x, ln):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6) * (1 + ln)

    def rope(v):
        a, b = v[..., :128], v[..., 128:]
        cc, ss = (cos[:, None], sin[:, None]) if v.dim() == 3 else (cos, sin)
        return torch.cat([a * cc - b * ss, b * cc + a * ss], -1)

    NL, Lp = c["NL"], c["Lp"]
    Ks, Vs = [], []
    for b in range(c["batch"]):
        x = c["x"][b].float().cpu().clone()
        kl, vl = [], []
        for l in range(NL):
            h = bf(rms(x, w["ln_in"][l].float().cpu()))
            q = bf(rope((h @ w["wq"][l].float().cpu().T).view(Lp, 8, 256)))
            k = bf(rope(h @ w["wk"][l].float().cpu().T))
            v = bf(h @ w["wv"][l].float().cpu().T)
            kl.append(k)
            vl.append(v)
            if l == NL - 1:
                break
            s = torch.einsum("thd,jd->htj", q, k) / 16.0
            outs, ms, ls = [], [], []
            for c0 in range(0, Lp, 128):
                sc = s[:, :, c0:c0 + 128]
                m = sc.amax(-1, keepdim=True)
                p = torch.exp(sc - m)
                lsum = p.sum(-1, keepdim=True)
                outs.append(bf((bf(p) @ v[c0:c0 + 128]) / lsum))
                ms.append(m)
                ls.append(lsum)
            M = torch.stack(ms).amax(0)
            wsum = sum(l_ * torch.exp(m_ - M) for l_, m_ in zip(ls, ms))
            att = sum(o * l_ * torch.exp(m_ - M) for o, l_, m_ in zip(outs, ls, ms)) / wsum
            att = bf(att).permute(1, 0, 2).reshape(Lp, 8 * 256)
            wo = w["wo"][l].float().cpu()
            x = x + sum(bf(att[:, k0:k0 + 1024] @ wo[:, k0:k0 + 1024].T) for k0 in range(0, 2048, 1024))
            h = bf(rms(x, w["ln_post"][l].float().cpu()))
            g = h @ w["wg"][l].float().cpu().T
            u = h @ w["wu"][l].float().cpu().T
            m = bf(torch.nn.functional.gelu(g, approximate="tanh") * u)
            wd = w["wd"][l].float().cpu()
            x = x + sum(bf(m[:, k0:k0 + 2048] @ wd[:, k0:k0 + 2048].T) for k0 in range(0, 16384, 2048))
        Ks.append(torch.stack(kl))
        Vs.append(torch.stack(vl))
    return torch.stack(Ks).numpy(), torch.stack(Vs).numpy()
