"""A float64 restatement of the batch-1 pi0.5 loop that rounds exactly where the batch-1 kernel
rounds, used to size the error of those roundings against the fp32 oracle. It is not the oracle.

Roundings (as in flashact_amd/csrc/pi05_bs1.hip):
  * bf16 MFMA operands: the normed rows, q and k after RoPE, v, the softmax weights of each attention
    block, each chunk's normalised partial output, the combined attention output, the MLP activation;
  * attention in 32 chunks per head, as the kernel splits it (chunk r: prefix keys [C r, C r + C) with
    C = 32 ceil(Lp / 1024), then this step's keys of tokens r and r + 32 as one more block), online
    softmax per block, flash-decoding combine;
  * the cross-XCD partial sums of the O projection (one per head, K-window of 256) and of the down
    projection (one per 512-wide F-slice): ``exchange="fp16"`` rounds each to fp16 and forces its lowest
    mantissa bit to the layer's parity (what the kernel exchanges), ``"fp32"`` keeps them exact, so the
    two runs isolate what the fp16 exchange adds. The kernel's parity of layer pass li is
    (1 + li) & 1 on a freshly initialised workspace.
The residual stream, the norm statistics and the final action projection stay unrounded.
"""
from __future__ import annotations

import math

import numpy as np
import torch

f64 = torch.float64
D, H, HD, F, AD = 1024, 8, 256, 4096, 32


def bf(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(f64)


def f16_tagged(t: torch.Tensor, par: int) -> torch.Tensor:
    """fp16 round to nearest even (clamped to the finite range), then the lowest mantissa bit := par."""
    h = t.clamp(-65504.0, 65504.0).to(torch.float16)
    b = h.view(torch.int16)
    b = (b & ~1) | par
    return b.view(torch.float16).to(f64)


def ada_rms(x, scale, shift):
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6) * (1 + scale) + shift


def rope(v, cos, sin):
    a, b = v[..., :HD // 2], v[..., HD // 2:]
    return torch.cat([a * cos - b * sin, b * cos + a * sin], -1)


@torch.no_grad()
def denoise(c, exchange: str = "fp16") -> np.ndarray:
    """x_t [Tv][32] after the S-step loop on case ``c`` (tests/pi05_case.make_case, batch 1)."""
    assert exchange in ("fp16", "fp32")
    w = {k: v.to(f64) for k, v in c["w"].items()}
    NL, Lp, Tv, S = c["NL"], c["Lp"], c["Tv"], c["S"]
    mods, modf = c["mods"].to(f64), c["mod_final"].to(f64)
    cos, sin = c["cos"].to(f64), c["sin"].to(f64)
    kpre, vpre = c["inp"]["kpre"][0].to(f64), c["inp"]["vpre"][0].to(f64)  # [NL][Lp][HD], bf16-exact
    xt = c["inp"]["noise"][0].to(f64).clone()
    C = 32 * max(1, math.ceil(Lp / 1024))
    gelu = lambda z: 0.5 * z * (1 + torch.tanh(math.sqrt(2 / math.pi) * (z + 0.044715 * z ** 3)))  # noqa: E731

    def xchg(parts, par):  # parts [G][Tv][D] partial sums -> their sum as the norm stage forms it
        if exchange == "fp16":
            parts = f16_tagged(parts, par)
        return parts.sum(0)

    dt = -1.0 / S
    li = 0
    for s in range(S):
        x = xt @ w["w_ain"].T + w["b_ain"]
        for l in range(NL):
            par = (1 + li) & 1
            mi, mp = mods[s, l, 0], mods[s, l, 1]
            h = bf(ada_rms(x, mi[:D], mi[D:2 * D]))
            q = bf(rope((h @ w["wq"][l].T).view(Tv, H, HD), cos[:, None], sin[:, None]))  # [Tv][H][HD]
            k = bf(rope(h @ w["wk"][l].T, cos, sin))
            v = bf(h @ w["wv"][l].T)
            attn = torch.empty(Tv, H, HD, dtype=f64)
            for hh in range(H):
                qh = q[:, hh]
                outs, ms, ls = [], [], []
                for r in range(32):
                    blocks = []
                    kb, ke = C * r, min(C * r + C, Lp)
                    for b0 in range(kb, ke, 32):
                        b1 = min(b0 + 32, ke)
                        blocks.append((kpre[l, b0:b1], vpre[l, b0:b1]))
                    sfx = [t for t in (r, r + 32) if t < Tv]
                    if sfx:
                        blocks.append((k[sfx], v[sfx]))
                    if not blocks:
                        continue
                    m = torch.full((Tv, 1), -1e30, dtype=f64)
                    lsum = torch.zeros(Tv, 1, dtype=f64)
                    o = torch.zeros(Tv, HD, dtype=f64)
                    for K, V in blocks:
                        sc = (qh @ K.T) / 16.0
                        mnew = torch.maximum(m, sc.max(-1, keepdim=True).values)
                        alpha = torch.exp(m - mnew)
                        p = torch.exp(sc - mnew)
                        lsum = lsum * alpha + p.sum(-1, keepdim=True)
                        o = o * alpha + bf(p) @ V
                        m = mnew
                    outs.append(bf(o / lsum))
                    ms.append(m)
                    ls.append(lsum)
                M = torch.stack(ms).amax(0)
                wts = [l_ * torch.exp(m_ - M) for l_, m_ in zip(ls, ms)]
                attn[:, hh] = bf(sum(wt * o_ for wt, o_ in zip(wts, outs)) / sum(wts))
            parts = torch.stack([attn[:, g] @ w["wo"][l][:, HD * g:HD * g + HD].T for g in range(H)])
            x = x + mi[2 * D:] * xchg(parts, par)
            h2 = bf(ada_rms(x, mp[:D], mp[D:2 * D]))
            m_ = bf(gelu(h2 @ w["wg"][l].T) * (h2 @ w["wu"][l].T))
            parts = torch.stack([m_[:, 512 * g:512 * g + 512] @ w["wd"][l][:, 512 * g:512 * g + 512].T for g in range(8)])
            x = x + mp[2 * D:] * xchg(parts, par)
            li += 1
        mf = modf[s]
        hf = ada_rms(x, mf[:D], mf[D:2 * D])
        xt = xt + dt * (hf @ w["w_aout"].T + w["b_aout"])
    return xt.numpy()


def unit_gates(c):
    """The hard case: every residual gate of every layer (and step) set to 1, so each layer's
    attention and MLP outputs enter the residual stream whole."""
    c = dict(c)
    mods = c["mods"].clone()
    mods[..., 2 * D:3 * D] = 1.0
    c["mods"] = mods
    return c
