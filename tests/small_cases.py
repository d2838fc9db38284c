"""Seeded small-shape cases (oracle input format) for the CPU pins of the oracle.

Weights are drawn with a larger spread than the benchmark's N(0, 0.02) so that every layer and
every term moves the output well above fp32 rounding (a dropped term must show).
"""
from __future__ import annotations

import numpy as np
import torch

PI05_SMALL = dict(NL=2, D=64, H=2, HD=16, F=96, AD=8, Lp=11, Tv=5, S=3, B=2)
MA2_SMALL = dict(NL=2, D=48, H=2, HD=24, F=80, AD=8, Lk=9, Tv=6, S=3, adim=5, B=2)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def pi05_case(seed=0, NL=2, D=64, H=2, HD=16, F=96, AD=8, Lp=11, Tv=5, S=3, B=2, std=0.15):
    g = torch.Generator().manual_seed(seed)
    n = lambda *s, sd=std: torch.randn(*s, generator=g) * sd  # noqa: E731
    w = {"wq": bits(n(NL, H * HD, D)), "wk": bits(n(NL, HD, D)), "wv": bits(n(NL, HD, D)),
         "wo": bits(n(NL, D, H * HD)), "wg": bits(n(NL, F, D)), "wu": bits(n(NL, F, D)),
         "wd": bits(n(NL, D, F))}
    mods = n(S, NL, 2, 3 * D, sd=0.3)
    mods[..., 2 * D:] += 1.0  # residual gates near 1 so each block contributes
    w.update(mods=mods.numpy(), mod_final=n(S, 3 * D, sd=0.3).numpy(),
             w_ain=n(D, AD, sd=0.3).numpy(), b_ain=n(D, sd=0.3).numpy(),
             w_aout=n(AD, D, sd=0.3).numpy(), b_aout=n(AD, sd=0.3).numpy(),
             kpre=bits(n(B, NL, Lp, HD, sd=1.0)), vpre=bits(n(B, NL, Lp, HD, sd=1.0)))
    pos = torch.arange(Lp, Lp + Tv, dtype=torch.float32)
    inv = 1.0 / (10000.0 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))
    ang = torch.outer(pos, inv)
    w.update(rope_cos=ang.cos().numpy(), rope_sin=ang.sin().numpy())
    x0 = n(B, Tv, AD, sd=1.0).numpy()
    dims = dict(NL=NL, D=D, H=H, HD=HD, F=F, AD=AD, Lp=Lp, Tv=Tv, S=S)
    return w, x0, dims


def pi05_time_weights(seed=0, NL=2, D=64, std=0.15):
    g = torch.Generator().manual_seed(seed)
    n = lambda *s: (torch.randn(*s, generator=g) * std).numpy()  # noqa: E731
    return {"w_ti": n(D, D), "b_ti": n(D), "w_to": n(D, D), "b_to": n(D), "w_in": n(NL, 3 * D, D),
            "b_in": n(NL, 3 * D), "w_post": n(NL, 3 * D, D), "b_post": n(NL, 3 * D), "w_fin": n(3 * D, D),
            "b_fin": n(3 * D)}


def ma2_case(seed=0, NL=2, D=48, H=2, HD=24, F=80, AD=8, Lk=9, Tv=6, S=3, adim=5, B=2, std=0.15):
    g = torch.Generator().manual_seed(seed)
    n = lambda *s, sd=std: torch.randn(*s, generator=g) * sd  # noqa: E731
    w = {"w_qkv": bits(n(NL, 3 * D, D)), "w_so": bits(n(NL, D, D)), "w_cq": bits(n(NL, D, D)),
         "w_co": bits(n(NL, D, D)), "w_g": bits(n(NL, F, D)), "w_u": bits(n(NL, F, D)),
         "w_dn": bits(n(NL, D, F)), "w_aout": bits(n(AD, D, sd=0.3))}
    mods = n(S, NL, 3, 3, D, sd=0.3)
    mods[:, :, :, 2] += 1.0
    w.update({k: n(*s).numpy() for k, s in (("b_qkv", (NL, 3 * D)), ("b_so", (NL, D)), ("b_cq", (NL, D)),
                                             ("b_co", (NL, D)), ("b_g", (NL, F)), ("b_u", (NL, F)),
                                             ("b_dn", (NL, D)))})
    w.update(mods=mods.numpy(), mod_final=n(S, 2, D, sd=0.3).numpy(), w_ain=n(D, AD, sd=0.3).numpy(),
             b_ain=n(D, sd=0.3).numpy(), b_aout=n(AD, sd=0.3).numpy(),
             kctx=bits(n(B, NL, Lk, D, sd=1.0)), vctx=bits(n(B, NL, Lk, D, sd=1.0)))
    pos = torch.arange(0, Tv, dtype=torch.float32)
    inv = 1.0 / (10000.0 ** (torch.arange(0, HD, 2, dtype=torch.float32) / HD))
    ang = torch.outer(pos, inv)
    w.update(rope_cos=ang.cos().numpy(), rope_sin=ang.sin().numpy())
    x0 = n(B, Tv, AD, sd=1.0)
    x0[..., adim:] = 0
    dims = dict(NL=NL, D=D, H=H, HD=HD, F=F, AD=AD, Lk=Lk, Tv=Tv, S=S, adim=adim)
    return w, x0.numpy(), dims
