"""Seeded synthetic weights and inputs of the benchmark configurations.

There is no network access for real checkpoints, so every run uses random-init weights of
the named architecture:
  * every weight and bias ~ N(0, 0.02), rounded to bf16 (fp32 consumers get the same
    bf16-representable values, so the CPU oracle and the GPU see identical inputs);
  * prefix K/V ~ N(0, 1) rounded to bf16 (treated as already-RoPE'd cached keys);
  * initial noise x ~ N(0, 1) fp32.
Generation runs on ``device`` with a torch.Generator seeded by ``seed``.
"""
from __future__ import annotations

import torch

PI05 = dict(NL=18, D=1024, H=8, HD=256, F=4096, AD=32)
PI05_BASELINE = dict(Lp=968, Tv=50, S=10)  # the pi0.5 expert workloads (batch 1 and 16)
BACKBONE = dict(NL=18, D=2048, H=8, HD=256, F=16384)  # the prefix prefill workload (Gemma-2B shape)
MA2 = dict(NL=36, D=768, H=8, HD=96, F=3072, AD=32)
MA2_BASELINE = dict(Lk=493, Tv=30, S=10, adim=6)


def _gen(seed: int, device) -> torch.Generator:
    return torch.Generator(device=torch.device(device)).manual_seed(int(seed))


def _normal(g, shape, std, device):
    x = torch.randn(*shape, generator=g, device=device, dtype=torch.float32)
    if std != 1.0:
        x.mul_(std)
    return x.to(torch.bfloat16)


def pi05_weights(seed: int = 0, device="cpu", NL=18, D=1024, H=8, HD=256, F=4096, AD=32, std=0.02):
    """Natural-layout pi0.5 expert weights ([out][in]). bf16 tensors for the GEMM weights,
    bf16-valued float32 for the time MLP, adaRMS dense layers and action projections."""
    g = _gen(seed, device)
    n = lambda *s: _normal(g, s, std, device)  # noqa: E731
    w = {
        "wq": n(NL, H * HD, D), "wk": n(NL, HD, D), "wv": n(NL, HD, D), "wo": n(NL, D, H * HD),
        "wg": n(NL, F, D), "wu": n(NL, F, D), "wd": n(NL, D, F),
    }
    f32 = {
        "w_ti": n(D, D), "b_ti": n(D), "w_to": n(D, D), "b_to": n(D),
        "w_in": n(NL, 3 * D, D), "b_in": n(NL, 3 * D), "w_post": n(NL, 3 * D, D), "b_post": n(NL, 3 * D),
        "w_fin": n(3 * D, D), "b_fin": n(3 * D),
        "w_ain": n(D, AD), "b_ain": n(D), "w_aout": n(AD, D), "b_aout": n(AD),
    }
    w.update({k: v.float() for k, v in f32.items()})
    return w


def pi05_inputs(seed: int = 1, device="cpu", batch=1, NL=18, Lp=968, Tv=50, HD=256, AD=32):
    """Prefix K/V [batch][NL][Lp][HD] bf16 ~ N(0,1) and noise [batch][Tv][AD] fp32 ~ N(0,1)."""
    g = _gen(seed, device)
    kpre = _normal(g, (batch, NL, Lp, HD), 1.0, device)
    vpre = _normal(g, (batch, NL, Lp, HD), 1.0, device)
    noise = torch.randn(batch, Tv, AD, generator=g, device=device, dtype=torch.float32)
    return {"kpre": kpre, "vpre": vpre, "noise": noise}


def backbone_weights(seed: int = 2, device="cpu", NL=18, D=2048, H=8, HD=256, F=16384, std=0.02):
    """Natural-layout Gemma-2B-shaped backbone weights ([out][in], bf16) and the two RMSNorm weight
    vectors per layer (bf16-valued float32)."""
    g = _gen(seed, device)
    n = lambda *s: _normal(g, s, std, device)  # noqa: E731
    w = {"wq": n(NL, H * HD, D), "wk": n(NL, HD, D), "wv": n(NL, HD, D), "wo": n(NL, D, H * HD),
         "wg": n(NL, F, D), "wu": n(NL, F, D), "wd": n(NL, D, F)}
    w["ln_in"] = n(NL, D).float()
    w["ln_post"] = n(NL, D).float()
    return w


def prefix_inputs(seed: int = 3, device="cpu", batch=1, Lp=968, D=2048):
    """Prefix hidden states entering backbone layer 0: [batch][Lp][D] fp32 ~ N(0, 1)."""
    g = _gen(seed, device)
    return torch.randn(batch, Lp, D, generator=g, device=device, dtype=torch.float32)


def ma2_weights(seed: int = 0, device="cpu", NL=36, D=768, F=3072, AD=32, S=10, std=0.02):
    """Natural-layout MolmoAct2 expert weights and synthetic adaLN modulations.

    The HF modulation cache is absent, so mods [S][NL][3][3][D] and mod_final [S][2][D]
    (scale, shift, gate / scale, shift) are drawn directly from N(0, 0.02).
    """
    g = _gen(seed, device)
    n = lambda *s: _normal(g, s, std, device)  # noqa: E731
    w = {"w_qkv": n(NL, 3 * D, D), "w_so": n(NL, D, D), "w_cq": n(NL, D, D), "w_co": n(NL, D, D),
         "w_g": n(NL, F, D), "w_u": n(NL, F, D), "w_dn": n(NL, D, F), "w_aout": n(AD, D)}
    f32 = {"b_qkv": n(NL, 3 * D), "b_so": n(NL, D), "b_cq": n(NL, D), "b_co": n(NL, D),
           "b_g": n(NL, F), "b_u": n(NL, F), "b_dn": n(NL, D),
           "mods": n(S, NL, 3, 3, D), "mod_final": n(S, 2, D),
           "w_ain": n(D, AD), "b_ain": n(D), "b_aout": n(AD)}
    w.update({k: v.float() for k, v in f32.items()})
    return w


def ma2_inputs(seed: int = 1, device="cpu", batch=1, NL=36, Lk=493, Tv=30, D=768, AD=32, adim=6):
    """Cross-attention context K/V [batch][NL][Lk][D] bf16 ~ N(0,1); noise [batch][Tv][AD]
    ~ N(0,1) with dims >= adim zeroed (benchmarks/molmoact2/eval_numerics.py:146-149)."""
    g = _gen(seed, device)
    kctx = _normal(g, (batch, NL, Lk, D), 1.0, device)
    vctx = _normal(g, (batch, NL, Lk, D), 1.0, device)
    noise = torch.randn(batch, Tv, AD, generator=g, device=device, dtype=torch.float32)
    noise[..., adim:] = 0
    return {"kctx": kctx, "vctx": vctx, "noise": noise}
