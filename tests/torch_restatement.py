"""PyTorch-CPU float64 restatement of both denoise loops, assembled from third-party blocks.

This is the second, independent statement of the math the C oracle (oracle/fa_oracle.c) restates;
tests compare the two. Every non-trivial block comes from a library rather than from this file:
  * adaRMS ........ transformers GemmaRMSNorm (x * rsqrt(mean(x^2) + eps) * (1 + weight)) with
                    weight = scale, then + shift (src/pi05/mk6.cu:145-161)
  * RoPE .......... transformers GemmaRotaryEmbedding (inv_freq = 1 / base^(2j/HD)) and
                    apply_rotary_pos_emb / rotate_half (split-half pairs j, j + HD/2;
                    src/pi05/mk6.cu:222-237, src/pi05/pack_weights.py:54-58)
  * attention ..... torch scaled_dot_product_attention (scale 1/sqrt(HD); src/pi05/mk6.cu:338)
  * MLP ........... transformers GELUTanh ("gelu_pytorch_tanh", src/pi05/mk6.cu:79-82) and SiLU
  * time embedding  transformers PI0TimestepEmbeddings frequencies (the openpi sinusoid,
                    src/pi05/pack_weights.py:26-31)
The stage order follows src/pi05/mk6.cu:279-518 and src/molmoact2/mk_ma2.cu:258-575.

``mutate`` plants one plausible mistake (for tests that show the comparison catches it).
"""
from __future__ import annotations

import types

import torch
import torch.nn.functional as F

from transformers import GemmaConfig
from transformers.activations import ACT2FN
from transformers.models.gemma.modeling_gemma import GemmaRMSNorm, GemmaRotaryEmbedding, apply_rotary_pos_emb
from transformers.models.pi0.modeling_pi0 import PI0TimestepEmbeddings

f64 = torch.float64


def _t(a):
    return torch.as_tensor(a).to(f64)


def bf16_bits_to_f64(u16) -> torch.Tensor:
    """uint16 bf16 bit patterns (numpy) -> float64 tensor (exact)."""
    import numpy as np
    u = np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16
    return torch.from_numpy(u.view(np.float32).copy()).to(f64)


@torch.no_grad()
def ada_rms(x, scale, shift, eps=1e-6):
    n = GemmaRMSNorm(x.shape[-1], eps=eps).to(f64)
    with torch.no_grad():
        n.weight.copy_(scale)
    # GemmaRMSNorm normalises in float32 internally; keep that (it is the library's statement)
    return n(x).to(f64) + shift


@torch.no_grad()
def rope_cos_sin(positions, head_dim, base=10000.0):
    """(cos, sin) [len(positions)][head_dim] from transformers' rotary embedding."""
    cfg = GemmaConfig(head_dim=head_dim, hidden_size=head_dim, num_attention_heads=1, num_key_value_heads=1,
                      intermediate_size=4)
    cfg.rope_parameters["rope_theta"] = base
    r = GemmaRotaryEmbedding(cfg)
    pos = torch.as_tensor(positions)[None]
    c, s = r(torch.zeros(1, 1, head_dim), pos)
    return c[0].to(f64), s[0].to(f64)


def time_frequencies(dim, min_period=4e-3, max_period=4.0):
    cfg = types.SimpleNamespace(dit_config=types.SimpleNamespace(hidden_size=dim), min_period=min_period,
                                max_period=max_period)
    return PI0TimestepEmbeddings.compute_freqs(cfg)


@torch.no_grad()
def time_embedding(t, dim):
    """PI0TimestepEmbeddings.forward (float32 frequencies and arithmetic, as the library states it)."""
    cfg = types.SimpleNamespace(dit_config=types.SimpleNamespace(hidden_size=dim), min_period=4e-3, max_period=4.0)
    m = PI0TimestepEmbeddings(cfg)
    return m(torch.as_tensor(t, dtype=torch.float32))


@torch.no_grad()
def pi05_mods(S, w):
    """mods [S][NL][2][3D], mod_final [S][3D]; cond = silu(W_to silu(W_ti temb + b) + b)
    (src/pi05/hybrid_model.py:111-128). temb in float64 from the library's frequency formula."""
    D = w["w_ti"].shape[1]
    t = torch.tensor([1.0 - i / S for i in range(S)], dtype=f64)
    fr = torch.linspace(0.0, 1.0, D // 2, dtype=f64)
    period = 4e-3 * (4.0 / 4e-3) ** fr
    arg = (2 * torch.pi / period)[None] * t[:, None]
    temb = torch.cat([arg.sin(), arg.cos()], 1)
    cond = F.silu(F.linear(F.silu(F.linear(temb, _t(w["w_ti"]), _t(w["b_ti"]))), _t(w["w_to"]), _t(w["b_to"])))
    NL = w["w_in"].shape[0]
    mods = torch.stack([torch.stack([F.linear(cond, _t(w["w_in"][l]), _t(w["b_in"][l])),
                                     F.linear(cond, _t(w["w_post"][l]), _t(w["b_post"][l]))], 1)
                        for l in range(NL)], 1)
    return mods, F.linear(cond, _t(w["w_fin"]), _t(w["b_fin"]))


@torch.no_grad()
def pi05_denoise(w, x_t, *, Lp, Tv, S, NL, H, HD, mutate=None):
    """Same inputs as oracle.pi05_denoise (uint16 bf16 bits for weights and prefix K/V)."""
    W = {k: bf16_bits_to_f64(w[k]) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")}
    kpre, vpre = bf16_bits_to_f64(w["kpre"]), bf16_bits_to_f64(w["vpre"])
    mods, modf = _t(w["mods"]), _t(w["mod_final"])
    w_ain, b_ain, w_aout, b_aout = (_t(w[k]) for k in ("w_ain", "b_ain", "w_aout", "b_aout"))
    D = W["wq"].shape[2]
    cos, sin = rope_cos_sin(list(range(Lp, Lp + Tv)), HD)
    if mutate == "rope_sign":
        sin = -sin
    gelu = ACT2FN["gelu_pytorch_tanh"]
    dt = -1.0 / S
    x_t = _t(x_t).clone()
    if x_t.dim() == 2:
        x_t = x_t[None]
    for b in range(x_t.shape[0]):
        xt = x_t[b]
        for s in range(S):
            x = F.linear(xt, w_ain, b_ain)
            for l in range(NL):
                mi, mp = mods[s, l, 0], mods[s, l, 1]
                h = ada_rms(x, mi[:D], mi[D:2 * D])
                q = F.linear(h, W["wq"][l]).view(Tv, H, HD).transpose(0, 1)   # [H][Tv][HD]
                k = F.linear(h, W["wk"][l]).view(1, Tv, HD)
                v = F.linear(h, W["wv"][l]).view(1, Tv, HD)
                q, k = apply_rotary_pos_emb(q[None], k[None], cos[None], sin[None])
                q, k = q[0], k[0]
                K = torch.cat([kpre[b, l][None], k], 1)
                V = torch.cat([vpre[b, l][None], v], 1)
                sc = None if mutate != "attn_scale" else 1.0 / HD
                a = F.scaled_dot_product_attention(q[None], K[None].expand(1, H, -1, -1),
                                                   V[None].expand(1, H, -1, -1), scale=sc)[0]
                a = a.transpose(0, 1).reshape(Tv, H * HD)
                gate_in = mi[2 * D:] if mutate != "gate_swap" else mp[2 * D:]
                x = x + gate_in * F.linear(a, W["wo"][l])
                h = ada_rms(x, mp[:D], mp[D:2 * D])
                m = gelu(F.linear(h, W["wg"][l])) * F.linear(h, W["wu"][l])
                x = x + mp[2 * D:] * F.linear(m, W["wd"][l])
            mf = modf[s]
            h = ada_rms(x, mf[:D], mf[D:2 * D])
            xt = xt + dt * F.linear(h, w_aout, b_aout)
        x_t[b] = xt
    return x_t


@torch.no_grad()
def ma2_flow(w, x_t, *, Lk, Tv, S, NL, H, HD, adim, mutate=None):
    """Same inputs as oracle.ma2_flow (src/molmoact2/mk_ma2.cu:258-575)."""
    U = {k: bf16_bits_to_f64(w[k]) for k in ("w_qkv", "w_so", "w_cq", "w_co", "w_g", "w_u", "w_dn", "w_aout",
                                              "kctx", "vctx")}
    Fv = {k: _t(w[k]) for k in ("b_qkv", "b_so", "b_cq", "b_co", "b_g", "b_u", "b_dn", "mods", "mod_final",
                                 "w_ain", "b_ain", "b_aout")}
    D = H * HD
    # rope tables are kernel inputs here (built by the caller from the HF rotary cache,
    # benchmarks/molmoact2/eval_numerics.py:112-115): [Tv][HD/2] -> full split-half form
    cos = torch.cat([_t(w["rope_cos"])] * 2, -1)
    sin = torch.cat([_t(w["rope_sin"])] * 2, -1)
    silu = ACT2FN["silu"]
    dt = 1.0 / S
    x_t = _t(x_t).clone()
    if x_t.dim() == 2:
        x_t = x_t[None]

    def heads(y):
        return y.view(Tv, H, HD).transpose(0, 1)

    def qk_norm(y):  # per-head RMS without weight (mk_ma2.cu:300-315)
        return F.rms_norm(y, (HD,), eps=1e-6)

    for b in range(x_t.shape[0]):
        xt = x_t[b]
        for s in range(S):
            x = F.linear(xt, Fv["w_ain"], Fv["b_ain"])
            for l in range(NL):
                m = Fv["mods"][s, l]   # [3][3][D]: {msa, mca, mlp} x {scale, shift, gate}
                h = ada_rms(x, m[0, 0], m[0, 1])
                qkv = F.linear(h, U["w_qkv"][l], Fv["b_qkv"][l])
                q, k, v = heads(qkv[:, :D]), heads(qkv[:, D:2 * D]), heads(qkv[:, 2 * D:])
                q, k = qk_norm(q), qk_norm(k)
                q, k = apply_rotary_pos_emb(q[None], k[None], cos[None], sin[None])
                a = F.scaled_dot_product_attention(q, k, v[None])[0].transpose(0, 1).reshape(Tv, D)
                x = x + m[0, 2] * F.linear(a, U["w_so"][l], Fv["b_so"][l])
                h = ada_rms(x, m[1, 0], m[1, 1])
                qc = qk_norm(heads(F.linear(h, U["w_cq"][l], Fv["b_cq"][l])))
                kc = U["kctx"][b, l].view(Lk, H, HD).transpose(0, 1)
                vc = U["vctx"][b, l].view(Lk, H, HD).transpose(0, 1)
                c = F.scaled_dot_product_attention(qc[None], kc[None], vc[None])[0].transpose(0, 1).reshape(Tv, D)
                x = x + m[1, 2] * F.linear(c, U["w_co"][l], Fv["b_co"][l])
                h = ada_rms(x, m[2, 0], m[2, 1])
                mm = silu(F.linear(h, U["w_g"][l], Fv["b_g"][l])) * F.linear(h, U["w_u"][l], Fv["b_u"][l])
                x = x + m[2, 2] * F.linear(mm, U["w_dn"][l], Fv["b_dn"][l])
            mf = Fv["mod_final"][s]
            h = ada_rms(x, mf[0], mf[1])
            act = F.linear(h, U["w_aout"], Fv["b_aout"])
            upd = torch.zeros_like(xt)
            upd[:, :adim] = dt * act[:, :adim]
            xt = xt + upd
        x_t[b] = xt
    return x_t
