"""Synthetic openpi-style pi0.5 checkpoints (the key names the reference loads,
src/pi05/hybrid_model.py:94-132) for the policy wrapper tests."""
from __future__ import annotations

import torch

EXPERT = "paligemma_with_expert.gemma_expert.model."
BACKBONE = "paligemma_with_expert.paligemma.model.language_model."


def checkpoint(NL=2, seed=0, device="cpu", backbone=False, std=0.02):
    """{key: tensor}: bf16 GEMM weights and fp32 norm / time-MLP / action weights, N(0, std)."""
    g = torch.Generator(device=device).manual_seed(seed)
    n = lambda *s: (torch.randn(*s, generator=g, device=device) * std)  # noqa: E731
    b16 = lambda *s: n(*s).to(torch.bfloat16)  # noqa: E731
    sd = {}
    for i in range(NL):
        p = f"{EXPERT}layers.{i}."
        sd[p + "self_attn.q_proj.weight"] = b16(2048, 1024)
        sd[p + "self_attn.k_proj.weight"] = b16(256, 1024)
        sd[p + "self_attn.v_proj.weight"] = b16(256, 1024)
        sd[p + "self_attn.o_proj.weight"] = b16(1024, 2048)
        sd[p + "mlp.gate_proj.weight"] = b16(4096, 1024)
        sd[p + "mlp.up_proj.weight"] = b16(4096, 1024)
        sd[p + "mlp.down_proj.weight"] = b16(1024, 4096)
        for nm in ("input_layernorm", "post_attention_layernorm"):
            sd[p + nm + ".dense.weight"] = n(3072, 1024)
            sd[p + nm + ".dense.bias"] = n(3072)
    sd[EXPERT + "norm.dense.weight"] = n(3072, 1024)
    sd[EXPERT + "norm.dense.bias"] = n(3072)
    for nm in ("time_mlp_in", "time_mlp_out"):
        sd[nm + ".weight"] = n(1024, 1024)
        sd[nm + ".bias"] = n(1024)
    sd["action_in_proj.weight"] = n(1024, 32)
    sd["action_in_proj.bias"] = n(1024)
    sd["action_out_proj.weight"] = n(32, 1024)
    sd["action_out_proj.bias"] = n(32)
    if backbone:
        for i in range(NL):
            p = f"{BACKBONE}layers.{i}."
            sd[p + "self_attn.q_proj.weight"] = b16(2048, 2048)
            sd[p + "self_attn.k_proj.weight"] = b16(256, 2048)
            sd[p + "self_attn.v_proj.weight"] = b16(256, 2048)
            sd[p + "self_attn.o_proj.weight"] = b16(2048, 2048)
            sd[p + "mlp.gate_proj.weight"] = b16(16384, 2048)
            sd[p + "mlp.up_proj.weight"] = b16(16384, 2048)
            sd[p + "mlp.down_proj.weight"] = b16(2048, 16384)
            sd[p + "input_layernorm.weight"] = n(2048)
            sd[p + "post_attention_layernorm.weight"] = n(2048)
    return sd


MA2_EXPERT = "model.action_expert."  # any prefix: Ma2Policy finds it by the first block's qkv key


def ma2_checkpoint(c, prefix=MA2_EXPERT):
    """A MolmoAct2 expert state dict with the module names the reference packs from
    (benchmarks/molmoact2/eval_numerics.py:78-118), holding the weights of ma2_case.make_case ``c``."""
    w = c["w"]
    sd = {}
    for l in range(c["NL"]):
        b = f"{prefix}blocks.{l}."
        for name, key in (("self_attn.qkv", "qkv"), ("self_attn.out_proj", "so"), ("cross_attn.q_proj", "cq"),
                          ("cross_attn.out_proj", "co"), ("mlp.gate_proj", "g"), ("mlp.up_proj", "u"),
                          ("mlp.down_proj", "dn")):
            sd[b + name + ".weight"] = w["w_" + key][l].clone()
            sd[b + name + ".bias"] = w["b_" + key][l].clone()
    sd[prefix + "action_embed.weight"] = w["w_ain"].clone()
    sd[prefix + "action_embed.bias"] = w["b_ain"].clone()
    sd[prefix + "final_layer.linear.weight"] = w["w_aout"].clone()
    sd[prefix + "final_layer.linear.bias"] = w["b_aout"].clone()
    return sd
