"""Pins of the CPU oracle's Gemma prefix prefill (oracle/fa_oracle.c: fo_gemma_prefill).

openpi, whose PaliGemma forward the reference calls for the prefill
(benchmarks/pi05/eval_numerics.py:50-57), is absent, so the restatement is pinned against an
independent implementation of the same layer: transformers' GemmaDecoderLayer (fp32, eager
attention, no mask: the prefix attends to itself), with the per-layer K/V read from its cache
exactly as the reference's compact_kv does (src/pi05/pack_weights.py:60-70). A wrong RoPE pairing,
a norm without the (1 + w) scale, a causal mask, a missing residual or the wrong MLP activation
each move K/V of the second layer far beyond the tolerance.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

tf = pytest.importorskip("transformers")
from transformers import DynamicCache, GemmaConfig  # noqa: E402
from transformers.models.gemma.modeling_gemma import GemmaDecoderLayer, GemmaRotaryEmbedding  # noqa: E402

NL, D, H, HD, F, LP = 3, 64, 4, 16, 96, 13


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def _hf_model(seed=0):
    cfg = GemmaConfig(hidden_size=D, intermediate_size=F, num_hidden_layers=NL, num_attention_heads=H,
                      num_key_value_heads=1, head_dim=HD, rms_norm_eps=1e-6, hidden_activation="gelu_pytorch_tanh",
                      attention_bias=False, vocab_size=16)
    cfg._attn_implementation = "eager"
    g = torch.Generator().manual_seed(seed)
    layers = []
    for i in range(NL):
        layer = GemmaDecoderLayer(cfg, i).float().eval()
        with torch.no_grad():
            for p in layer.parameters():  # bf16-representable weights, non-zero norm weights
                p.copy_((torch.randn(p.shape, generator=g) * (0.3 if p.dim() == 1 else 0.2)).to(torch.bfloat16).float())
        layers.append(layer)
    return cfg, layers


def _oracle_weights(layers, cos, sin):
    st = lambda f: torch.stack([f(l) for l in layers])  # noqa: E731
    return dict(wq=_bf16_bits(st(lambda l: l.self_attn.q_proj.weight)),
                wk=_bf16_bits(st(lambda l: l.self_attn.k_proj.weight)),
                wv=_bf16_bits(st(lambda l: l.self_attn.v_proj.weight)),
                wo=_bf16_bits(st(lambda l: l.self_attn.o_proj.weight)),
                wg=_bf16_bits(st(lambda l: l.mlp.gate_proj.weight)),
                wu=_bf16_bits(st(lambda l: l.mlp.up_proj.weight)),
                wd=_bf16_bits(st(lambda l: l.mlp.down_proj.weight)),
                ln_in=st(lambda l: l.input_layernorm.weight).detach().numpy(),
                ln_post=st(lambda l: l.post_attention_layernorm.weight).detach().numpy(),
                rope_cos=cos, rope_sin=sin)


def _hf_kv(cfg, layers, x):
    pos = torch.arange(LP)[None]
    cos, sin = GemmaRotaryEmbedding(cfg)(x, pos)
    cache = DynamicCache()
    h = x
    with torch.no_grad():
        for layer in layers:
            out = layer(h, attention_mask=None, position_ids=pos, past_key_values=cache, use_cache=True,
                        position_embeddings=(cos, sin))
            h = out[0] if isinstance(out, tuple) else out
    K = torch.stack([cache.layers[i].keys[0, 0] for i in range(NL)]).numpy()
    V = torch.stack([cache.layers[i].values[0, 0] for i in range(NL)]).numpy()
    return K, V, cos[0].numpy(), sin[0].numpy()


def test_rope_table_matches_transformers():
    cfg, _ = _hf_model()
    cos, sin = GemmaRotaryEmbedding(cfg)(torch.zeros(1, LP, D), torch.arange(LP)[None])
    c = np.zeros((LP, HD // 2), np.float32)
    s = np.zeros((LP, HD // 2), np.float32)
    O.lib().fo_rope_table(0, LP, HD, __import__("ctypes").c_double(10000.0), O._p(c, np.float32), O._p(s, np.float32))
    np.testing.assert_allclose(c, cos[0, :, :HD // 2].numpy(), atol=2e-6)
    np.testing.assert_allclose(s, sin[0, :, :HD // 2].numpy(), atol=2e-6)
    # transformers' table repeats the half-table: pairs (j, j + HD/2) share one angle
    np.testing.assert_array_equal(cos[0, :, :HD // 2].numpy(), cos[0, :, HD // 2:].numpy())


def test_prefill_kv_matches_transformers_gemma_layers():
    cfg, layers = _hf_model()
    x = torch.randn(1, LP, D, generator=torch.Generator().manual_seed(1))
    Kh, Vh, cos, sin = _hf_kv(cfg, layers, x)
    w = _oracle_weights(layers, np.ascontiguousarray(cos[:, :HD // 2]), np.ascontiguousarray(sin[:, :HD // 2]))
    K, V = O.gemma_prefill(w, x.numpy(), NL=NL, D=D, H=H, HD=HD, F=F)
    assert K.shape == (1, NL, LP, HD)
    for l in range(NL):
        scale = max(np.abs(Kh[l]).max(), np.abs(Vh[l]).max())
        np.testing.assert_allclose(K[0, l], Kh[l], atol=2e-5 * scale, rtol=0, err_msg=f"K layer {l}")
        np.testing.assert_allclose(V[0, l], Vh[l], atol=2e-5 * scale, rtol=0, err_msg=f"V layer {l}")
    # the layers really interact: a later layer's K/V depend on the earlier layers' outputs
    assert np.abs(K[0, 2] - K[0, 1]).max() > 0.1 * np.abs(K[0, 2]).max()


def test_prefill_batch_is_per_sample():
    cfg, layers = _hf_model(seed=3)
    x = torch.randn(2, LP, D, generator=torch.Generator().manual_seed(4))
    _, _, cos, sin = _hf_kv(cfg, layers, x[:1])
    w = _oracle_weights(layers, np.ascontiguousarray(cos[:, :HD // 2]), np.ascontiguousarray(sin[:, :HD // 2]))
    K2, V2 = O.gemma_prefill(w, x.numpy(), NL=NL, D=D, H=H, HD=HD, F=F)
    for b in range(2):
        K1, V1 = O.gemma_prefill(w, x[b].numpy(), NL=NL, D=D, H=H, HD=HD, F=F)
        np.testing.assert_array_equal(K2[b], K1[0])
        np.testing.assert_array_equal(V2[b], V1[0])
