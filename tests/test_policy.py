"""The policy wrapper's checkpoint loading on the CPU (construction launches no kernel).

The modulations the wrapper precomputes from the checkpoint's time-MLP and adaRMS dense layers
(src/pi05/hybrid_model.py:111-128) are checked against the oracle's fo_pi05_mods; the packed
weights against pack_weights of the same keys; a safetensors file against the in-memory dict."""
import numpy as np
import pytest
import torch

from flashact_amd import pi05, policy
from tests import policy_case as PC


@pytest.fixture(scope="module")
def sd():
    return PC.checkpoint(NL=2, seed=1)


def test_layer_count_and_backbone_prefix():
    keys = {f"{PC.EXPERT}layers.{i}.self_attn.q_proj.weight": None for i in range(3)}
    assert policy._count_layers(policy._Source(keys), PC.EXPERT) == 3
    for bp in (PC.BACKBONE, "paligemma_with_expert.paligemma.language_model.model."):
        src = policy._Source({bp + "layers.0.self_attn.q_proj.weight": torch.zeros(2048, 2048),
                              PC.EXPERT + "layers.0.self_attn.q_proj.weight": torch.zeros(2048, 1024)})
        assert policy.find_backbone_prefix(src) == bp
    assert policy.find_backbone_prefix(policy._Source({PC.EXPERT + "layers.0.self_attn.q_proj.weight":
                                                       torch.zeros(2048, 1024)})) is None


def test_mods_and_packing_from_checkpoint(sd):
    from oracle import oracle as O
    pol = policy.Pi05Policy(sd, num_steps=10, chunk_size=50, device="cpu", load_backbone=False)
    assert pol.num_layers == 2 and pol.backbone is None
    E = PC.EXPERT
    st = lambda n: torch.stack([sd[f"{E}layers.{i}.{n}"] for i in range(2)])  # noqa: E731
    npf = lambda t: t.float().numpy()  # noqa: E731
    mods, modf = O.pi05_mods(10, 2, 1024, npf(sd["time_mlp_in.weight"]), npf(sd["time_mlp_in.bias"]),
                             npf(sd["time_mlp_out.weight"]), npf(sd["time_mlp_out.bias"]),
                             npf(st("input_layernorm.dense.weight")), npf(st("input_layernorm.dense.bias")),
                             npf(st("post_attention_layernorm.dense.weight")),
                             npf(st("post_attention_layernorm.dense.bias")),
                             npf(sd[E + "norm.dense.weight"]), npf(sd[E + "norm.dense.bias"]))
    np.testing.assert_allclose(pol.mods.numpy(), mods, atol=1e-5, rtol=1e-4)
    np.testing.assert_allclose(pol.mod_final.numpy(), modf, atol=1e-5, rtol=1e-4)
    ref = pi05.pack_weights(st("self_attn.q_proj.weight"), st("self_attn.k_proj.weight"),
                            st("self_attn.v_proj.weight"), st("self_attn.o_proj.weight"),
                            st("mlp.gate_proj.weight"), st("mlp.up_proj.weight"), st("mlp.down_proj.weight"))
    for k in ("w1", "wo", "w2", "w3"):
        assert torch.equal(pol.packed[k], ref[k])
    assert torch.equal(pol.w_aout, sd["action_out_proj.weight"].float())


def test_safetensors_file_matches_dict(sd, tmp_path):
    from safetensors.torch import save_file
    f = tmp_path / "model.safetensors"
    save_file({k: v.contiguous() for k, v in sd.items()}, str(f))
    a = policy.Pi05Policy(sd, device="cpu", load_backbone=False)
    b = policy.Pi05Policy(str(f), device="cpu", load_backbone=False)
    assert torch.equal(a.mods, b.mods) and torch.equal(a.packed["w2"], b.packed["w2"])


def test_rejects_bad_arguments(sd):
    with pytest.raises(ValueError):
        policy.Pi05Policy(sd, device="cpu", initial_noise_mode="uniform")
    with pytest.raises(ValueError):
        policy.Pi05Policy(sd, device="cpu", chunk_size=65)
    with pytest.raises(KeyError):
        policy.Pi05Policy({"action_in_proj.weight": torch.zeros(1024, 32)}, device="cpu")
    pol = policy.Pi05Policy(sd, device="cpu", load_backbone=False, initial_noise_mode="zero", chunk_size=10)
    assert torch.count_nonzero(pol.initial_noise()) == 0
    with pytest.raises(ValueError):
        pol.predict()
    with pytest.raises(ValueError):
        pol.predict(torch.zeros(4, 2048))  # no backbone in this checkpoint
