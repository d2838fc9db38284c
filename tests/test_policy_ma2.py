"""MolmoAct2 policy wrapper on the CPU: the module-name key map and packing (against ma2.pack_weights
on the same tensors, bit for bit), the expert-prefix search, and argument validation before any launch."""
import pytest
import torch

from flashact_amd import ma2, policy
from tests import ma2_case as M
from tests import policy_case as PC


@pytest.fixture(scope="module")
def case():
    c = M.make_case(NL=2, Lk=40, Tv=30, S=2, seed=7)
    return c, PC.ma2_checkpoint(c)


def test_key_map_and_packing(case):
    c, sd = case
    pol = policy.Ma2Policy(sd, num_steps=2, chunk_size=30, device="cpu")
    assert pol.num_layers == 2
    w = c["w"]
    ws, bs = ma2.pack_weights(w["w_qkv"], w["w_so"], w["w_cq"], w["w_co"], w["w_g"], w["w_u"], w["w_dn"],
                              w["b_qkv"], w["b_so"], w["b_cq"], w["b_co"], w["b_g"], w["b_u"], w["b_dn"])
    for a, b in zip(pol.ws + pol.bs, ws + bs):
        assert a.dtype == b.dtype and torch.equal(a, b)
    # gate/up interleaved: row 2f is gate f, row 2f + 1 up f
    assert torch.equal(pol.ws[4][1, 10], w["w_g"][1, 5].to(torch.bfloat16))
    assert torch.equal(pol.ws[4][1, 11], w["w_u"][1, 5].to(torch.bfloat16))
    assert torch.equal(pol.w_ain, w["w_ain"].float()) and torch.equal(pol.b_aout, w["b_aout"].float())
    assert pol.w_aout.dtype == torch.bfloat16 and torch.equal(pol.w_aout, w["w_aout"].to(torch.bfloat16))


def test_prefix_search_and_missing_keys(case):
    c, _ = case
    sd = PC.ma2_checkpoint(c, prefix="")
    assert policy.find_ma2_prefix(sd) == ""
    assert policy.Ma2Policy(sd, num_steps=2, device="cpu").num_layers == 2
    assert policy.find_ma2_prefix({"x.weight": torch.zeros(1)}) is None
    with pytest.raises(KeyError):
        policy.Ma2Policy({"x.weight": torch.zeros(1)}, device="cpu")
    bad = dict(sd)
    bad["blocks.1.mlp.down_proj.weight"] = torch.zeros(768, 1024)
    with pytest.raises(ValueError, match="down_proj"):
        policy.Ma2Policy(bad, device="cpu")


def test_predict_validates_before_launch(case):
    c, sd = case
    pol = policy.Ma2Policy(sd, num_steps=2, chunk_size=30, device="cpu")
    kv = [(c["inp"]["kctx"][0, l][None], c["inp"]["vctx"][0, l][None]) for l in range(2)]
    with pytest.raises(ValueError, match="layers"):
        pol.predict(kv[:1], c["w"]["mods"], c["w"]["mod_final"])
    with pytest.raises(ValueError, match="mods"):
        pol.predict(kv, c["w"]["mods"][:1], c["w"]["mod_final"])
    with pytest.raises(ValueError, match="noise"):
        pol.predict(kv, c["w"]["mods"], c["w"]["mod_final"], noise=torch.zeros(10, 32))
    with pytest.raises(ValueError):
        policy.Ma2Policy(sd, chunk_size=65, device="cpu")
