"""The policy wrapper end to end on the MI355X: checkpoint -> (prefill | K/V hand-off) -> denoise
loop -> raw action chunk, against the oracle chain on the same weights and inputs.
Tolerance as in the parity tests: max-abs <= 2e-2 and mean-abs <= 2e-3 on the chunk."""
import numpy as np
import pytest
import torch

from flashact_amd import pi05, policy
from tests import pi05_case as P
from tests import policy_case as PC

pytestmark = pytest.mark.gpu

NL, LP, T, S = 2, 200, 50, 2


def _oracle_chain(sd, pol, x, noise, K=None, V=None, fp8=False):
    from oracle import oracle as O
    E, B = PC.EXPERT, PC.BACKBONE
    st = lambda p, n: torch.stack([sd[f"{p}layers.{i}.{n}"] for i in range(NL)]).cpu()  # noqa: E731
    if K is None:
        cos0, sin0 = pi05.rope_table(0, LP)
        bw = {k: P.u16(st(B, f"{m}.weight")) for k, m in (("wq", "self_attn.q_proj"), ("wk", "self_attn.k_proj"),
                                                            ("wv", "self_attn.v_proj"), ("wo", "self_attn.o_proj"),
                                                            ("wg", "mlp.gate_proj"), ("wu", "mlp.up_proj"),
                                                            ("wd", "mlp.down_proj"))}
        bw.update(ln_in=st(B, "input_layernorm.weight").float().numpy(),
                  ln_post=st(B, "post_attention_layernorm.weight").float().numpy(),
                  rope_cos=cos0.numpy(), rope_sin=sin0.numpy())
        K, V = O.gemma_prefill(bw, x.cpu().numpy(), NL=NL)
        K = torch.from_numpy(K).to(torch.bfloat16)
        V = torch.from_numpy(V).to(torch.bfloat16)
    cos, sin = pi05.rope_table(LP, T)
    ew = {k: P.u16(st(E, f"{m}.weight")) for k, m in (("wq", "self_attn.q_proj"), ("wk", "self_attn.k_proj"),
                                                        ("wv", "self_attn.v_proj"), ("wo", "self_attn.o_proj"),
                                                        ("wg", "mlp.gate_proj"), ("wu", "mlp.up_proj"),
                                                        ("wd", "mlp.down_proj"))}
    f = lambda k: sd[k].float().cpu().numpy()  # noqa: E731
    ew.update(mods=pol.mods.cpu().numpy(), mod_final=pol.mod_final.cpu().numpy(), rope_cos=cos.numpy(),
              rope_sin=sin.numpy(), w_ain=f("action_in_proj.weight"), b_ain=f("action_in_proj.bias"),
              w_aout=f("action_out_proj.weight"), b_aout=f("action_out_proj.bias"),
              kpre=P.u16(K.reshape(1, NL, LP, 256)), vpre=P.u16(V.reshape(1, NL, LP, 256)))
    if fp8:  # the expert's per-row e4m3 codes and scales, natural layouts
        for n, m in (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
                     ("o", "self_attn.o_proj"), ("g", "mlp.gate_proj"), ("u", "mlp.up_proj"), ("d", "mlp.down_proj")):
            q, sc = pi05.quantize_fp8(st(E, f"{m}.weight"))
            ew["q" + n], ew["s" + n] = q.numpy(), sc.numpy()
        return O.pi05_denoise_fp8(ew, noise.cpu().numpy()[None], Lp=LP, Tv=T, S=S, NL=NL)[0]
    return O.pi05_denoise(ew, noise.cpu().numpy()[None], Lp=LP, Tv=T, S=S, NL=NL)[0]


@pytest.fixture(scope="module")
def setup(gpu):
    sd = PC.checkpoint(NL=NL, seed=3, device=gpu, backbone=True)
    pol = policy.Pi05Policy(sd, num_steps=S, chunk_size=T, device=gpu)
    g = torch.Generator(device=gpu).manual_seed(4)
    x = torch.randn(LP, 2048, generator=g, device=gpu)
    noise = torch.randn(T, 32, generator=g, device=gpu)
    return sd, pol, x, noise


def test_predict_from_prefix_hidden(setup):
    sd, pol, x, noise = setup
    assert pol.backbone is not None and pol.num_layers == NL
    out = pol.predict(x, noise=noise)
    ref = _oracle_chain(sd, pol, x, noise)
    st = P.parity(out, ref)
    print(f"policy prefill path: {st}", flush=True)
    assert st["max_abs"] <= 2e-2 and st["mean_abs"] <= 2e-3, st
    assert np.array_equal(out, pol.predict(x, noise=noise))  # deterministic


def test_predict_from_handoff_rows(setup):
    sd, pol, x, noise = setup
    g = torch.Generator().manual_seed(5)
    K = torch.randn(NL, LP, 256, generator=g).to(torch.bfloat16)
    V = torch.randn(NL, LP, 256, generator=g).to(torch.bfloat16)
    srows = LP + 5
    ksrc = torch.zeros(NL, srows, 256, dtype=torch.bfloat16)
    vsrc = torch.zeros(NL, srows, 256, dtype=torch.bfloat16)
    ksrc[:, :LP] = torch.stack([K[..., :128], K[..., 128:]], dim=-1).reshape(NL, LP, 256)
    vsrc[:, :LP] = V
    dev = x.device
    out = pol.predict(kv_rows=(ksrc.to(dev), vsrc.to(dev), LP), noise=noise)
    ref = _oracle_chain(sd, pol, x, noise, K, V)
    st = P.parity(out, ref)
    print(f"policy hand-off path: {st}", flush=True)
    assert st["max_abs"] <= 2e-2 and st["mean_abs"] <= 2e-3, st


def test_noise_modes(setup):
    sd, pol, x, noise = setup
    z = policy.Pi05Policy(sd, num_steps=S, chunk_size=T, device=x.device, initial_noise_mode="zero",
                          load_backbone=False)
    assert torch.count_nonzero(z.initial_noise()) == 0
    sc = policy.Pi05Policy(sd, num_steps=S, chunk_size=T, device=x.device, initial_noise_mode="scale",
                           initial_noise_scale=0.5, load_backbone=False)
    g1 = torch.Generator(device=x.device).manual_seed(9)
    g2 = torch.Generator(device=x.device).manual_seed(9)
    assert torch.allclose(sc.initial_noise(g1), 0.5 * pol.initial_noise(g2))


def test_predict_fp8_weights(setup):
    """weight_format="fp8": the expert runs FP8-W8A16 on the per-row e4m3 codes of the same checkpoint,
    against the oracle chain with the oracle's fp8 loop on those codes."""
    sd, pol, x, noise = setup
    pol8 = policy.Pi05Policy(sd, num_steps=S, chunk_size=T, device=x.device, weight_format="fp8")
    assert pol8.packed["w1"].dtype == torch.uint8 and "s1" in pol8.packed
    out = pol8.predict(x, noise=noise)
    ref = _oracle_chain(sd, pol8, x, noise, fp8=True)
    st = P.parity(out, ref)
    print(f"policy fp8 path: {st}", flush=True)
    assert st["max_abs"] <= 2e-2 and st["mean_abs"] <= 2e-3, st
    assert not np.array_equal(out, pol.predict(x, noise=noise))  # the weights really are quantised


def test_ma2_policy_predict(gpu):
    """MolmoAct2: checkpoint (module names) -> Ma2Policy.predict -> the chunk, against the oracle on the
    same weights; then with a boolean context mask, against the oracle on the rows the mask keeps."""
    from tests import ma2_case as M
    # 5 steps: with unit gates the bf16-operand error floor falls with the step size (1.4e-3 mean-abs
    # at 2 steps, close to the 2e-3 tolerance)
    c = M.make_case(NL=2, Lk=40, Tv=30, S=5, seed=9)
    sd = {k: v.to(gpu) for k, v in PC.ma2_checkpoint(c).items()}
    pol = policy.Ma2Policy(sd, num_steps=5, chunk_size=30, action_dims=c["adim"], device=gpu)
    kv = [(c["inp"]["kctx"][0, l][None], c["inp"]["vctx"][0, l][None]) for l in range(2)]
    out = pol.predict(kv, c["w"]["mods"], c["w"]["mod_final"], noise=c["inp"]["noise"][0])
    st = M.parity(out, M.run_oracle(c)[0], c["adim"])
    print(f"Ma2Policy.predict vs oracle: {st}", flush=True)
    assert st["max_abs"] <= 2e-2 and st["mean_abs"] <= 2e-3, st
    assert np.all(out[:, c["adim"]:] == 0)

    keep = torch.ones(40, dtype=torch.bool)
    keep[3::5] = False  # 8 of the 40 context rows masked out
    out_m = pol.predict(kv, c["w"]["mods"], c["w"]["mod_final"], cross_mask=keep, noise=c["inp"]["noise"][0])
    cm = dict(c)
    cm["inp"] = dict(c["inp"], kctx=c["inp"]["kctx"][:, :, keep], vctx=c["inp"]["vctx"][:, :, keep])
    cm["Lk"] = int(keep.sum())
    st_m = M.parity(out_m, M.run_oracle(cm)[0], c["adim"])
    print(f"Ma2Policy.predict with a context mask vs oracle on the kept rows: {st_m}", flush=True)
    assert st_m["max_abs"] <= 2e-2 and st_m["mean_abs"] <= 2e-3, st_m
    assert np.abs(out_m - out).max() > 0  # the mask changed the context
