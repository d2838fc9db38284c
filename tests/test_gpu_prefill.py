"""pi0.5 prefix prefill (the benchmark's prefill workload) on the MI355X vs the CPU fp32 oracle.

Two gates:
  * the K/V cache the prefill writes (bf16) against the oracle's fp32 K/V of every layer:
    max-abs <= 4e-2 and mean-abs <= 4e-3 (K and V have unit scale here; a bf16 output alone is
    off by up to 2^-9 relative, and bf16 GEMM operands through the layers add about as much again);
  * end to end (prefill, then the 10-step-style denoise loop reading that cache) against the
    oracle chain, on the final actions, with the acceptance tolerance: max-abs <= 2e-2 and
    mean-abs <= 2e-3. The oracle chain casts its fp32 K/V to bf16 between the two stages, as the
    reference's hand-off does (src/pi05/pack_weights.py:70).
"""
import numpy as np
import pytest
import torch

from flashact_amd import pi05, prefill
from tests import pi05_case as P
from tests import prefill_case as C

KV_MAX, KV_MEAN = 4e-2, 4e-3
MAX_ABS, MEAN_ABS = 2e-2, 2e-3

pytestmark = pytest.mark.gpu


def _check_kv(c, kc, vt, K=None, V=None):
    if K is None:
        K, V = C.run_oracle(c)
    st = C.kv_diff(kc, vt, K, V, c["Lp"])
    print(f"prefill NL={c['NL']} Lp={c['Lp']} B={c['batch']}: {st}", flush=True)
    assert st["k_max"] <= KV_MAX and st["v_max"] <= KV_MAX, st
    assert st["k_mean"] <= KV_MEAN and st["v_mean"] <= KV_MEAN, st
    return st


def test_prefill_small(gpu):
    c = C.make_case(NL=2, Lp=200)
    Lmax = pi05.lmax_for(200, 50)
    kc, vt = C.run_gpu(c, gpu, Lmax=Lmax)
    ws = prefill.workspace(gpu, 1, 200, Lmax)
    assert prefill.read_status(ws) == 0
    _check_kv(c, kc, vt)
    # rows / columns past the prefix (the suffix slots of the denoise loop) are left alone
    assert torch.count_nonzero(kc[:, :, 200:]) == 0 and torch.count_nonzero(vt[:, :, :, 200:]) == 0


@pytest.mark.parametrize("Lp,B", [(1, 1), (17, 2), (129, 1), (256, 1), (300, 2)])  # 256: whole key chunks
def test_prefill_edge_shapes(gpu, Lp, B):
    c = C.make_case(NL=2, Lp=Lp, batch=B, seed=Lp)
    kc, vt = C.run_gpu(c, gpu)
    _check_kv(c, kc, vt)


@pytest.fixture(scope="module")
def config3(gpu):
    """The benchmark's prefill (18 layers, Lp = 968) on the GPU and in the oracle, shared by the
    full-depth K/V check and the full chain below (the oracle prefill is the slow part)."""
    c = C.make_case(NL=18, Lp=968)
    Lmax = pi05.lmax_for(968, 50)
    kc, vt = C.run_gpu(c, gpu, Lmax=Lmax)
    ws = prefill.workspace(gpu, 1, 968, Lmax)
    assert prefill.read_status(ws) == 0
    K, V = C.run_oracle(c)
    return c, kc, vt, K, V, Lmax


def test_prefill_config3_all_layers(config3):
    """The full benchmark prefill launch: K/V of every one of the 18 layers against the oracle.

    Through 18 layers of a 2048-wide residual stream the bf16 roundings compound: the error to the
    fp32 oracle grows from 1.7e-3 (layer 0) to about 8.7e-3 mean-abs (layer 17) for K and V of unit
    scale. Each layer is therefore held to the error of a restatement that rounds exactly where the
    kernel rounds (bf16 operands and bf16 K-split partials, prefill_case.run_bf16_floor) on the same
    inputs: mean-abs within 1.05x that floor + 1e-4 and max-abs within 1.5x + 5e-3; layers 0-1 also to
    the fixed gates (4e-2 max, 4e-3 mean). The mean-abs ratio to the floor is printed per layer."""
    c, kc, vt, K, V, _ = config3
    Kf, Vf = C.run_bf16_floor(c)
    for l in range(c["NL"]):
        st = C.kv_diff(kc[:, l:l + 1], vt[:, l:l + 1], K[:, l:l + 1], V[:, l:l + 1], c["Lp"])
        fk, fv = np.abs(Kf[:, l] - K[:, l]), np.abs(Vf[:, l] - V[:, l])
        fl = {"k_mean": float(fk.mean()), "k_max": float(fk.max()), "v_mean": float(fv.mean()), "v_max": float(fv.max())}
        ratio = {kv: st[f"{kv}_mean"] / max(fl[f"{kv}_mean"], 1e-30) for kv in ("k", "v")}
        print(f"config 3 prefill layer {l}: {st}; bf16 floor {fl}; mean-abs / floor K {ratio['k']:.3f} "
              f"V {ratio['v']:.3f}", flush=True)
        for kv in ("k", "v"):
            assert st[f"{kv}_mean"] <= 1.05 * fl[f"{kv}_mean"] + 1e-4, (l, kv, st, fl)
            assert st[f"{kv}_max"] <= 1.5 * fl[f"{kv}_max"] + 5e-3, (l, kv, st, fl)
        if l < 2:
            assert st["k_max"] <= KV_MAX and st["v_max"] <= KV_MAX, (l, st)
            assert st["k_mean"] <= KV_MEAN and st["v_mean"] <= KV_MEAN, (l, st)


def test_config3_full_chain(gpu, config3):
    """The benchmark prefill end to end at full size: the 18-layer prefill over 968 tokens writes the
    caches, the 18-layer, 10-step, Tv = 50 denoise loop reads them; final actions against the oracle
    chain (oracle prefill -> bf16 K/V -> oracle denoise), as eval_numerics.py:50-69 and :81-107 chain
    openpi's prefill, the cache fill and the loop."""
    pc, kc, vt, K, V, Lmax = config3
    Tv = 50
    dc = P.make_case(NL=18, Lp=968, Tv=Tv, S=10, seed=41)
    dc["inp"]["kpre"] = torch.from_numpy(K).to(torch.bfloat16)
    dc["inp"]["vpre"] = torch.from_numpy(V).to(torch.bfloat16)
    ref = P.run_oracle(dc)[0]
    g = P.gpu_tensors(dc, gpu)
    assert g["Lmax"] == Lmax
    g["caches"] = [(kc[0].clone(), vt[0].clone())]
    out = P.run_gpu(dc, gpu, g)[0]
    st = P.parity(out[:Tv], ref)
    print(f"config 3 full chain (18-layer prefill Lp=968 -> 18 layers x 10 steps, Tv={Tv}): {st}", flush=True)
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st


def test_prefill_batch_matches_single(gpu):
    c = C.make_case(NL=2, Lp=150, batch=3, seed=9)
    g = C.gpu_weights(c, gpu)
    kb, vb = C.run_gpu(c, gpu, g)
    for b in range(3):
        k1, v1 = C.run_gpu(c, gpu, g, samples=[b])
        assert torch.equal(k1[0], kb[b]) and torch.equal(v1[0], vb[b])


def test_prefill_deterministic(gpu):
    c = C.make_case(NL=2, Lp=333, seed=4)
    g = C.gpu_weights(c, gpu)
    a = C.run_gpu(c, gpu, g)
    b = C.run_gpu(c, gpu, g)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_config3_prefill_then_denoise(gpu):
    """Prefill writes the cache, the batch-1 denoise loop reads it; final actions vs the oracle chain."""
    Lp, Tv = 200, 50
    pc = C.make_case(NL=2, Lp=Lp, seed=7)
    K, V = C.run_oracle(pc)
    dc = P.make_case(NL=2, Lp=Lp, Tv=Tv, S=2, seed=8)
    dc["inp"]["kpre"] = torch.from_numpy(K).to(torch.bfloat16)
    dc["inp"]["vpre"] = torch.from_numpy(V).to(torch.bfloat16)
    ref = P.run_oracle(dc)[0]
    g = P.gpu_tensors(dc, gpu)
    kc, vt = C.run_gpu(pc, gpu, Lmax=g["Lmax"])
    g["caches"] = [(kc[0], vt[0])]
    out = P.run_gpu(dc, gpu, g)[0]
    st = P.parity(out[:Tv], ref)
    print(f"config 3 chain (NL=2, Lp={Lp}, Tv={Tv}, S=2): {st}", flush=True)
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st
