"""Pins of the CPU oracle (oracle/fa_oracle.c), on the CPU.

The reference holds no golden vectors for this path, so the oracle is pinned by:
  * golden vectors in tests/golden/ made by third-party library routines (transformers'
    PI0TimestepEmbeddings and GemmaRotaryEmbedding) and by the float64 PyTorch restatement
    tests/torch_restatement.py (GemmaRMSNorm, apply_rotary_pos_emb, torch SDPA, GELUTanh);
  * the live restatement on further seeds and edge shapes, with planted mistakes that must fail;
  * closed forms and invariants: all-zero weights, prefix permutation, batch independence,
    the Euler schedule rebuilt from single steps, masked action dims.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests import small_cases as C

GOLD = os.path.join(os.path.dirname(__file__), "golden")
TOL = 2e-5  # fp32 oracle vs float64 statement, outputs of magnitude ~5


def _load(name):
    z = np.load(os.path.join(GOLD, name))  # allow_pickle=False (numpy default)
    return {k: z[k] for k in z.files}


def _pi05(w, x0, d):
    return O.pi05_denoise(w, x0, Lp=d["Lp"], Tv=d["Tv"], S=d["S"], NL=d["NL"], D=d["D"], H=d["H"], HD=d["HD"],
                          F=d["F"], AD=d["AD"])


def _ma2(w, x0, d):
    return O.ma2_flow(w, x0, Lk=d["Lk"], Tv=d["Tv"], S=d["S"], NL=d["NL"], adim=d["adim"], D=d["D"], H=d["H"],
                      HD=d["HD"], F=d["F"], AD=d["AD"])


# ------------------------------------------------------------------ golden vectors
def test_golden_time_embedding():
    """PI0TimestepEmbeddings evaluates in float32 (arguments up to 1571 rad), hence 3e-4."""
    g = _load("time_embedding.npz")
    e = O.sinusoid_embedding(g["t"], int(g["dim"]))
    assert np.abs(e - g["emb"]).max() <= 3e-4
    # the first half is sin, the second cos: at t = 0 exactly [0...0, 1...1]
    z = O.sinusoid_embedding(np.zeros(1, np.float32), 1024)
    assert np.all(z[0, :512] == 0) and np.all(z[0, 512:] == 1)


def test_golden_rope_table():
    g = _load("rope_hd256.npz")
    for i, p in enumerate(g["pos"]):
        c, s = O.rope_table(int(p), 1, 256)
        assert np.abs(c[0] - g["cos"][i]).max() <= 3e-7 and np.abs(s[0] - g["sin"][i]).max() <= 3e-7, p
    c, s = O.rope_table(968, 50, 256)
    assert np.abs(c * c + s * s - 1).max() < 1e-6


def test_golden_time_mlp_mods():
    g = _load("pi05_mods_small.npz")
    keys = ("w_ti", "b_ti", "w_to", "b_to", "w_in", "b_in", "w_post", "b_post", "w_fin", "b_fin")
    m, mf = O.pi05_mods(int(g["S"]), g["w_in"].shape[0], g["w_ti"].shape[0], *[g[k] for k in keys])
    assert np.abs(m - g["mods"]).max() <= 1e-5 and np.abs(mf - g["mod_final"]).max() <= 1e-5


def test_golden_pi05_loop():
    g = _load("pi05_small.npz")
    d = dict(zip(("NL", "D", "H", "HD", "F", "AD", "Lp", "Tv", "S"), map(int, g["dims"])))
    out = _pi05(g, g["x0"], d)
    assert np.abs(g["out"] - g["x0"]).max() > 1.0  # the loop moves the actions
    assert np.abs(out - g["out"]).max() <= TOL


def test_golden_ma2_loop():
    g = _load("ma2_small.npz")
    d = dict(zip(("NL", "D", "H", "HD", "F", "AD", "Lk", "Tv", "S", "adim"), map(int, g["dims"])))
    out = _ma2(g, g["x0"], d)
    assert np.abs(g["out"] - g["x0"]).max() > 1.0
    assert np.abs(out - g["out"]).max() <= TOL


# ------------------------------------------------------------------ live restatement
R = pytest.importorskip("tests.torch_restatement", reason="transformers blocks unavailable")


@pytest.mark.parametrize("shape", [dict(), dict(Lp=0, Tv=1, S=1), dict(Lp=40, Tv=9, S=2, NL=1, B=1)])
def test_pi05_matches_restatement(shape):
    kw = dict(C.PI05_SMALL, **shape)
    w, x0, d = C.pi05_case(seed=21, **kw)
    ref = R.pi05_denoise(w, x0, Lp=d["Lp"], Tv=d["Tv"], S=d["S"], NL=d["NL"], H=d["H"], HD=d["HD"]).numpy()
    assert np.abs(_pi05(w, x0, d) - ref).max() <= TOL


@pytest.mark.parametrize("mistake", ["rope_sign", "attn_scale", "gate_swap"])
def test_pi05_planted_mistakes_are_caught(mistake):
    """A restatement with one planted mistake must miss the oracle by far more than TOL."""
    w, x0, d = C.pi05_case(seed=22, **C.PI05_SMALL)
    bad = R.pi05_denoise(w, x0, Lp=d["Lp"], Tv=d["Tv"], S=d["S"], NL=d["NL"], H=d["H"], HD=d["HD"],
                         mutate=mistake).numpy()
    assert np.abs(_pi05(w, x0, d) - bad).max() > 100 * TOL


def test_ma2_matches_restatement():
    w, x0, d = C.ma2_case(seed=23, **C.MA2_SMALL)
    ref = R.ma2_flow(w, x0, Lk=d["Lk"], Tv=d["Tv"], S=d["S"], NL=d["NL"], H=d["H"], HD=d["HD"],
                     adim=d["adim"]).numpy()
    assert np.abs(_ma2(w, x0, d) - ref).max() <= TOL


# ------------------------------------------------------------------ closed forms / invariants
@pytest.mark.parametrize("S", [1, 4, 10])
def test_pi05_zero_weights_closed_form(S):
    """All matrices zero: x stays b_ain through the layers, v = b_aout, so x_S = x_0 - b_aout."""
    w, x0, d = C.pi05_case(seed=24, **dict(C.PI05_SMALL, S=S))
    for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"):
        w[k] = np.zeros_like(w[k])
    w["w_ain"] = np.zeros_like(w["w_ain"])
    w["w_aout"] = np.zeros_like(w["w_aout"])
    out = _pi05(w, x0, d)
    assert np.abs(out - (x0 - w["b_aout"])).max() <= 1e-5 * S


def test_pi05_prefix_permutation_invariance():
    """Prefix keys are pre-RoPE'd and unmasked: a joint row permutation changes nothing."""
    w, x0, d = C.pi05_case(seed=25, **C.PI05_SMALL)
    perm = np.random.default_rng(0).permutation(d["Lp"])
    w2 = dict(w, kpre=np.ascontiguousarray(w["kpre"][:, :, perm]), vpre=np.ascontiguousarray(w["vpre"][:, :, perm]))
    assert np.abs(_pi05(w, x0, d) - _pi05(w2, x0, d)).max() <= 1e-5
    # permuting K alone does change the result (the check has power)
    w3 = dict(w, kpre=np.ascontiguousarray(w["kpre"][:, :, perm]))
    assert np.abs(_pi05(w, x0, d) - _pi05(w3, x0, d)).max() > 1e-3


def test_pi05_batch_independence():
    w, x0, d = C.pi05_case(seed=26, **C.PI05_SMALL)
    both = _pi05(w, x0, d)
    for b in range(x0.shape[0]):
        wb = dict(w, kpre=np.ascontiguousarray(w["kpre"][b:b + 1]), vpre=np.ascontiguousarray(w["vpre"][b:b + 1]))
        assert np.array_equal(_pi05(wb, x0[b:b + 1], d), both[b:b + 1])


def test_pi05_euler_schedule_from_single_steps():
    """S steps of dt = -1/S with mods[s] at step s, rebuilt from S=1 launches (dt = -1)."""
    w, x0, d = C.pi05_case(seed=27, **dict(C.PI05_SMALL, S=3))
    full = _pi05(w, x0, d)
    x = x0.astype(np.float64)
    for s in range(3):
        ws = dict(w, mods=np.ascontiguousarray(w["mods"][s:s + 1]),
                  mod_final=np.ascontiguousarray(w["mod_final"][s:s + 1]))
        y = _pi05(ws, x.astype(np.float32), dict(d, S=1))   # y = x - v
        x = x + (y - x) / 3.0                               # x + dt v with dt = -1/3
    assert np.abs(full - x).max() <= 1e-5


def test_ma2_masked_dims_and_permutation():
    w, x0, d = C.ma2_case(seed=28, **C.MA2_SMALL)
    out = _ma2(w, x0, d)
    assert np.array_equal(out[..., d["adim"]:], x0[..., d["adim"]:])
    perm = np.random.default_rng(1).permutation(d["Lk"])
    w2 = dict(w, kctx=np.ascontiguousarray(w["kctx"][:, :, perm]), vctx=np.ascontiguousarray(w["vctx"][:, :, perm]))
    assert np.abs(_ma2(w2, x0, d) - out).max() <= 1e-5
