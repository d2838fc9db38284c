"""Host-side logic of the pi0.5 shim (flashact_amd/pi05.py) on the CPU: packing, tables, caches."""
import os

import numpy as np
import torch

from flashact_amd import pi05
from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def test_qk_row_permutations_pair_rope_halves():
    qsrc, ksrc = pi05.qk_row_permutations()
    assert sorted(qsrc.tolist()) == list(range(2048)) and sorted(ksrc.tolist()) == list(range(256))
    for p in (0, 1, 127, 128, 1000, 1023):
        h, j = divmod(p, 128)
        assert qsrc[2 * p] == h * 256 + j and qsrc[2 * p + 1] == h * 256 + j + 128
    assert ksrc[2 * 5] == 5 and ksrc[2 * 5 + 1] == 133


def test_pack_weights_layout():
    g = torch.Generator().manual_seed(0)
    mk = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)  # noqa: E731
    wq, wk, wv = mk(1, 2048, 1024), mk(1, 256, 1024), mk(1, 256, 1024)
    wo, wg, wu, wd = mk(1, 1024, 2048), mk(1, 4096, 1024), mk(1, 4096, 1024), mk(1, 1024, 4096)
    p = pi05.pack_weights(wq, wk, wv, wo, wg, wu, wd)
    assert p["w1"].shape == (1, 2560, 1024) and p["w2"].shape == (1, 8192, 1024)
    assert torch.equal(p["w1"][0, 2 * 130], wq[0, 1 * 256 + 2]) and torch.equal(p["w1"][0, 2 * 130 + 1], wq[0, 258 + 128])
    assert torch.equal(p["w1"][0, 2048 + 2 * 7 + 1], wk[0, 135]) and torch.equal(p["w1"][0, 2304 + 9], wv[0, 9])
    assert torch.equal(p["w2"][0, 2 * 77], wg[0, 77]) and torch.equal(p["w2"][0, 2 * 77 + 1], wu[0, 77])
    assert torch.equal(p["wo"], wo) and torch.equal(p["w3"], wd)


def test_time_embedding_matches_oracle_and_golden():
    t = torch.tensor([1.0, 0.9, 0.5, 0.0])
    e = pi05.create_sinusoidal_pos_embedding(t, 1024).float().numpy()
    assert np.abs(e - O.sinusoid_embedding(t.numpy(), 1024)).max() <= 1e-6
    g = np.load(os.path.join(GOLD, "time_embedding.npz"))
    e = pi05.create_sinusoidal_pos_embedding(torch.from_numpy(g["t"]), 1024).float().numpy()
    assert np.abs(e - g["emb"]).max() <= 3e-4


def test_rope_table_matches_golden():
    g = np.load(os.path.join(GOLD, "rope_hd256.npz"))
    c, s = pi05.rope_table(968, 50)
    assert np.abs(c.numpy() - g["cos"][:50]).max() <= 3e-7 and np.abs(s.numpy() - g["sin"][:50]).max() <= 3e-7


def test_precompute_mods_matches_oracle():
    g = np.load(os.path.join(GOLD, "pi05_mods_small.npz"))
    keys = ("w_ti", "b_ti", "w_to", "b_to", "w_in", "b_in", "w_post", "b_post", "w_fin", "b_fin")
    m, mf = pi05.precompute_mods(int(g["S"]), *[torch.from_numpy(g[k]) for k in keys])
    assert np.abs(m.numpy() - g["mods"]).max() <= 1e-5 and np.abs(mf.numpy() - g["mod_final"]).max() <= 1e-5


def test_caches_and_compaction():
    NL, Lp, hd = 2, 7, 256
    kv = torch.randn(NL, 2, Lp, hd).to(torch.bfloat16)
    Lmax = pi05.lmax_for(Lp, 50)
    assert Lmax == 64 and pi05.lmax_for(968, 50) == 1024 and pi05.lmax_for(0, 1) == 16
    kc, vc = pi05.make_caches(kv, Lmax)
    assert kc.shape == (NL, Lmax, hd) and vc.shape == (NL, hd, Lmax)
    assert torch.equal(kc[:, :Lp], kv[:, 0]) and torch.equal(vc[:, :, :Lp], kv[:, 1].transpose(1, 2))
    assert not kc[:, Lp:].any() and not vc[:, :, Lp:].any()
    # compact_kv keeps the rows the pad mask marks valid, in order
    mask = torch.tensor([[1, 0, 1, 1, 0, 1, 1, 1, 1]], dtype=torch.bool)
    keys = [torch.randn(1, 1, 9, hd) for _ in range(NL)]
    vals = [torch.randn(1, 1, 9, hd) for _ in range(NL)]
    ckv = pi05.compact_kv(keys, vals, mask)
    assert ckv.shape == (NL, 2, 7, hd)
    assert torch.equal(ckv[1, 0], keys[1][0, 0][mask[0]].to(torch.bfloat16))
