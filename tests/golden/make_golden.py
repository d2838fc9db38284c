"""Writes the golden vectors under tests/golden/ (run: python tests/golden/make_golden.py).

The reference ships no test vectors for this path, so the fixtures come from third-party library
routines that restate its pieces (transformers' PI0TimestepEmbeddings and GemmaRotaryEmbedding) and
from the float64 PyTorch restatement of both loops (tests/torch_restatement.py), evaluated on the
seeded small cases of tests/small_cases.py. The fixtures hold inputs and expected outputs, so the
tests that read them need neither transformers nor the generator.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests import small_cases as C  # noqa: E402
from tests import torch_restatement as R  # noqa: E402


def main():
    # time embedding: PI0TimestepEmbeddings (float32 library statement) at the pi0.5 width
    t = np.array([1.0, 0.9, 0.5, 0.1, 0.0, 0.37], np.float32)
    emb = R.time_embedding(t, 1024).numpy()
    np.savez_compressed(os.path.join(HERE, "time_embedding.npz"), t=t, dim=np.int32(1024), emb=emb)

    # RoPE cos/sin from transformers' Gemma rotary embedding, head_dim 256, positions of the
    # benchmark's action tokens (968..1017) and of the largest supported prefix (8191)
    pos = np.array(list(range(968, 1018)) + [0, 1, 8191], np.int64)
    c, s = R.rope_cos_sin(pos.tolist(), 256)
    np.savez_compressed(os.path.join(HERE, "rope_hd256.npz"), pos=pos, cos=c[:, :128].float().numpy(),
                        sin=s[:, :128].float().numpy())

    # pi0.5 time MLP -> mods (float64)
    tw = C.pi05_time_weights(seed=3, NL=2, D=32)
    mods, modf = R.pi05_mods(4, tw)
    np.savez_compressed(os.path.join(HERE, "pi05_mods_small.npz"), S=np.int32(4), **tw,
                        mods=mods.numpy(), mod_final=modf.numpy())

    # whole loops (float64)
    w, x0, d = C.pi05_case(seed=11, **C.PI05_SMALL)
    out = R.pi05_denoise(w, x0, Lp=d["Lp"], Tv=d["Tv"], S=d["S"], NL=d["NL"], H=d["H"], HD=d["HD"]).numpy()
    np.savez_compressed(os.path.join(HERE, "pi05_small.npz"), **w, x0=x0, out=out,
                        dims=np.array([d[k] for k in ("NL", "D", "H", "HD", "F", "AD", "Lp", "Tv", "S")], np.int32))
    w, x0, d = C.ma2_case(seed=12, **C.MA2_SMALL)
    out = R.ma2_flow(w, x0, Lk=d["Lk"], Tv=d["Tv"], S=d["S"], NL=d["NL"], H=d["H"], HD=d["HD"],
                     adim=d["adim"]).numpy()
    np.savez_compressed(os.path.join(HERE, "ma2_small.npz"), **w, x0=x0, out=out,
                        dims=np.array([d[k] for k in ("NL", "D", "H", "HD", "F", "AD", "Lk", "Tv", "S", "adim")],
                                      np.int32))
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    torch.manual_seed(0)
    main()
