"""MolmoAct2 flow loop on the MI355X vs the CPU fp32 oracle (parity gate).

Tolerance (the acceptance tolerance for bf16 operands with fp32 accumulation vs the fp32 oracle, on the
final actions, integrated dims [0, adim)): max-abs <= 2e-2 and mean-abs <= 2e-3.
"""
import numpy as np
import pytest

from tests import ma2_case as C
from flashact_amd import ma2

MAX_ABS, MEAN_ABS = 2e-2, 2e-3

pytestmark = pytest.mark.gpu


def _check(c, gpu, **kw):
    ref = C.run_oracle(c)
    out = C.run_gpu(c, gpu, **kw)
    ws = ma2.workspace(gpu, c["batch"], c["Tv"], ma2.lkmax_for(c["Lk"]))
    assert ma2.read_status(ws) == 0
    assert np.isfinite(out).all()
    for b in range(c["batch"]):
        st = C.parity(out[b, :c["Tv"]], ref[b], c["adim"])
        print(f"B={c['batch']} sample {b} NL={c['NL']} Lk={c['Lk']} Tv={c['Tv']} S={c['S']}: {st}", flush=True)
        assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, (b, st)
        # dims past adim are left as they were (the noise is zero there)
        assert np.all(out[b, :c["Tv"], c["adim"]:] == c["inp"]["noise"][b, :, c["adim"]:].numpy())
    return out, ref


def test_ma2_small(gpu):
    _check(C.make_case(NL=2, Lk=493, Tv=30, S=2), gpu)


def test_ma2_config4_bs1(gpu):
    """The MolmoAct2 benchmark workload at batch 1: 36 layers, Lk=493, Tv=30, adim=6, 10 steps."""
    _check(C.make_case(NL=36, Lk=493, Tv=30, S=10), gpu)


# Batch 1 runs the XCD-local kernel up to Tv = 32 and Lk = 512: (1, 512, 32) fills every token lane
# and context rank; (1, 65, 17) leaves one token in the second token tile and a ragged key chunk.
# (1, 300, 40) runs the generic kernel's small-tile path with four waves per cross-attention item.
@pytest.mark.parametrize("B,Lk,Tv,S,adim", [(1, 1, 1, 2, 6), (2, 700, 64, 1, 32), (3, 37, 17, 2, 5),
                                            (1, 128, 16, 1, 6), (2, 129, 33, 1, 1), (1, 512, 32, 2, 6),
                                            (1, 65, 17, 2, 7), (1, 300, 40, 2, 6)])
def test_ma2_edge_shapes(gpu, B, Lk, Tv, S, adim):
    _check(C.make_case(NL=2, Lk=Lk, Tv=Tv, S=S, adim=adim, batch=B, seed=Lk + Tv), gpu)


def test_ma2_batch16(gpu):
    """The MolmoAct2 benchmark workload at batch 16 (the large-tile path) at full depth, 36 layers x 10 steps, every
    sample against the oracle (benchmarks/molmoact2/eval_numerics.py:147-159 is the reference's
    fidelity check of the same loop)."""
    _check(C.make_case(NL=36, Lk=493, Tv=30, S=10, batch=16), gpu)


def test_ma2_batch16_shallow(gpu):
    """Batch 16 at 2 layers and 2 steps: a quick first signal before the full-depth case."""
    _check(C.make_case(NL=2, Lk=493, Tv=30, S=2, batch=16), gpu)


def test_ma2_batched_matches_single(gpu):
    c = C.make_case(NL=2, Lk=200, Tv=30, S=2, batch=3, seed=5)
    g = C.gpu_tensors(c, gpu)
    outb = C.run_gpu(c, gpu, g)
    for b in range(3):
        out1 = C.run_gpu(c, gpu, g, samples=[b])[0]
        assert np.abs(out1 - outb[b]).max() <= MAX_ABS


def test_ma2_deterministic(gpu):
    c = C.make_case(NL=2, Lk=300, Tv=30, S=2)
    g = C.gpu_tensors(c, gpu)
    assert np.array_equal(C.run_gpu(c, gpu, g), C.run_gpu(c, gpu, g))


def test_ma2_padded_rows_untouched(gpu):
    c = C.make_case(NL=1, Lk=50, Tv=10, S=1)
    out = C.run_gpu(c, gpu, xt_rows=16)
    assert np.all(out[:, 10:] == 0.0)
