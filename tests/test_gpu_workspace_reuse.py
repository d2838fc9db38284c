"""One workspace shared by every entry point and shape, on the MI355X, vs the CPU fp32 oracle.

The batch-1 kernels exchange parity-tagged partial sums through the workspace; the layout kernels
(batched pi0.5, generic MolmoAct2) keep shape-dependent data and split-K counters there. A caller
may hand the same workspace to any sequence of launches (the C ABI only asks that it be large
enough), so each launch below must agree with the oracle whatever ran before it: a growing token
count on the batch-1 kernel, the generic kernel between two batch-1 launches, a change of batch and
shape on the generic kernel, and the other model family in between.
Tolerance as in the parity tests: max-abs <= 2e-2 and mean-abs <= 2e-3.
"""
import ctypes

import numpy as np
import pytest
import torch

from flashact_amd import _lib, ma2, pi05
from tests import ma2_case as C
from tests import pi05_case as P

MAX_ABS, MEAN_ABS = 2e-2, 2e-3

pytestmark = pytest.mark.gpu

MA2_SEQ = [  # (batch, Lk, Tv, S, adim); batch 1 with Tv <= 32 runs the batch-1 kernel
    (1, 100, 8, 2, 6),
    (1, 200, 30, 2, 6),   # more tokens than the launch before
    (1, 100, 40, 2, 6),   # generic kernel at batch 1; at S = 1 a numpy model of the kernel's bf16
                          # rounding points puts this case at 1.96e-3 mean-abs, i.e. on the floor
    (1, 200, 30, 2, 6),   # batch-1 kernel after the generic one
    (3, 200, 17, 2, 5),   # generic, small tiles with split-K counters
    (2, 129, 33, 1, 1),   # generic, another layout
    (1, 50, 31, 2, 32),   # all 32 dims integrated; at S = 1 (one Euler step of dt = 1) this
                          # case sits at the bf16-operand floor of ~2e-3 mean-abs
]
PI05_SEQ = [(1, 200, 50, 2), (2, 200, 50, 2), (1, 150, 20, 1), (1, 150, 64, 1)]  # (batch, Lp, Tv, S)


def _shared_workspace(gpu):
    L = _lib.lib()
    need = max([L.fa_ma2_workspace_bytes(b, tv, ma2.lkmax_for(lk)) for b, lk, tv, _, _ in MA2_SEQ] +
               [L.fa_pi05_workspace_bytes(b, tv, pi05.lmax_for(lp, tv)) for b, lp, tv, _ in PI05_SEQ])
    raw = torch.empty(need + 256, dtype=torch.uint8, device=gpu)
    off = (-raw.data_ptr()) % 256
    ws = raw[off:off + need]
    _lib.check(L.fa_ma2_workspace_init(ctypes.c_void_p(ws.data_ptr()), need,
                                       ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)),
               "fa_ma2_workspace_init")
    return ws


def _ma2(gpu, ws, B, Lk, Tv, S, adim, seed):
    c = C.make_case(NL=2, Lk=Lk, Tv=Tv, S=S, adim=adim, batch=B, seed=seed)
    out = C.run_gpu(c, gpu, ws=ws)
    assert ma2.read_status(ws) == 0
    ref = C.run_oracle(c)
    for b in range(B):
        st = C.parity(out[b, :Tv], ref[b], adim)
        print(f"ma2 B={B} Lk={Lk} Tv={Tv} S={S} sample {b}: {st}", flush=True)
        assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, (B, Lk, Tv, b, st)


def _pi05(gpu, ws, B, Lp, Tv, S, seed):
    c = P.make_case(NL=2, Lp=Lp, Tv=Tv, S=S, batch=B, seed=seed)
    out = P.run_gpu_batched(c, gpu, ws=ws)[0] if B > 1 else P.run_gpu(c, gpu, ws=ws)[0][None]
    assert pi05.read_status(ws) == 0
    ref = P.run_oracle(c)
    for b in range(B):
        st = P.parity(out[b, :Tv], ref[b])
        print(f"pi05 B={B} Lp={Lp} Tv={Tv} S={S} sample {b}: {st}", flush=True)
        assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, (B, Lp, Tv, b, st)


def test_ma2_shape_sequence_one_workspace(gpu):
    ws = _shared_workspace(gpu)
    for i, (B, Lk, Tv, S, adim) in enumerate(MA2_SEQ):
        _ma2(gpu, ws, B, Lk, Tv, S, adim, seed=11 + i)


def test_both_models_one_workspace(gpu):
    ws = _shared_workspace(gpu)
    _pi05(gpu, ws, *PI05_SEQ[0], seed=21)
    _ma2(gpu, ws, *MA2_SEQ[1], seed=22)
    _pi05(gpu, ws, *PI05_SEQ[1], seed=23)
    _pi05(gpu, ws, *PI05_SEQ[0], seed=24)
    _ma2(gpu, ws, *MA2_SEQ[0], seed=25)
    _pi05(gpu, ws, *PI05_SEQ[2], seed=26)
    _ma2(gpu, ws, *MA2_SEQ[4], seed=27)
    _ma2(gpu, ws, *MA2_SEQ[1], seed=28)


def test_pi05_shape_sequence_one_workspace(gpu):
    """pi0.5 on one workspace: a growing token count on the batch-1 kernel, the batched kernel in
    between, then batch 1 again at the largest token count."""
    ws = _shared_workspace(gpu)
    for i, (B, Lp, Tv, S) in enumerate([(1, 200, 20, 2), (1, 200, 50, 2), (2, 150, 33, 1), (1, 150, 64, 1)]):
        _pi05(gpu, ws, B, Lp, Tv, S, seed=41 + i)
