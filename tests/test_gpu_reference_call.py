"""The reference's own pi0.5 call, replayed through the drop-in ``launch``.

benchmarks/pi05/eval_numerics.py:71-107 builds: per-row e4m3 codes (uint8) with fp32 row scales,
fp16 caches kcache [NL][Lmax][256] / vtcache [NL][256][Lmax] with Lmax = ceil16(Lp + T), x_t of
T = 16 rows of which Tv = 10 are valid, the fp32 / fp16 scratch tensors x, xp, xn, q, attn, hmlp,
scores, probs, an int64 stage counter, empty bf16 hand-off tensors with srows = 0, and 170 x 256
threads; then calls ``launch`` with them in that order. The same call here runs the batch-1 loop
directly on the fp16 caches with its attention in fp16 (as src/pi05/mk6.cu:35, 95-101 computes it),
must match the oracle's fp8 loop on the same codes, scales and the caller's fp16 cache values as
they are (the oracle reads the fp16 bits; nothing is rounded for it), write the suffix rows back into
the fp16 caches, and leave rows [Tv, T) of x_t alone. The same values in bf16 caches (each rounded to
8 significant bits) run the bf16 attention; both errors are printed side by side. Each launch starts
from a freshly initialised workspace, so the comparison does not depend on the workspace's history.
"""
import numpy as np
import pytest
import torch

from flashact_amd import pi05
from tests import pi05_case as P

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
D, QD, F, H, HD, AD = 1024, 2048, 4096, 8, 256, 32

pytestmark = pytest.mark.gpu


def _fp16_caches(NL, Lp, Lmax, seed, batch=1):
    g = torch.Generator().manual_seed(seed)
    kh = torch.randn(batch, NL, Lp, HD, generator=g).half()  # fp16-precision values
    vh = torch.randn(batch, NL, Lp, HD, generator=g).half()
    return kh, vh


def _caches(kh, vh, Lmax, dtype, dev):
    b, nl, lp, _ = kh.shape
    kc = torch.zeros(b, nl, Lmax, HD, dtype=dtype, device=dev)
    vc = torch.zeros(b, nl, HD, Lmax, dtype=dtype, device=dev)
    kc[:, :, :lp] = kh.to(dev, dtype)
    vc[:, :, :, :lp] = vh.transpose(-1, -2).to(dev, dtype)
    return kc, vc


def test_reference_call_fp8_fp16_caches(gpu):
    NL, Lp, T, TV, S = 18, 968, 16, 10, 10  # the reference's LIBERO setup: horizon 10, T = 16
    c = P.make_case(NL=NL, Lp=Lp, Tv=TV, S=S, seed=21)
    Lmax = (Lp + T + 15) // 16 * 16
    kh, vh = _fp16_caches(NL, Lp, Lmax, seed=22)
    c["inp"]["kpre"], c["inp"]["vpre"] = kh.bfloat16(), vh.bfloat16()  # the GPU side reads kh / vh below
    w = c["w"]
    nat = {k: w[k] for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")}
    pk = pi05.pack_weights_fp8(*(nat[k].to(gpu) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")))
    cos, sin = pi05.rope_table(Lp, device=gpu)  # 16 rows, as pack_weights.rope_table(Lp)
    dev = gpu
    kcache, vtcache = _caches(kh, vh, Lmax, torch.float16, dev)
    kcache, vtcache = kcache[0].contiguous(), vtcache[0].contiguous()
    x_t = torch.zeros(T, AD, dtype=torch.float32, device=dev)
    x_t[:TV] = c["inp"]["noise"][0].to(dev)
    x = torch.zeros(2 * T, D, dtype=torch.float32, device=dev)
    xp = torch.zeros(4, T, D, dtype=torch.float32, device=dev)
    xn = torch.zeros(T, D, dtype=torch.float16, device=dev)
    qb = torch.zeros(T, QD, dtype=torch.float16, device=dev)
    attnb = torch.zeros(T, QD, dtype=torch.float16, device=dev)
    hmlp = torch.zeros(T, F, dtype=torch.float16, device=dev)
    scores = torch.zeros(H, T, Lmax, dtype=torch.float32, device=dev)
    probs = torch.zeros(H, T, Lmax, dtype=torch.float16, device=dev)
    sc_cyc = torch.zeros(16, dtype=torch.int64, device=dev)
    mods, modf = c["mods"].to(dev), c["mod_final"].to(dev)
    wv = {k: w[k].to(dev) for k in ("w_ain", "b_ain", "w_aout", "b_aout")}
    empty = torch.empty(0, dtype=torch.bfloat16, device=dev)
    pi05.reset_workspace(pi05.workspace(dev))
    pi05.launch(pk["w1"], pk["wo"], pk["w2"], pk["w3"], pk["s1"], pk["so"], pk["s2"], pk["s3"],
                mods, modf, cos, sin, wv["w_ain"], wv["b_ain"], wv["w_aout"], wv["b_aout"],
                empty, empty, 0, kcache, vtcache, Lp, Lmax, S, TV, x_t, x, xp, sc_cyc,
                xn, qb, attnb, hmlp, scores, probs, 170, 256)
    torch.cuda.synchronize()
    assert pi05.read_status(pi05.workspace(dev)) == 0
    out = x_t.cpu().numpy()

    from oracle import oracle as O
    ow = P.oracle_weights(c)
    for n, k in (("q", "wq"), ("k", "wk"), ("v", "wv"), ("o", "wo"), ("g", "wg"), ("u", "wu"), ("d", "wd")):
        q, s = pi05.quantize_fp8(nat[k])
        ow["q" + n], ow["s" + n] = q.numpy(), s.numpy()
    ow["kpre"] = kh.numpy().view(np.uint16)  # the caller's fp16 values, unrounded
    ow["vpre"] = vh.numpy().view(np.uint16)
    ref = O.pi05_denoise_fp8(ow, c["inp"]["noise"].numpy(), Lp=Lp, Tv=TV, S=S, NL=NL, kv_dtype="f16")[0]
    st = P.parity(out[:TV], ref)
    print(f"reference call (fp8 codes, fp16 caches, T=16, Tv=10, 18 layers x 10 steps), fp16 attention, vs the "
          f"oracle on the fp16 cache values: {st}", flush=True)
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st
    assert np.all(out[TV:] == 0.0), "rows [Tv, T) of x_t must be left untouched"
    assert int(sc_cyc.sum()) > 0

    # the same cache values in bf16 caches (rounded to 8 significant bits): the bf16 attention
    kb, vb = _caches(kh, vh, Lmax, torch.bfloat16, dev)
    kb, vb = kb[0].contiguous(), vb[0].contiguous()
    x2 = torch.zeros(T, AD, dtype=torch.float32, device=dev)
    x2[:TV] = c["inp"]["noise"][0].to(dev)
    pi05.reset_workspace(pi05.workspace(dev))
    pi05.launch(pk["w1"], pk["wo"], pk["w2"], pk["w3"], pk["s1"], pk["so"], pk["s2"], pk["s3"],
                mods, modf, cos, sin, wv["w_ain"], wv["b_ain"], wv["w_aout"], wv["b_aout"],
                empty, empty, 0, kb, vb, Lp, Lmax, S, TV, x2)
    torch.cuda.synchronize()
    st2 = P.parity(x2[:TV].cpu().numpy(), ref)
    print(f"the same call on bf16 caches of the same values (bf16 attention): {st2}", flush=True)
    assert st2["max_abs"] <= MAX_ABS and st2["mean_abs"] <= MEAN_ABS, st2
    # the prefix rows of the fp16 caches are untouched; the suffix rows hold this call's keys and
    # values in fp16, within bf16 rounding of the bf16 launch's rows (the two loops' states differ by
    # their attention precision only)
    assert torch.equal(kcache[:, :Lp].cpu(), kh[0]) and torch.equal(vtcache[:, :, :Lp].cpu(), vh[0].transpose(1, 2))
    for a16, b16 in ((kcache[:, Lp:Lp + TV].float(), kb[:, Lp:Lp + TV].float()),
                     (vtcache[:, :, Lp:Lp + TV].float(), vb[:, :, Lp:Lp + TV].float())):
        assert torch.count_nonzero(a16) == a16.numel()
        assert float((a16 - b16).abs().max()) <= 0.02 * float(b16.abs().max()) + 1e-3
    assert torch.count_nonzero(kcache[:, Lp + TV:]) == 0


def test_fp16_caches_batched(gpu):
    """Batch 3 on fp16 caches equals batch 3 on the same values in bf16, bit for bit, and the suffix
    rows come back in fp16."""
    NL, Lp, TV, S, B = 2, 300, 50, 2, 3
    c = P.make_case(NL=NL, Lp=Lp, Tv=TV, S=S, seed=5, batch=B)
    g = P.gpu_tensors(c, gpu)
    p = g["packed"]
    Lmax = g["Lmax"]
    kh, vh = _fp16_caches(NL, Lp, Lmax, seed=6, batch=B)
    outs = {}
    for dt in (torch.float16, torch.bfloat16):
        kc, vc = _caches(kh, vh, Lmax, dt, gpu)
        x_t = c["inp"]["noise"].to(gpu).clone()
        empty = torch.empty(0, device=gpu)
        pi05.launch(p["w1"], p["wo"], p["w2"], p["w3"], empty, empty, empty, empty, g["mods"], g["mod_final"],
                    g["cos"], g["sin"], g["w_ain"], g["b_ain"], g["w_aout"], g["b_aout"], None, None, 0,
                    kc, vc, Lp, Lmax, S, TV, x_t, check_status=True)
        outs[dt] = (x_t, kc, vc)
    a, b = outs[torch.float16], outs[torch.bfloat16]
    assert torch.equal(a[0], b[0])
    assert torch.equal(a[1][:, :, Lp:Lp + TV], b[1][:, :, Lp:Lp + TV].half())
    assert torch.equal(a[2][..., Lp:Lp + TV], b[2][..., Lp:Lp + TV].half())


@pytest.mark.parametrize("NL,Lp,Tv,S", [(2, 968, 50, 2), (2, 0, 17, 2), (1, 2003, 33, 2), (2, 37, 1, 3), (18, 968, 50, 10)])
def test_fp16_caches_batch1_bf16_weights(gpu, NL, Lp, Tv, S):
    """Batch 1 on fp16 caches with bf16 weights: the fp16 attention against the oracle reading the
    same fp16 cache values (Lp = 2003: the keys past each rank's first 32 come from the caches; Lp = 0:
    this step's keys only)."""
    c = P.make_case(NL=NL, Lp=Lp, Tv=Tv, S=S, seed=40 + Lp + Tv)
    g = P.gpu_tensors(c, gpu)
    Lmax = g["Lmax"]
    kh, vh = _fp16_caches(NL, Lp, Lmax, seed=41 + Lp)
    kc, vc = _caches(kh, vh, Lmax, torch.float16, gpu)
    kc, vc = kc[0].contiguous(), vc[0].contiguous()
    p = g["packed"]
    x_t = c["inp"]["noise"][0].to(gpu).clone()
    empty = torch.empty(0, device=gpu)
    pi05.reset_workspace(pi05.workspace(gpu))
    pi05.launch(p["w1"], p["wo"], p["w2"], p["w3"], empty, empty, empty, empty, g["mods"], g["mod_final"],
                g["cos"], g["sin"], g["w_ain"], g["b_ain"], g["w_aout"], g["b_aout"], None, None, 0,
                kc, vc, Lp, Lmax, S, Tv, x_t, check_status=True)
    from oracle import oracle as O
    ow = P.oracle_weights(c)
    ow["kpre"], ow["vpre"] = kh.numpy().view(np.uint16), vh.numpy().view(np.uint16)
    ref = O.pi05_denoise(ow, c["inp"]["noise"].numpy(), Lp=Lp, Tv=Tv, S=S, NL=NL, kv_dtype="f16")[0]
    st = P.parity(x_t.cpu().numpy(), ref)
    print(f"fp16 caches, bf16 weights NL={NL} Lp={Lp} Tv={Tv} S={S}: {st}", flush=True)
    assert st["max_abs"] <= MAX_ABS and st["mean_abs"] <= MEAN_ABS, st
    assert torch.equal(kc[:, :Lp].cpu(), kh[0][:, :Lp])
    assert torch.count_nonzero(kc[:, Lp:Lp + Tv]) == kc[:, Lp:Lp + Tv].numel()
