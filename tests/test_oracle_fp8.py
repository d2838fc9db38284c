"""Pins of the oracle's FP8-W8A16 path (fo_pi05_denoise_fp8) and of the FP8 weight quantiser.

* e4m3 decoding: all 256 codes against torch's float8_e4m3fn (OCP E4M3), NaN codes included.
* The W8A16 loop, (sum_k x_k q_nk) s_n per output row, against the bf16 loop run on the weights
  decode(q) s: with power-of-two row scales both are exact scalings of the same sums, so the two
  loops must agree bit for bit (a scale applied twice, to the wrong row, or not at all breaks it).
* quantize_fp8 (the reference's per-row quantisation, src/pi05/hybrid_model.py:105-110): the
  largest element of each row maps to +-448 and the round trip stays within e4m3's step.
* fp16 prefix K/V (the reference's cache dtype, benchmarks/pi05/eval_numerics.py:83-85): the
  oracle's binary16 decoding against numpy's float16 on all 65536 bit patterns, and the loop on fp16
  bits equal, bit for bit, to the loop on bf16 bits when every value is exact in both formats.
"""
import numpy as np
import torch

from flashact_amd import pi05
from oracle import oracle as O

DIMS = dict(NL=2, D=64, H=2, HD=16, F=48, AD=32)


def test_e4m3_decode_all_codes():
    c = np.arange(256, dtype=np.uint8)
    got = O.e4m3_decode(c)
    want = torch.from_numpy(c).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    assert np.array_equal(np.signbit(got[ok]), np.signbit(want[ok]))  # -0 is 0x80


def test_f16_decode_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_decode(bits)
    want = bits.view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    assert np.array_equal(np.signbit(got[ok]), np.signbit(want[ok]))


def _case(rng, Lp=5, Tv=3, S=2):
    NL, D, H, HD, F, AD = (DIMS[k] for k in ("NL", "D", "H", "HD", "F", "AD"))
    shapes = {"q": (NL, H * HD, D), "k": (NL, HD, D), "v": (NL, HD, D), "o": (NL, D, H * HD),
              "g": (NL, F, D), "u": (NL, F, D), "d": (NL, D, F)}
    w = {}
    for n, shp in shapes.items():
        codes = rng.integers(0, 256, size=shp, dtype=np.uint8)
        codes[(codes & 0x7f) == 0x7f] = 0x3c  # no NaN codes
        w["q" + n] = codes
        w["s" + n] = np.ldexp(1.0, rng.integers(-9, -3, size=shp[:2])).astype(np.float32)  # powers of two
    half = HD // 2
    ang = rng.normal(size=(Tv, half)).astype(np.float32)
    bf = lambda a: torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    w.update(mods=(0.1 * rng.normal(size=(S, NL, 2, 3 * D))).astype(np.float32),
             mod_final=(0.1 * rng.normal(size=(S, 3 * D))).astype(np.float32),
             rope_cos=np.cos(ang), rope_sin=np.sin(ang),
             w_ain=(0.1 * rng.normal(size=(D, AD))).astype(np.float32), b_ain=np.zeros(D, np.float32),
             w_aout=(0.1 * rng.normal(size=(AD, D))).astype(np.float32), b_aout=np.zeros(AD, np.float32),
             kpre=bf(rng.normal(size=(1, NL, Lp, HD))), vpre=bf(rng.normal(size=(1, NL, Lp, HD))))
    x = rng.normal(size=(1, Tv, AD)).astype(np.float32)
    return w, x, Lp, Tv, S


def test_fp8_loop_equals_bf16_loop_on_dequantised_weights():
    rng = np.random.default_rng(0)
    w, x, Lp, Tv, S = _case(rng)
    out8 = O.pi05_denoise_fp8(w, x, Lp=Lp, Tv=Tv, S=S, **DIMS)
    wb = dict(w)
    for n in "qkvogud":
        deq = O.e4m3_decode(w["q" + n]) * w["s" + n][..., None]
        wb["w" + n] = torch.from_numpy(deq).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(torch.from_numpy(deq).to(torch.bfloat16).float().numpy(), deq)  # exact in bf16
    out16 = O.pi05_denoise(wb, x, Lp=Lp, Tv=Tv, S=S, **DIMS)
    assert np.array_equal(out8, out16)
    # a wrong scale changes the result
    w2 = dict(w)
    w2["sg"] = w["sg"] * 2
    assert not np.array_equal(O.pi05_denoise_fp8(w2, x, Lp=Lp, Tv=Tv, S=S, **DIMS), out8)


def test_f16_kv_loop_equals_bf16_kv_loop_on_shared_values():
    rng = np.random.default_rng(3)
    w, x, Lp, Tv, S = _case(rng)
    wb = dict(w)
    for n in "qkvogud":
        deq = O.e4m3_decode(w["q" + n]) * w["s" + n][..., None]
        wb["w" + n] = torch.from_numpy(deq).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    wh = dict(wb)
    for k in ("kpre", "vpre"):
        vals = (w[k].astype(np.uint32) << 16).view(np.float32)
        vals = np.where(np.abs(vals) < 2.0 ** -14, 0.0, vals).astype(np.float32)  # normal in fp16 too
        wb[k] = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        wh[k] = vals.astype(np.float16).view(np.uint16)
        assert np.array_equal(wh[k].view(np.float16).astype(np.float32), vals)  # exact in fp16
    ob = O.pi05_denoise(wb, x, Lp=Lp, Tv=Tv, S=S, **DIMS)
    oh = O.pi05_denoise(wh, x, Lp=Lp, Tv=Tv, S=S, kv_dtype="f16", **DIMS)
    assert np.array_equal(ob, oh)
    # the same bits read as the other format are other values
    assert not np.array_equal(O.pi05_denoise(wb, x, Lp=Lp, Tv=Tv, S=S, kv_dtype="f16", **DIMS), ob)


def test_quantize_fp8_rows():
    g = torch.Generator().manual_seed(1)
    w = torch.randn(3, 40, 96, generator=g) * 0.02
    w[0, 5] = 0.0  # all-zero row
    q, s = pi05.quantize_fp8(w)
    assert q.dtype == torch.uint8 and s.shape == (3, 40)
    deq = torch.from_numpy(O.e4m3_decode(q.numpy())) * s[..., None]
    assert torch.all(deq[0, 5] == 0)
    nz = w.abs().amax(dim=-1) > 0
    amax_codes = torch.from_numpy(O.e4m3_decode(q.numpy())).abs().amax(dim=-1)
    assert torch.all(amax_codes[nz] == 448.0)
    rel = (deq - w).abs() / w.abs().amax(dim=-1, keepdim=True).clamp(min=1e-30)
    assert float(rel.max()) <= 2 ** -4 + 1e-6  # half a step of 3 mantissa bits at the top binade
    packed = pi05.pack_weights_fp8(*(torch.randn(2, *shp, generator=g).to(torch.bfloat16) * 0.02 for shp in
                                     ((2048, 1024), (256, 1024), (256, 1024), (1024, 2048), (4096, 1024),
                                      (4096, 1024), (1024, 4096))))
    assert packed["w1"].shape == (2, 2560, 1024) and packed["s1"].shape == (2, 2560)
    assert packed["w2"].dtype == torch.uint8 and packed["s3"].shape == (2, 1024)
