"""ctypes front-end of the CPU fp32 oracle (fa_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker. The product package (flashact_amd) never imports it.

All arrays are numpy. bf16 tensors are passed as uint16 bit patterns (torch bf16
``.view(torch.int16)`` / ``.view(torch.uint16)`` reinterpreted), fp32 as float32.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfa_oracle.so")

_lib = None


def build(force: bool = False) -> str:
    """Compile fa_oracle.c with the Makefile beside it (gcc, OpenMP)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE] + (["-B"] if force else []), check=True)
    return LIB_PATH


class Pi05Dims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("NL", "D", "H", "HD", "F", "AD", "Lp", "Tv", "S", "batch", "kv_f16")]


class PrefillDims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("NL", "D", "H", "HD", "F", "Lp", "batch")]


class Ma2Dims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("NL", "D", "H", "HD", "F", "AD", "Lk", "Tv", "S", "adim", "batch")]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.fo_num_threads.restype = ctypes.c_int
        _lib.fo_pi05_denoise.restype = ctypes.c_int
        _lib.fo_ma2_flow.restype = ctypes.c_int
        _lib.fo_gemma_prefill.restype = ctypes.c_int
        _lib.fo_pi05_denoise_fp8.restype = ctypes.c_int
    return _lib


def _p(a: np.ndarray, dtype) -> ctypes.c_void_p:
    if a is None:
        return ctypes.c_void_p(0)
    assert a.dtype == dtype, (a.dtype, dtype)
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u16(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.int16:
        a = a.view(np.uint16)
    assert a.dtype == np.uint16, a.dtype
    return a


def _kv_f16(kv_dtype: str) -> int:
    if kv_dtype not in ("bf16", "f16"):
        raise ValueError(f"kv_dtype must be 'bf16' or 'f16', got {kv_dtype!r}")
    return int(kv_dtype == "f16")


def num_threads() -> int:
    return int(lib().fo_num_threads())


def sinusoid_embedding(t, dim: int, min_period: float = 4e-3, max_period: float = 4.0) -> np.ndarray:
    t = _f32(t).reshape(-1)
    out = np.empty((t.size, dim), np.float32)
    lib().fo_sinusoid_embedding(_p(t, np.float32), ctypes.c_int(t.size), ctypes.c_int(dim),
                                ctypes.c_double(min_period), ctypes.c_double(max_period), _p(out, np.float32))
    return out


def rope_table(start: int, T: int, HD: int, base: float = 10000.0):
    c = np.empty((T, HD // 2), np.float32)
    s = np.empty((T, HD // 2), np.float32)
    lib().fo_rope_table(ctypes.c_int(start), ctypes.c_int(T), ctypes.c_int(HD), ctypes.c_double(base),
                        _p(c, np.float32), _p(s, np.float32))
    return c, s


def pi05_mods(S: int, NL: int, D: int, w_ti, b_ti, w_to, b_to, w_in, b_in, w_post, b_post, w_fin, b_fin):
    """mods [S][NL][2][3D], mod_final [S][3D] for t_s = 1 - s/S (all weights fp32)."""
    args = [_f32(a) for a in (w_ti, b_ti, w_to, b_to, w_in, b_in, w_post, b_post, w_fin, b_fin)]
    mods = np.empty((S, NL, 2, 3 * D), np.float32)
    modf = np.empty((S, 3 * D), np.float32)
    lib().fo_pi05_mods(ctypes.c_int(S), ctypes.c_int(NL), ctypes.c_int(D), *[_p(a, np.float32) for a in args],
                       _p(mods, np.float32), _p(modf, np.float32))
    return mods, modf


def pi05_denoise(w: dict, x_t, *, Lp: int, Tv: int, S: int, NL: int, D: int = 1024, H: int = 8, HD: int = 256,
                 F: int = 4096, AD: int = 32, kv_dtype: str = "bf16") -> np.ndarray:
    """Runs the S-step Euler loop; returns the updated x_t [batch][Tv][AD].

    ``w`` keys: wq wk wv wo wg wu wd (uint16 bf16 bits, natural layouts), mods, mod_final,
    rope_cos, rope_sin, w_ain, b_ain, w_aout, b_aout (fp32), kpre, vpre ([B][NL][Lp][HD] bf16 bits,
    or fp16 bits with kv_dtype="f16").
    """
    x = _f32(x_t).copy()
    B = x.shape[0] if x.ndim == 3 else 1
    dims = Pi05Dims(NL, D, H, HD, F, AD, Lp, Tv, S, B, _kv_f16(kv_dtype))
    u = {k: _u16(w[k]) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "kpre", "vpre")}
    f = {k: _f32(w[k]) for k in ("mods", "mod_final", "rope_cos", "rope_sin", "w_ain", "b_ain", "w_aout", "b_aout")}
    rc = lib().fo_pi05_denoise(
        ctypes.byref(dims), *[_p(u[k], np.uint16) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")],
        *[_p(f[k], np.float32) for k in ("mods", "mod_final", "rope_cos", "rope_sin", "w_ain", "b_ain", "w_aout",
                                          "b_aout")],
        _p(u["kpre"], np.uint16), _p(u["vpre"], np.uint16), _p(x, np.float32))
    if rc != 0:
        raise ValueError(f"fo_pi05_denoise rejected the dimensions (rc={rc})")
    return x


def f16_decode(bits) -> np.ndarray:
    """fp32 values of IEEE binary16 bit patterns (uint16)."""
    c = _u16(bits)
    out = np.empty(c.shape, np.float32)
    lib().fo_f16_decode(_p(c, np.uint16), ctypes.c_int(c.size), _p(out, np.float32))
    return out


def e4m3_decode(codes) -> np.ndarray:
    """fp32 values of OCP E4M3 codes (uint8)."""
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(c.shape, np.float32)
    lib().fo_e4m3_decode(_p(c, np.uint8), ctypes.c_int(c.size), _p(out, np.float32))
    return out


def pi05_denoise_fp8(w: dict, x_t, *, Lp: int, Tv: int, S: int, NL: int, D: int = 1024, H: int = 8, HD: int = 256,
                     F: int = 4096, AD: int = 32, kv_dtype: str = "bf16") -> np.ndarray:
    """pi05_denoise with FP8-W8A16 weights: ``w`` holds e4m3 codes qq qk qv qo qg qu qd (uint8,
    natural layouts) and their per-row fp32 scales sq sk sv so sg su sd, plus the fp32 / bf16 (or
    fp16 K/V) inputs of ``pi05_denoise``."""
    x = _f32(x_t).copy()
    B = x.shape[0] if x.ndim == 3 else 1
    dims = Pi05Dims(NL, D, H, HD, F, AD, Lp, Tv, S, B, _kv_f16(kv_dtype))
    q = {k: np.ascontiguousarray(w[k], dtype=np.uint8) for k in ("qq", "qk", "qv", "qo", "qg", "qu", "qd")}
    sc = {k: _f32(w[k]) for k in ("sq", "sk", "sv", "so", "sg", "su", "sd")}
    f = {k: _f32(w[k]) for k in ("mods", "mod_final", "rope_cos", "rope_sin", "w_ain", "b_ain", "w_aout", "b_aout")}
    u = {k: _u16(w[k]) for k in ("kpre", "vpre")}
    args = []
    for a, b in (("qq", "sq"), ("qk", "sk"), ("qv", "sv"), ("qo", "so"), ("qg", "sg"), ("qu", "su"), ("qd", "sd")):
        args += [_p(q[a], np.uint8), _p(sc[b], np.float32)]
    rc = lib().fo_pi05_denoise_fp8(
        ctypes.byref(dims), *args,
        *[_p(f[k], np.float32) for k in ("mods", "mod_final", "rope_cos", "rope_sin", "w_ain", "b_ain", "w_aout",
                                          "b_aout")],
        _p(u["kpre"], np.uint16), _p(u["vpre"], np.uint16), _p(x, np.float32))
    if rc != 0:
        raise ValueError(f"fo_pi05_denoise_fp8 rejected the dimensions (rc={rc})")
    return x


def ma2_flow(w: dict, x_t, *, Lk: int, Tv: int, S: int, NL: int, adim: int, D: int = 768, H: int = 8, HD: int = 96,
             F: int = 3072, AD: int = 32) -> np.ndarray:
    """Runs the MolmoAct2 S-step flow loop; returns the updated x_t [batch][Tv][AD].

    ``w`` keys: w_qkv w_so w_cq w_co w_g w_u w_dn w_aout kctx vctx (uint16 bf16 bits) and
    b_qkv b_so b_cq b_co b_g b_u b_dn mods mod_final rope_cos rope_sin w_ain b_ain b_aout (fp32).
    """
    x = _f32(x_t).copy()
    B = x.shape[0] if x.ndim == 3 else 1
    dims = Ma2Dims(NL, D, H, HD, F, AD, Lk, Tv, S, adim, B)
    keep = {k: _u16(w[k]) for k in ("w_qkv", "w_so", "w_cq", "w_co", "w_g", "w_u", "w_dn", "w_aout", "kctx", "vctx")}
    keepf = {k: _f32(w[k]) for k in ("b_qkv", "b_so", "b_cq", "b_co", "b_g", "b_u", "b_dn", "mods", "mod_final",
                                      "rope_cos", "rope_sin", "w_ain", "b_ain", "b_aout")}
    U = lambda k: _p(keep[k], np.uint16)  # noqa: E731
    Fp = lambda k: _p(keepf[k], np.float32)  # noqa: E731
    rc = lib().fo_ma2_flow(ctypes.byref(dims), U("w_qkv"), Fp("b_qkv"), U("w_so"), Fp("b_so"), U("w_cq"), Fp("b_cq"),
                           U("w_co"), Fp("b_co"), U("w_g"), Fp("b_g"), U("w_u"), Fp("b_u"), U("w_dn"), Fp("b_dn"),
                           Fp("mods"), Fp("mod_final"), Fp("rope_cos"), Fp("rope_sin"), Fp("w_ain"), Fp("b_ain"),
                           U("w_aout"), Fp("b_aout"), U("kctx"), U("vctx"), _p(x, np.float32))
    if rc != 0:
        raise ValueError(f"fo_ma2_flow rejected the dimensions (rc={rc})")
    return x


def gemma_prefill(w: dict, x, *, NL: int, D: int = 2048, H: int = 8, HD: int = 256,
                  F: int = 16384) -> tuple[np.ndarray, np.ndarray]:
    """Prefix prefill through the Gemma backbone; returns (K, V), each [batch][NL][Lp][HD] fp32.

    ``w`` keys: wq wk wv wo wg wu wd (uint16 bf16 bits, natural layouts), ln_in, ln_post, rope_cos,
    rope_sin (fp32). ``x`` [batch][Lp][D] (or [Lp][D]) fp32: hidden states entering layer 0.
    """
    xx = _f32(x)
    if xx.ndim == 2:
        xx = xx[None]
    B, Lp = xx.shape[0], xx.shape[1]
    dims = PrefillDims(NL, D, H, HD, F, Lp, B)
    u = {k: _u16(w[k]) for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")}
    f = {k: _f32(w[k]) for k in ("ln_in", "ln_post", "rope_cos", "rope_sin")}
    K = np.zeros((B, NL, Lp, HD), np.float32)
    V = np.zeros((B, NL, Lp, HD), np.float32)
    rc = lib().fo_gemma_prefill(ctypes.byref(dims), *[_p(u[k], np.uint16) for k in ("wq", "wk", "wv", "wo", "wg", "wu",
                                                                                      "wd")],
                                *[_p(f[k], np.float32) for k in ("ln_in", "ln_post", "rope_cos", "rope_sin")],
                                _p(xx, np.float32), _p(K, np.float32), _p(V, np.float32))
    if rc != 0:
        raise ValueError(f"fo_gemma_prefill rejected the dimensions (rc={rc})")
    return K, V
