"""ctypes binding of libflashact_mi355x.so (the C ABI declared in include/flashact_mi355x.h).

The library is built in-tree by ``flashact_amd.build`` (``__graft_entry__.build()``). There is
no fallback: if the shared library is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

from .build import LIB_PATH

ABI_VERSION = 2
STAGE_TICK_HZ = 100_000_000  # FA_STAGE_TICK_HZ: unit of the stage_cycles counters

FA_OK = 0
FA_DTYPE_BF16 = 0
FA_DTYPE_FP8_E4M3 = 1
FA_DTYPE_F16 = 2
FA_KSTATUS_SPIN_TIMEOUT = 1
FA_KSTATUS_XCD_MAP = 2
FA_KSTATUS_RANGE = 4


class FlashActError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


class Pi05Args(ctypes.Structure):
    _fields_ = [
        ("weight_dtype", ctypes.c_int),
        ("w1", ctypes.c_void_p), ("wo", ctypes.c_void_p), ("w2", ctypes.c_void_p), ("w3", ctypes.c_void_p),
        ("s1", ctypes.c_void_p), ("so", ctypes.c_void_p), ("s2", ctypes.c_void_p), ("s3", ctypes.c_void_p),
        ("mods", ctypes.c_void_p), ("mod_final", ctypes.c_void_p),
        ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p),
        ("w_ain", ctypes.c_void_p), ("b_ain", ctypes.c_void_p), ("w_aout", ctypes.c_void_p), ("b_aout", ctypes.c_void_p),
        ("kvsrc_k", ctypes.c_void_p), ("kvsrc_v", ctypes.c_void_p), ("srows", ctypes.c_int),
        ("kcache", ctypes.c_void_p), ("vtcache", ctypes.c_void_p),
        ("Lp", ctypes.c_int), ("Lmax", ctypes.c_int), ("num_steps", ctypes.c_int), ("Tv", ctypes.c_int),
        ("num_layers", ctypes.c_int), ("batch", ctypes.c_int),
        ("x_t", ctypes.c_void_p), ("xt_rows", ctypes.c_int),
        ("stage_cycles", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("trace", ctypes.c_void_p), ("trace_layer", ctypes.c_int),
        ("cache_dtype", ctypes.c_int), ("cache_shadow", ctypes.c_void_p), ("cache_shadow_bytes", ctypes.c_size_t),
    ]


class Ma2Args(ctypes.Structure):
    _fields_ = [
        ("weight_dtype", ctypes.c_int),
        ("w_qkv", ctypes.c_void_p), ("w_so", ctypes.c_void_p), ("w_cq", ctypes.c_void_p), ("w_co", ctypes.c_void_p),
        ("w_gu", ctypes.c_void_p), ("w_dn", ctypes.c_void_p),
        ("b_qkv", ctypes.c_void_p), ("b_so", ctypes.c_void_p), ("b_cq", ctypes.c_void_p), ("b_co", ctypes.c_void_p),
        ("b_gu", ctypes.c_void_p), ("b_dn", ctypes.c_void_p),
        ("mods", ctypes.c_void_p), ("mod_final", ctypes.c_void_p),
        ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p),
        ("w_ain", ctypes.c_void_p), ("b_ain", ctypes.c_void_p), ("w_aout", ctypes.c_void_p), ("b_aout", ctypes.c_void_p),
        ("kctx", ctypes.c_void_p), ("vtctx", ctypes.c_void_p),
        ("Lk", ctypes.c_int), ("Lkmax", ctypes.c_int), ("Tv", ctypes.c_int), ("adim", ctypes.c_int),
        ("num_steps", ctypes.c_int), ("num_layers", ctypes.c_int), ("batch", ctypes.c_int),
        ("x_t", ctypes.c_void_p), ("xt_rows", ctypes.c_int),
        ("stage_cycles", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
    ]


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("weight_dtype", ctypes.c_int),
        ("wqkv", ctypes.c_void_p), ("wo", ctypes.c_void_p), ("wgu", ctypes.c_void_p), ("wdn", ctypes.c_void_p),
        ("ln_in", ctypes.c_void_p), ("ln_post", ctypes.c_void_p),
        ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p),
        ("x", ctypes.c_void_p), ("kcache", ctypes.c_void_p), ("vtcache", ctypes.c_void_p),
        ("Lp", ctypes.c_int), ("Lmax", ctypes.c_int), ("num_layers", ctypes.c_int), ("batch", ctypes.c_int),
        ("stage_cycles", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
    ]


class DeviceInfo(ctypes.Structure):
    _fields_ = [("cus", ctypes.c_int), ("xcds", ctypes.c_int), ("lds_bytes", ctypes.c_int),
                ("coop_launch", ctypes.c_int), ("coop_max_blocks", ctypes.c_int), ("arch", ctypes.c_char * 64)]


# (name, restype, argtypes) of every symbol declared in include/flashact_mi355x.h
SYMBOLS = [
    ("fa_pi05_denoise", ctypes.c_int, [ctypes.POINTER(Pi05Args), ctypes.c_void_p]),
    ("fa_pi05_denoise_noalloc", ctypes.c_int,
     [ctypes.POINTER(Pi05Args), ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
    ("fa_pi05_workspace_bytes", ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    ("fa_pi05_cache_shadow_bytes", ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    ("fa_pi05_workspace_init", ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    ("fa_pi05_read_status", ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint)]),
    ("fa_pi05_max_batch", ctypes.c_int, []),
    ("fa_ma2_flow", ctypes.c_int, [ctypes.POINTER(Ma2Args), ctypes.c_void_p]),
    ("fa_ma2_workspace_bytes", ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    ("fa_ma2_workspace_init", ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    ("fa_ma2_read_status", ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint)]),
    ("fa_ma2_max_batch", ctypes.c_int, []),
    ("fa_pi05_prefill", ctypes.c_int, [ctypes.POINTER(PrefillArgs), ctypes.c_void_p]),
    ("fa_pi05_prefill_workspace_bytes", ctypes.c_size_t, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    ("fa_device_query", ctypes.c_int, [ctypes.c_int, ctypes.POINTER(DeviceInfo)]),
    ("fa_last_error", ctypes.c_char_p, []),
    ("fa_abi_version", ctypes.c_int, []),
]

_lib = None


def lib() -> ctypes.CDLL:
    """Loads the in-tree shared library once; raises if it is absent (no fallback path)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FlashActError(f"{LIB_PATH} is missing: build it with `python -m flashact_amd.build` "
                                "(or __graft_entry__.build())")
        so = ctypes.CDLL(LIB_PATH)
        for name, res, args in SYMBOLS:
            fn = getattr(so, name)
            fn.restype = res
            fn.argtypes = args
        if so.fa_abi_version() != ABI_VERSION:
            raise FlashActError(f"ABI mismatch: library {so.fa_abi_version()} vs binding {ABI_VERSION}")
        _lib = so
    return _lib


def check(rc: int, what: str) -> None:
    if rc != FA_OK:
        msg = lib().fa_last_error()
        raise FlashActError(f"{what} failed (status {rc}): {msg.decode() if msg else ''}")
