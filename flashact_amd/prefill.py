"""pi0.5 prefix prefill on MI355X: the Gemma-2B-shaped backbone writes the K/V cache of the denoise loop.

``prefill`` replaces the reference's prefill and the cache hand-off after it: openpi's PaliGemma
forward with use_cache (benchmarks/pi05/eval_numerics.py:50-57), then compact_kv and the cache fill
(src/pi05/pack_weights.py:60-70; benchmarks/pi05/eval_numerics.py:83-87). It enqueues ONE
cooperative launch (C ABI ``fa_pi05_prefill``) that writes the RoPE'd keys into kcache rows
[0, Lp) and the transposed values into vtcache columns [0, Lp) of every layer, so the caches go
straight to ``pi05.launch`` with no copy in between.

Backbone shape: D = 2048, 8 query heads / 1 K/V head of 256, F = 16384 (GeLU-tanh gate), RMSNorm
eps 1e-6 scaled by (1 + w), RoPE base 10000 at positions 0..Lp-1, no mask inside the prefix.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib, pi05

D, F, HD = 2048, 16384, 256


def pack_backbone(wq, wk, wv, wo, wg, wu, wd) -> dict:
    """Natural [NL][out][in] backbone weights -> packed bf16 buffers (the expert's packing: q/k
    RoPE pairs adjacent, gate/up rows interleaved): {"wqkv", "wo", "wgu", "wdn"}."""
    p = pi05.pack_weights(wq, wk, wv, wo, wg, wu, wd)
    return {"wqkv": p["w1"], "wo": p["wo"], "wgu": p["w2"], "wdn": p["w3"]}


def rope_table(Lp: int, device=None):
    """cos/sin [Lp][128] for positions 0..Lp-1."""
    return pi05.rope_table(0, Lp, device=device)


_WS: dict = {}


def workspace(device, batch: int, Lp: int, Lmax: int) -> torch.Tensor:
    """Per-device cached workspace (zeroed once). One launch at a time may use it."""
    dev = torch.device(device)
    L = _lib.lib()
    nbytes = int(L.fa_pi05_prefill_workspace_bytes(batch, Lp, Lmax))
    if nbytes == 0:
        raise _lib.FlashActError(f"no prefill workspace for batch={batch} Lp={Lp} Lmax={Lmax}")
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        _WS.pop(key, None)
        raw = torch.empty(nbytes + 256, dtype=torch.uint8, device=dev)
        off = (-raw.data_ptr()) % 256
        ws = raw[off:off + nbytes]
        _lib.check(L.fa_pi05_workspace_init(ctypes.c_void_p(ws.data_ptr()), nbytes,
                                            ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)),
                   "fa_pi05_workspace_init")
        _WS[key] = ws
    return ws


def read_status(ws: torch.Tensor) -> int:
    return pi05.read_status(ws)


def release_buffers() -> None:
    """Drops the cached workspaces (they are re-created on the next launch)."""
    _WS.clear()


def _ptr(t, name):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


def prefill(packed: dict, ln_in, ln_post, x, kcache, vtcache, rope_cos=None, rope_sin=None, *, stage_cycles=None,
            workspace_tensor=None, check_status=False):
    """Runs every backbone layer over the prefix and fills the caches in place.

    check_status=True waits for the launch and reads the kernel status; a non-zero status (a capped
    barrier wait expired, or the XCD placement differed, which leaves the caches unfinished)
    re-initialises the workspace and raises FlashActError.

    packed: ``pack_backbone`` output. ln_in, ln_post [NL][2048] fp32. x [B][Lp][2048] (or [Lp][2048])
    fp32: the hidden states entering layer 0. kcache [B][NL][Lmax][256] / vtcache [B][NL][256][Lmax]
    bf16 (or without the batch dimension). rope_cos/sin [Lp][128] (default: positions 0..Lp-1).
    """
    L = _lib.lib()
    for k in ("wqkv", "wo", "wgu", "wdn"):
        if packed[k].dtype != torch.bfloat16:
            raise TypeError(f"packed[{k!r}] must be bfloat16")
    if x.dtype != torch.float32 or ln_in.dtype != torch.float32 or ln_post.dtype != torch.float32:
        raise TypeError("x, ln_in and ln_post must be float32")
    if kcache.dtype != torch.bfloat16 or vtcache.dtype != torch.bfloat16:
        raise TypeError("kcache and vtcache must be bfloat16")
    batch = int(x.shape[0]) if x.dim() == 3 else 1
    Lp = int(x.shape[-2])
    NL = int(packed["wqkv"].shape[0])
    Lmax = int(kcache.shape[-2])
    if x.shape[-1] != D or kcache.shape[-1] != HD or vtcache.shape[-1] != Lmax:
        raise ValueError(f"shapes: x {tuple(x.shape)}, kcache {tuple(kcache.shape)}, vtcache {tuple(vtcache.shape)}")
    if kcache.numel() != batch * NL * Lmax * HD or vtcache.numel() != kcache.numel():
        raise ValueError("kcache / vtcache must hold [batch][NL][Lmax][256] / [batch][NL][256][Lmax]")
    dev = x.device
    if rope_cos is None or rope_sin is None:
        rope_cos, rope_sin = rope_table(Lp, device=dev)
    if rope_cos.shape != (Lp, HD // 2) or rope_sin.shape != (Lp, HD // 2):
        raise ValueError(f"rope tables must be [{Lp}][128]")
    wsp = workspace_tensor if workspace_tensor is not None else workspace(dev, batch, Lp, Lmax)
    a = _lib.PrefillArgs()
    a.weight_dtype = _lib.FA_DTYPE_BF16
    a.wqkv, a.wo, a.wgu, a.wdn = (_ptr(packed[k], k) for k in ("wqkv", "wo", "wgu", "wdn"))
    a.ln_in, a.ln_post = _ptr(ln_in, "ln_in"), _ptr(ln_post, "ln_post")
    a.rope_cos, a.rope_sin = _ptr(rope_cos, "rope_cos"), _ptr(rope_sin, "rope_sin")
    a.x = _ptr(x, "x")
    a.kcache, a.vtcache = _ptr(kcache, "kcache"), _ptr(vtcache, "vtcache")
    a.Lp, a.Lmax, a.num_layers, a.batch = Lp, Lmax, NL, batch
    if stage_cycles is not None and stage_cycles.numel() > 0:
        if stage_cycles.dtype != torch.int64 or stage_cycles.numel() < 16:
            raise TypeError("stage_cycles must be an int64 tensor with >= 16 entries")
        a.stage_cycles = _ptr(stage_cycles, "stage_cycles")
    a.workspace, a.workspace_bytes = wsp.data_ptr(), wsp.numel()
    stream = torch.cuda.current_stream(dev).cuda_stream
    _lib.check(L.fa_pi05_prefill(ctypes.byref(a), ctypes.c_void_p(stream)), "fa_pi05_prefill")
    if check_status:
        pi05.raise_on_status(wsp, torch.cuda.current_stream(dev), what="fa_pi05_prefill")
