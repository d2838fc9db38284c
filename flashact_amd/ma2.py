"""MolmoAct2 action expert on MI355X: host-side packing and the ``launch`` entry point.

``launch`` keeps the positional signature of the reference's ``mk_ma2.launch``
(src/molmoact2/binding.cpp:28-35) so the harness call site stays drop-in
(benchmarks/molmoact2/eval_numerics.py:141-144). It forwards device pointers to the C ABI
``fa_ma2_flow`` (include/flashact_mi355x.h), which enqueues ONE cooperative HIP launch for the
whole flow loop on the current torch stream.

Packing helpers mirror the reference's host code (benchmarks/molmoact2/eval_numerics.py:77-133):
  pack_weights ........ per-layer stacks; gate/up rows and biases interleaved (2f = gate, 2f+1 = up)
  make_context ........ compact context K rows [NL][Lkmax][768] and V transposed [NL][768][Lkmax]
  rope_table .......... cos/sin [Tv][48] of the split-half RoPE at positions 0..Tv-1
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

D, NH, HD, FF, AD = 768, 8, 96, 3072, 32
MAX_TV = 64


def pack_weights(w_qkv, w_so, w_cq, w_co, w_g, w_u, w_dn, b_qkv, b_so, b_cq, b_co, b_g, b_u, b_dn):
    """Natural [NL][out][in] weights + [NL][out] biases -> (ws, bs), the reference's two lists."""
    bf = torch.bfloat16
    nl = w_g.shape[0]
    w_gu = torch.stack([w_g, w_u], dim=2).reshape(nl, 2 * w_g.shape[1], w_g.shape[2]).to(bf).contiguous()
    b_gu = torch.stack([b_g, b_u], dim=2).reshape(nl, 2 * b_g.shape[1]).float().contiguous()
    ws = [w_qkv.to(bf).contiguous(), w_so.to(bf).contiguous(), w_cq.to(bf).contiguous(), w_co.to(bf).contiguous(),
          w_gu, w_dn.to(bf).contiguous()]
    bs = [b_qkv.float().contiguous(), b_so.float().contiguous(), b_cq.float().contiguous(),
          b_co.float().contiguous(), b_gu, b_dn.float().contiguous()]
    return ws, bs


def lkmax_for(Lk: int) -> int:
    return (Lk + 15) // 16 * 16


def make_context(kctx, vctx, Lkmax: int | None = None):
    """[.., NL, Lk, 768] context K and V -> kctx [.., NL, Lkmax, 768] and vtctx [.., NL, 768, Lkmax]
    (bf16, zero padded), for one sample or a leading batch dimension."""
    Lk = kctx.shape[-2]
    Lkmax = Lkmax or lkmax_for(Lk)
    kc = torch.zeros(*kctx.shape[:-2], Lkmax, kctx.shape[-1], dtype=torch.bfloat16, device=kctx.device)
    vt = torch.zeros(*vctx.shape[:-2], vctx.shape[-1], Lkmax, dtype=torch.bfloat16, device=vctx.device)
    kc[..., :Lk, :] = kctx
    vt[..., :Lk] = vctx.transpose(-1, -2)
    return kc.contiguous(), vt.contiguous()


def rope_table(Tv: int, head_dim: int = HD, base: float = 10000.0, device=None):
    """cos/sin [Tv][head_dim/2] for positions 0..Tv-1 (fp32). The reference builds the table from the
    model's own rotary module (eval_numerics.py:108-111); its base is a model parameter."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
    pos = torch.arange(0, Tv, dtype=torch.float32, device=device)
    freqs = torch.outer(pos, inv_freq)
    return freqs.cos().contiguous(), freqs.sin().contiguous()


# ---------------------------------------------------------------- workspace
_WS: dict = {}


def workspace(device, batch: int = 1, Tv: int = 30, Lkmax: int = 496) -> torch.Tensor:
    """Per-device cached workspace (zeroed once). One launch at a time may use it."""
    dev = torch.device(device)
    L = _lib.lib()
    nbytes = int(L.fa_ma2_workspace_bytes(batch, Tv, Lkmax))
    if nbytes == 0:
        raise _lib.FlashActError(f"no workspace size for batch={batch} Tv={Tv} Lkmax={Lkmax}")
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), batch)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=dev)
        off = (-ws.data_ptr()) % 256
        ws = ws[off:off + nbytes]
        _lib.check(L.fa_ma2_workspace_init(ctypes.c_void_p(ws.data_ptr()), nbytes,
                                           ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)),
                   "fa_ma2_workspace_init")
        _WS[key] = ws
    return ws


def read_status(ws: torch.Tensor) -> int:
    st = ctypes.c_uint(0)
    _lib.check(_lib.lib().fa_ma2_read_status(ctypes.c_void_p(ws.data_ptr()), ctypes.byref(st)), "fa_ma2_read_status")
    return int(st.value)


def _ptr(t):
    if t is None or (isinstance(t, torch.Tensor) and t.numel() == 0):
        return None
    if not t.is_cuda:
        raise ValueError("all tensors must be on the GPU")
    if not t.is_contiguous():
        raise ValueError("all tensors must be contiguous")
    return t.data_ptr()


def launch(ws, bs, mods, mod_final, rope_cos, rope_sin, w_ain, b_ain, w_aout, b_aout, kctx, vtctx,
           Lk, Lkmax, Tv, adim, num_steps, x_t, x=None, xp=None, stage_cycles=None, bufs=None, scores=None,
           probs=None, nblocks=None, nthreads=None, *, workspace_tensor=None):
    """Runs the whole ``num_steps`` flow loop; ``x_t`` is updated in place (the output).

    Same positional order as the reference ``launch``. ``ws`` = [w_qkv, w_so, w_cq, w_co, w_gu, w_dn]
    (bf16), ``bs`` = their fp32 biases. A leading batch dimension on ``x_t`` [B][T][32] (with
    ``kctx`` [B][NL][Lkmax][768] and ``vtctx`` [B][NL][768][Lkmax]) runs B samples in one launch.
    The scratch tensors x, xp, bufs, scores, probs and nblocks/nthreads are accepted and ignored: the
    engine keeps its intermediates in one workspace (``workspace()``). Rows [Tv, T) of x_t and dims
    >= adim are left untouched.
    """
    L = _lib.lib()
    if len(ws) != 6 or len(bs) != 6:
        raise ValueError("ws and bs must hold the 6 projections (qkv, self-out, cross-q, cross-out, gate/up, down)")
    for i, t in enumerate(ws):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"ws[{i}] must be bfloat16, got {t.dtype}")
    for i, t in enumerate(bs):
        if t.dtype != torch.float32:
            raise TypeError(f"bs[{i}] must be float32, got {t.dtype}")
    if kctx.dtype != torch.bfloat16 or vtctx.dtype != torch.bfloat16 or w_aout.dtype != torch.bfloat16:
        raise TypeError("kctx, vtctx and w_aout must be bfloat16")
    for name, t in (("mods", mods), ("mod_final", mod_final), ("rope_cos", rope_cos), ("rope_sin", rope_sin),
                    ("w_ain", w_ain), ("b_ain", b_ain), ("b_aout", b_aout), ("x_t", x_t)):
        if t.dtype != torch.float32:
            raise TypeError(f"{name} must be float32, got {t.dtype}")
    batch = int(x_t.shape[0]) if x_t.dim() == 3 else 1
    dev = x_t.device
    wsp = workspace_tensor if workspace_tensor is not None else workspace(dev, batch, int(Tv), int(Lkmax))
    a = _lib.Ma2Args()
    a.weight_dtype = _lib.FA_DTYPE_BF16
    a.w_qkv, a.w_so, a.w_cq, a.w_co, a.w_gu, a.w_dn = (_ptr(t) for t in ws)
    a.b_qkv, a.b_so, a.b_cq, a.b_co, a.b_gu, a.b_dn = (_ptr(t) for t in bs)
    a.mods, a.mod_final = _ptr(mods), _ptr(mod_final)
    a.rope_cos, a.rope_sin = _ptr(rope_cos), _ptr(rope_sin)
    a.w_ain, a.b_ain, a.w_aout, a.b_aout = _ptr(w_ain), _ptr(b_ain), _ptr(w_aout), _ptr(b_aout)
    a.kctx, a.vtctx = _ptr(kctx), _ptr(vtctx)
    a.Lk, a.Lkmax, a.Tv, a.adim, a.num_steps = int(Lk), int(Lkmax), int(Tv), int(adim), int(num_steps)
    a.num_layers, a.batch = int(ws[0].shape[0]), batch
    a.x_t, a.xt_rows = _ptr(x_t), int(x_t.shape[-2])
    if stage_cycles is not None and stage_cycles.numel() > 0:
        if stage_cycles.dtype != torch.int64 or stage_cycles.numel() < 16:
            raise TypeError("stage_cycles must be an int64 tensor with >= 16 entries")
        a.stage_cycles = _ptr(stage_cycles)
    a.workspace, a.workspace_bytes = wsp.data_ptr(), wsp.numel()
    stream = torch.cuda.current_stream(dev).cuda_stream
    _lib.check(L.fa_ma2_flow(ctypes.byref(a), ctypes.c_void_p(stream)), "fa_ma2_flow")
