"""MolmoAct2 action expert on MI355X: host-side packing and the ``launch`` entry point.

``launch`` keeps the positional signature of the reference's ``mk_ma2.launch``
(src/molmoact2/binding.cpp:28-35) so the harness call site stays drop-in
(benchmarks/molmoact2/eval_numerics.py:147-150). It forwards device pointers to the C ABI
``fa_ma2_flow`` (include/flashact_mi355x.h), which enqueues ONE cooperative HIP launch for the
whole flow loop on the current torch stream.

Packing helpers mirror the reference's host code (benchmarks/molmoact2/eval_numerics.py:77-133):
  pack_weights ........ per-layer stacks; gate/up rows and biases interleaved (2f = gate, 2f+1 = up)
  make_context ........ compact context K rows [NL][Lkmax][768] and V transposed [NL][768][Lkmax]
  compact_context ..... the masked compaction of the encoder's per-layer context K/V
                        (benchmarks/molmoact2/eval_e2e.py:105-125, eval_numerics.py:123-132)
  rope_table .......... cos/sin [Tv][48] of the split-half RoPE at positions 0..Tv-1
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib, pi05

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


def context_mask(cross_mask, length: int, device=None) -> torch.Tensor:
    """The valid context rows of sample 0, as the reference derives them: no mask -> every row;
    a boolean mask -> its True rows (eval_numerics.py:123); an additive float mask (0 = attend,
    a large negative value = masked) -> the rows holding its maximum, read from [0, 0, 0] of a
    [B][1][T][L] mask (eval_e2e.py:107-113)."""
    if cross_mask is None:
        return torch.ones(length, dtype=torch.bool, device=device)
    m = cross_mask
    if m.dtype == torch.bool:
        while m.dim() > 1:
            m = m[0]
        return m.to(device)
    while m.dim() > 1:
        m = m[0]
    m = m.float()
    return (m == m.max()).to(device)


def compact_context(kv_contexts, cross_mask=None, Lkmax: int | None = None):
    """Per-layer encoder context [(k, v)] with k, v [1][L][8][96] (or [1][L][768]) and an optional
    mask -> (kctx [NL][Lkmax][768], vtctx [NL][768][Lkmax] bf16, Lk): the valid rows kept in order,
    zero padded to Lkmax = ceil16(Lk) (eval_e2e.py:114-125)."""
    k0 = kv_contexts[0][0]
    vmask = context_mask(cross_mask, int(k0.shape[1]), device=k0.device)
    if vmask.numel() != k0.shape[1]:
        raise ValueError(f"mask covers {vmask.numel()} context rows, the context has {k0.shape[1]}")
    Lk = int(vmask.sum().item())
    Lkmax = Lkmax or lkmax_for(Lk)
    if Lkmax < Lk or Lkmax % 16:
        raise ValueError(f"Lkmax={Lkmax} must be a multiple of 16 and >= Lk={Lk}")
    nl = len(kv_contexts)
    kctx = torch.zeros(nl, Lkmax, D, dtype=torch.bfloat16, device=k0.device)
    vtctx = torch.zeros(nl, D, Lkmax, dtype=torch.bfloat16, device=k0.device)
    for l, (kc, vc) in enumerate(kv_contexts):
        kctx[l, :Lk] = kc[0][vmask].reshape(Lk, D).to(torch.bfloat16)
        vtctx[l, :, :Lk] = vc[0][vmask].reshape(Lk, D).t().to(torch.bfloat16)
    return kctx, vtctx, Lk


def rope_table(Tv: int, head_dim: int = HD, base: float = 10000.0, device=None):
    """cos/sin [Tv][head_dim/2] for positions 0..Tv-1 (fp32). The reference builds the table from the
    model's own rotary module (eval_numerics.py:112-115); its base is a model parameter."""
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


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def check_shapes(ws, bs, mods, mod_final, rope_cos, rope_sin, w_ain, b_ain, w_aout, b_aout, kctx, vtctx, Lk, Lkmax,
                 Tv, adim, num_steps, x_t, nl, batch):
    """Every size the kernels address, checked on the host (src/molmoact2/binding.cpp:36-58 takes the
    same tensors unchecked)."""
    _need(nl >= 1 and num_steps >= 1, f"need num_layers >= 1 and num_steps >= 1 (got {nl}, {num_steps})")
    _need(1 <= Tv <= MAX_TV, f"Tv={Tv} outside [1, {MAX_TV}]")
    _need(1 <= adim <= AD, f"adim={adim} outside [1, {AD}]")
    _need(0 <= Lk <= Lkmax and Lkmax % 16 == 0 and Lkmax >= 16, f"Lkmax={Lkmax} must be a multiple of 16 and >= Lk={Lk}")
    wper = (3 * D * D, D * D, D * D, D * D, 2 * FF * D, D * FF)
    bper = (3 * D, D, D, D, 2 * FF, D)
    names = ("qkv", "so", "cq", "co", "gu", "dn")
    for n, w, b, pw, pb in zip(names, ws, bs, wper, bper):
        _need(w.numel() == nl * pw, f"w_{n} holds {w.numel()} elements, need [{nl}][{pw}]")
        _need(b.numel() == nl * pb, f"b_{n} holds {b.numel()} elements, need [{nl}][{pb}]")
    _need(mods.numel() >= num_steps * nl * 9 * D, f"mods holds {mods.numel()} values, need [{num_steps}][{nl}][3][3][768]")
    _need(mod_final.numel() >= num_steps * 2 * D, f"mod_final holds {mod_final.numel()} values, need [{num_steps}][2][768]")
    for name, t in (("rope_cos", rope_cos), ("rope_sin", rope_sin)):
        _need(t.dim() == 2 and t.shape[1] == HD // 2 and t.shape[0] >= Tv,
              f"{name} must be [>= Tv={Tv}][48], got {tuple(t.shape)}")
    for name, t, n in (("w_ain", w_ain, D * AD), ("b_ain", b_ain, D), ("w_aout", w_aout, AD * D), ("b_aout", b_aout, AD)):
        _need(t.numel() == n, f"{name} holds {t.numel()} values, need {n}")
    _need(x_t.shape[-1] == AD and x_t.dim() in (2, 3) and x_t.shape[-2] >= Tv,
          f"x_t must be [batch][rows >= Tv][32] or [rows][32], got {tuple(x_t.shape)}")
    per = nl * Lkmax * D
    for name, t in (("kctx", kctx), ("vtctx", vtctx)):
        _need(t.numel() == batch * per, f"{name} holds {t.numel()} elements, need [batch={batch}][NL={nl}][{Lkmax}][{D}]")
    _need(kctx.shape[-1] == D and kctx.shape[-2] == Lkmax, f"kctx must end in [Lkmax={Lkmax}][768], got {tuple(kctx.shape)}")
    _need(vtctx.shape[-1] == Lkmax and vtctx.shape[-2] == D, f"vtctx must end in [768][Lkmax={Lkmax}], got {tuple(vtctx.shape)}")


def release_buffers() -> None:
    """Drops the cached workspaces (they are re-created on the next launch)."""
    _WS.clear()


def launch(ws, bs, mods, mod_final, rope_cos, rope_sin, w_ain, b_ain, w_aout, b_aout, kctx, vtctx,
           Lk, Lkmax, Tv, adim, num_steps, x_t, x=None, xp=None, stage_cycles=None, bufs=None, scores=None,
           probs=None, nblocks=None, nthreads=None, *, workspace_tensor=None, check_status=False):
    """Runs the whole ``num_steps`` flow loop; ``x_t`` is updated in place (the output).

    Same positional order as the reference ``launch``. ``ws`` = [w_qkv, w_so, w_cq, w_co, w_gu, w_dn]
    (bf16), ``bs`` = their fp32 biases. A leading batch dimension on ``x_t`` [B][T][32] (with
    ``kctx`` [B][NL][Lkmax][768] and ``vtctx`` [B][NL][768][Lkmax]) runs B samples in one launch.
    The scratch tensors x, xp, bufs, scores, probs and nblocks/nthreads are accepted and ignored: the
    engine keeps its intermediates in one workspace (``workspace()``). Rows [Tv, T) of x_t and dims
    >= adim are left untouched. stage_cycles accumulates 100 MHz GPU-clock ticks per stage.
    check_status=True waits for the launch and raises FlashActError (after re-initialising the
    workspace) on a non-zero kernel status.
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
    nl = int(ws[0].shape[0])
    Lk, Lkmax, Tv, adim, num_steps = int(Lk), int(Lkmax), int(Tv), int(adim), int(num_steps)
    check_shapes(ws, bs, mods, mod_final, rope_cos, rope_sin, w_ain, b_ain, w_aout, b_aout, kctx, vtctx, Lk, Lkmax, Tv,
                 adim, num_steps, x_t, nl, batch)
    if not x_t.is_cuda:
        raise ValueError("all tensors must be on the GPU (x_t is not)")
    dev = x_t.device
    wsp = workspace_tensor if workspace_tensor is not None else workspace(dev, batch, Tv, Lkmax)
    a = _lib.Ma2Args()
    a.weight_dtype = _lib.FA_DTYPE_BF16
    a.w_qkv, a.w_so, a.w_cq, a.w_co, a.w_gu, a.w_dn = (_ptr(t) for t in ws)
    a.b_qkv, a.b_so, a.b_cq, a.b_co, a.b_gu, a.b_dn = (_ptr(t) for t in bs)
    a.mods, a.mod_final = _ptr(mods), _ptr(mod_final)
    a.rope_cos, a.rope_sin = _ptr(rope_cos), _ptr(rope_sin)
    a.w_ain, a.b_ain, a.w_aout, a.b_aout = _ptr(w_ain), _ptr(b_ain), _ptr(w_aout), _ptr(b_aout)
    a.kctx, a.vtctx = _ptr(kctx), _ptr(vtctx)
    a.Lk, a.Lkmax, a.Tv, a.adim, a.num_steps = Lk, Lkmax, Tv, adim, num_steps
    a.num_layers, a.batch = nl, batch
    a.x_t, a.xt_rows = _ptr(x_t), int(x_t.shape[-2])
    if stage_cycles is not None and stage_cycles.numel() > 0:
        if stage_cycles.dtype != torch.int64 or stage_cycles.numel() < 16:
            raise TypeError("stage_cycles must be an int64 tensor with >= 16 entries")
        a.stage_cycles = _ptr(stage_cycles)
    a.workspace, a.workspace_bytes = wsp.data_ptr(), wsp.numel()
    stream = torch.cuda.current_stream(dev)
    _lib.check(L.fa_ma2_flow(ctypes.byref(a), ctypes.c_void_p(stream.cuda_stream)), "fa_ma2_flow")
    if check_status:
        stream.synchronize()
        st = read_status(wsp)
        if st != 0:
            _lib.check(L.fa_ma2_workspace_init(ctypes.c_void_p(wsp.data_ptr()), wsp.numel(),
                                               ctypes.c_void_p(stream.cuda_stream)), "fa_ma2_workspace_init")
            raise _lib.FlashActError(f"fa_ma2_flow kernel status {st:#x} ({pi05.describe_status(st)}): the chunk "
                                     "is invalid; the workspace was re-initialised")
