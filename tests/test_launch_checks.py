"""Host-side checks of the drop-in ``launch`` shims on the CPU (no kernel runs).

* Shape validation: every size the kernels address is checked before any device work, so a
  mismatched cache, modulation table or RoPE table raises ValueError instead of reaching a kernel
  (the reference's bindings take the same tensors unchecked: src/pi05/binding.cpp:38-56,
  src/molmoact2/binding.cpp:36-58).
* Kernel status: ``check_status`` / ``Pi05Policy.predict`` re-initialise the workspace and raise on
  a non-zero status word.
* fp16 caches (the reference's dtype, benchmarks/pi05/eval_numerics.py:83-85) through the C ABI:
  the shadow-buffer validation.
* MolmoAct2 context compaction against the reference's mask rule
  (benchmarks/molmoact2/eval_e2e.py:105-125, eval_numerics.py:123-132).
"""
import ctypes

import pytest
import torch

from flashact_amd import _lib, ma2, pi05, policy
from tests import policy_case as PC

NL, LP, TV, S, LMAX = 2, 40, 10, 3, 64


def _pi05_args(batch=1, **over):
    bf = torch.bfloat16
    a = dict(w1=torch.zeros(NL, 2560, 1024, dtype=bf), wo=torch.zeros(NL, 1024, 2048, dtype=bf),
             w2=torch.zeros(NL, 8192, 1024, dtype=bf), w3=torch.zeros(NL, 1024, 4096, dtype=bf),
             s1=None, so_=None, s2=None, s3=None,
             mods=torch.zeros(S, NL, 2, 3072), mod_final=torch.zeros(S, 3072),
             rope_cos=torch.zeros(16, 128), rope_sin=torch.zeros(16, 128),
             w_ain=torch.zeros(1024, 32), b_ain=torch.zeros(1024), w_aout=torch.zeros(32, 1024), b_aout=torch.zeros(32),
             kvsrc_k=None, kvsrc_v=None, srows=0,
             kcache=torch.zeros(batch, NL, LMAX, 256, dtype=bf), vtcache=torch.zeros(batch, NL, 256, LMAX, dtype=bf),
             Lp=LP, Lmax=LMAX, num_steps=S, Tv=TV,
             x_t=torch.zeros(batch, 16, 32) if batch > 1 else torch.zeros(16, 32))
    a.update(over)
    return a


def _call_pi05(a):
    order = ["w1", "wo", "w2", "w3", "s1", "so_", "s2", "s3", "mods", "mod_final", "rope_cos", "rope_sin", "w_ain",
             "b_ain", "w_aout", "b_aout", "kvsrc_k", "kvsrc_v", "srows", "kcache", "vtcache", "Lp", "Lmax",
             "num_steps", "Tv", "x_t"]
    pi05.launch(*[a[k] for k in order])


def test_pi05_well_formed_request_reaches_the_device_check():
    # every shape is right: the first failure is the CPU tensors themselves
    with pytest.raises(ValueError, match="on the GPU"):
        _call_pi05(_pi05_args())


@pytest.mark.parametrize("batch,over,text", [
    (2, dict(kcache=torch.zeros(NL, LMAX, 256, dtype=torch.bfloat16)), "kcache"),       # 2-D cache, 3-D x_t
    (2, dict(vtcache=torch.zeros(1, NL, 256, LMAX, dtype=torch.bfloat16)), "vtcache"),
    (1, dict(mods=torch.zeros(S - 1, NL, 2, 3072)), "mods"),
    (1, dict(mod_final=torch.zeros(S, 1024)), "mod_final"),
    (1, dict(rope_cos=torch.zeros(TV - 1, 128)), "rope_cos"),
    (1, dict(rope_sin=torch.zeros(16, 64)), "rope_sin"),
    (1, dict(Lmax=48), "Lmax"),
    (1, dict(Tv=65, x_t=torch.zeros(70, 32), rope_cos=torch.zeros(70, 128), rope_sin=torch.zeros(70, 128)), "Tv"),
    (1, dict(x_t=torch.zeros(8, 32)), "x_t"),
    (1, dict(w2=torch.zeros(NL, 4096, 1024, dtype=torch.bfloat16)), "w2"),
    (1, dict(kcache=torch.zeros(NL, 256, LMAX, dtype=torch.bfloat16)), "kcache"),  # transposed layout
    (1, dict(w_ain=torch.zeros(32, 1000)), "w_ain"),
    (1, dict(srows=LP, kvsrc_k=torch.zeros(NL, LP, 256, dtype=torch.bfloat16)), "kvsrc_v"),
])
def test_pi05_rejects_mismatched_shapes(batch, over, text):
    with pytest.raises(ValueError, match=text):
        _call_pi05(_pi05_args(batch, **over))


def test_pi05_rejects_mixed_cache_dtypes():
    with pytest.raises(TypeError, match="both"):
        _call_pi05(_pi05_args(vtcache=torch.zeros(1, NL, 256, LMAX, dtype=torch.float16)))


def _ma2_args(batch=1, **over):
    bf = torch.bfloat16
    D, FF, LK, LKM, nl = 768, 3072, 30, 32, 2
    ws = [torch.zeros(nl, 2304, D, dtype=bf), torch.zeros(nl, D, D, dtype=bf), torch.zeros(nl, D, D, dtype=bf),
          torch.zeros(nl, D, D, dtype=bf), torch.zeros(nl, 2 * FF, D, dtype=bf), torch.zeros(nl, D, FF, dtype=bf)]
    bs = [torch.zeros(nl, 2304), torch.zeros(nl, D), torch.zeros(nl, D), torch.zeros(nl, D), torch.zeros(nl, 2 * FF),
          torch.zeros(nl, D)]
    kshape = (batch, nl, LKM, D) if batch > 1 else (nl, LKM, D)
    vshape = (batch, nl, D, LKM) if batch > 1 else (nl, D, LKM)
    a = dict(ws=ws, bs=bs, mods=torch.zeros(S, nl, 3, 3, D), mod_final=torch.zeros(S, 2, D),
             rope_cos=torch.zeros(TV, 48), rope_sin=torch.zeros(TV, 48), w_ain=torch.zeros(D, 32),
             b_ain=torch.zeros(D), w_aout=torch.zeros(32, D, dtype=bf), b_aout=torch.zeros(32),
             kctx=torch.zeros(*kshape, dtype=bf), vtctx=torch.zeros(*vshape, dtype=bf), Lk=LK, Lkmax=LKM, Tv=TV,
             adim=6, num_steps=S, x_t=torch.zeros(batch, 16, 32) if batch > 1 else torch.zeros(16, 32))
    a.update(over)
    return a


def _call_ma2(a):
    order = ["ws", "bs", "mods", "mod_final", "rope_cos", "rope_sin", "w_ain", "b_ain", "w_aout", "b_aout", "kctx",
             "vtctx", "Lk", "Lkmax", "Tv", "adim", "num_steps", "x_t"]
    ma2.launch(*[a[k] for k in order])


def test_ma2_well_formed_request_reaches_the_device_check():
    with pytest.raises(ValueError, match="on the GPU"):
        _call_ma2(_ma2_args())


@pytest.mark.parametrize("batch,over,text", [
    (2, dict(kctx=torch.zeros(2, 32, 768, dtype=torch.bfloat16)), "kctx"),
    (1, dict(mods=torch.zeros(S, 2, 3, 768)), "mods"),
    (1, dict(rope_cos=torch.zeros(TV - 1, 48)), "rope_cos"),
    (1, dict(Lk=40), "Lkmax"),
    (1, dict(adim=0), "adim"),
    (1, dict(x_t=torch.zeros(16, 6)), "x_t"),
])
def test_ma2_rejects_mismatched_shapes(batch, over, text):
    with pytest.raises(ValueError, match=text):
        _call_ma2(_ma2_args(batch, **over))


class _Stream:
    def synchronize(self):
        pass


def test_status_word_raises_and_reinitialises(monkeypatch):
    calls = []
    monkeypatch.setattr(pi05, "read_status", lambda ws: 1)
    monkeypatch.setattr(pi05, "reset_workspace", lambda ws: calls.append("reset"))
    with pytest.raises(_lib.FlashActError, match="status 0x1"):
        pi05.raise_on_status(torch.zeros(4), _Stream())
    assert calls == ["reset"]
    monkeypatch.setattr(pi05, "read_status", lambda ws: 0)
    pi05.raise_on_status(torch.zeros(4), _Stream())  # status 0: no error, no reset
    assert calls == ["reset"]


def test_predict_checks_the_kernel_status(monkeypatch):
    seen = {}

    def fake_launch(*args, **kw):
        seen.update(kw)

    pol = policy.Pi05Policy(PC.checkpoint(NL=2, seed=1), device="cpu", load_backbone=False, chunk_size=10)
    monkeypatch.setattr(pi05, "launch", fake_launch)
    out = pol.predict(kv_rows=(torch.zeros(2, 16, 256, dtype=torch.bfloat16),
                               torch.zeros(2, 16, 256, dtype=torch.bfloat16), 16))
    assert seen.get("check_status") is True and out.shape == (10, 32)


def test_predict_checks_the_prefill_status(monkeypatch):
    """A prefill whose status is non-zero leaves the caches unfinished: predict asks prefill to check
    its status, and a raise there stops the chunk before the denoise loop reads the caches."""
    from flashact_amd import prefill
    seen = {}
    pol = policy.Pi05Policy(PC.checkpoint(NL=2, seed=1), device="cpu", load_backbone=False, chunk_size=10)
    pol.backbone = {"packed": None, "ln_in": None, "ln_post": None}
    monkeypatch.setattr(prefill, "prefill", lambda *a, **kw: seen.setdefault("prefill", kw))
    monkeypatch.setattr(pi05, "launch", lambda *a, **kw: seen.setdefault("launch", kw))
    pol.predict(prefix_hidden=torch.zeros(16, 2048))
    assert seen["prefill"].get("check_status") is True and seen["launch"].get("check_status") is True

    def bad_prefill(*a, **kw):
        raise _lib.FlashActError("fa_pi05_prefill kernel status 0x1")
    seen.clear()
    monkeypatch.setattr(prefill, "prefill", bad_prefill)
    with pytest.raises(_lib.FlashActError, match="prefill"):
        pol.predict(prefix_hidden=torch.zeros(16, 2048))
    assert "launch" not in seen


@pytest.mark.parametrize("st,text", [(1, "capped barrier wait"), (2, "XCD"), (4, "fp16 range"),
                                     (5, "capped barrier wait expired; 4 = an exchanged"), (8, "unknown bits 0x8")])
def test_status_message_names_every_bit(monkeypatch, st, text):
    monkeypatch.setattr(pi05, "read_status", lambda ws: st)
    monkeypatch.setattr(pi05, "reset_workspace", lambda ws: None)
    with pytest.raises(_lib.FlashActError, match=text):
        pi05.raise_on_status(torch.zeros(4), _Stream())


def test_status_bits_match_the_header():
    import os
    import re
    hdr = open(os.path.join(os.path.dirname(__file__), "..", "include", "flashact_mi355x.h")).read()
    bits = {int(v.rstrip("u")) for v in re.findall(r"#define FA_KSTATUS_\w+ (\d+u)", hdr)}
    assert bits == set(pi05.STATUS_BITS)


def _c_args(**kw):
    a = _lib.Pi05Args()
    fake = 1 << 20
    for f in ("w1", "wo", "w2", "w3", "mods", "mod_final", "rope_cos", "rope_sin", "w_ain", "b_ain", "w_aout",
              "b_aout", "kcache", "vtcache", "x_t", "workspace"):
        setattr(a, f, fake)
    a.Lp, a.Lmax, a.num_steps, a.Tv, a.num_layers, a.batch, a.xt_rows = 968, 1024, 10, 50, 18, 1, 50
    a.workspace_bytes = 1 << 30
    for k, v in kw.items():
        setattr(a, k, v)
    return a


# fp16 caches need the bf16 shadow only where the loop does not run on them directly: batch >= 2 or
# a hand-off (srows > 0)
@pytest.mark.parametrize("kw,text", [
    (dict(cache_dtype=_lib.FA_DTYPE_F16, batch=2), "cache_shadow"),
    (dict(cache_dtype=_lib.FA_DTYPE_F16, srows=968, kvsrc_k=1 << 20, kvsrc_v=1 << 21), "cache_shadow"),
    (dict(cache_dtype=_lib.FA_DTYPE_F16, batch=2, cache_shadow=(1 << 20) + 16, cache_shadow_bytes=1 << 30),
     "cache_shadow"),
    (dict(cache_dtype=_lib.FA_DTYPE_F16, batch=2, cache_shadow=1 << 20, cache_shadow_bytes=1 << 20), "cache_shadow"),
    (dict(cache_dtype=7), "cache_dtype"),
])
def test_c_abi_fp16_cache_validation(kw, text):
    L = _lib.lib()
    rc = L.fa_pi05_denoise(ctypes.byref(_c_args(**kw)), None)
    assert rc == 1 and text in L.fa_last_error().decode()


def test_c_abi_fp16_caches_at_batch_1_need_no_shadow():
    """The reference's own call (batch 1, no hand-off) runs on the fp16 caches: no shadow is asked for,
    and the request gets as far as the device check (there is no GPU here)."""
    L = _lib.lib()
    rc = L.fa_pi05_denoise(ctypes.byref(_c_args(cache_dtype=_lib.FA_DTYPE_F16)), None)
    err = L.fa_last_error().decode()
    assert "cache_shadow" not in err and rc != 0


def test_cache_shadow_bytes():
    L = _lib.lib()
    assert L.fa_pi05_cache_shadow_bytes(1, 18, 1024) == 2 * 18 * 1024 * 256 * 2
    assert L.fa_pi05_cache_shadow_bytes(16, 18, 1024) == 16 * 2 * 18 * 1024 * 256 * 2
    assert L.fa_pi05_cache_shadow_bytes(1, 18, 1000) == 0  # Lmax must be a multiple of 16


def test_context_compaction_follows_the_reference_rule():
    g = torch.Generator().manual_seed(3)
    nl, L = 3, 40
    kv = [(torch.randn(1, L, 8, 96, generator=g), torch.randn(1, L, 8, 96, generator=g)) for _ in range(nl)]
    valid = torch.rand(L, generator=g) > 0.3
    # additive float mask [B][1][T][L]: 0 where attended, large negative where masked (eval_e2e.py:107-113)
    add = torch.where(valid, 0.0, -1e9).reshape(1, 1, 1, L).expand(1, 1, 5, L).contiguous()
    for mask in (add, valid.reshape(1, L)):
        kctx, vtctx, Lk = ma2.compact_context(kv, mask)
        assert Lk == int(valid.sum()) and kctx.shape == (nl, (Lk + 15) // 16 * 16, 768)
        for l, (k, v) in enumerate(kv):
            rows = [i for i in range(L) if valid[i]]  # valid rows kept in order
            assert torch.equal(kctx[l, :Lk], k[0, rows].reshape(Lk, 768).bfloat16())
            assert torch.equal(vtctx[l, :, :Lk], v[0, rows].reshape(Lk, 768).t().bfloat16())
            assert torch.count_nonzero(kctx[l, Lk:]) == 0 and torch.count_nonzero(vtctx[l, :, Lk:]) == 0
    kctx, _, Lk = ma2.compact_context(kv, None)
    assert Lk == L and torch.equal(kctx[1, :L], kv[1][0][0].reshape(L, 768).bfloat16())
    with pytest.raises(ValueError):
        ma2.compact_context(kv, torch.ones(1, L + 1, dtype=torch.bool))
