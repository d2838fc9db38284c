"""Policy wrappers: checkpoint loading and a ``predict`` call over the MI355X kernels.

``Pi05Policy`` (pi0.5) and ``Ma2Policy`` (MolmoAct2, at the end of this file).

Mirrors the reference's ``HybridPi05`` (src/pi05/hybrid_model.py:23-228) minus its FlashRT
front-end (vision encoder, tokenizer, encoder CUDA graph), which is outside this build:

  * weights come from the same checkpoint keys (``paligemma_with_expert.gemma_expert.model.*``,
    ``time_mlp_in/out``, ``action_in/out_proj``; hybrid_model.py:94-132), read from a
    ``.safetensors`` file or a state dict; the backbone layers (for the prefill) from the PaliGemma
    language-model keys of the same checkpoint;
  * ``weight_format="fp8"`` quantises the expert weights per row to e4m3 as the reference does
    (hybrid_model.py:105-110) and runs the FP8-W8A16 loop;
  * the adaRMS modulations are computed once on the device for the fixed schedule
    t_i = 1 - i / num_steps (hybrid_model.py:111-128);
  * ``predict`` takes the prefix either as hidden states (the backbone prefill runs on the GPU and
    writes the expert's caches) or as the K/V rows of another prefill with interleaved RoPE pairs
    (the reference's FlashRT hand-off, hybrid_model.py:199-221), draws the initial noise in the
    reference's modes ("gaussian", "zero", "scale"; :206-211) and returns the raw chunk
    [chunk_size][32] (the reference's ``return_raw``; un-normalisation needs FlashRT's norm stats).

There is no fallback: every call runs the HIP kernels through the C ABI.
"""
from __future__ import annotations

import os
import re

import numpy as np
import torch

from . import ma2, pi05, prefill

EXPERT = "paligemma_with_expert.gemma_expert.model."
D, HD, F, AD = 1024, 256, 4096, 32


class _Source:
    """Key -> tensor access over a state dict or a safetensors file (nothing is executed from it)."""

    def __init__(self, source):
        if isinstance(source, (str, os.PathLike)):
            from safetensors import safe_open
            self._h = safe_open(str(source), framework="pt", device="cpu")
            self._keys = set(self._h.keys())
            self._get = self._h.get_tensor
        else:
            self._keys = set(source.keys())
            self._get = source.__getitem__

    def keys(self):
        return self._keys

    def __getitem__(self, k):
        return self._get(k)

    def __contains__(self, k):
        return k in self._keys


def _count_layers(src, prefix):
    pat = re.compile(re.escape(prefix) + r"layers\.(\d+)\.self_attn\.q_proj\.weight$")
    ids = [int(m.group(1)) for k in src.keys() for m in [pat.match(k)] if m]
    return max(ids) + 1 if ids else 0


def find_backbone_prefix(src) -> str | None:
    """The PaliGemma language-model layer prefix of an openpi checkpoint (it differs between
    transformers versions): the prefix P with P + 'layers.0.self_attn.q_proj.weight' of width 2048."""
    for k in sorted(src.keys()):
        if k.endswith("layers.0.self_attn.q_proj.weight") and not k.startswith(EXPERT):
            if src[k].shape[-1] == prefill.D:
                return k[: -len("layers.0.self_attn.q_proj.weight")]
    return None


class Pi05Policy:
    """Expert (and optionally backbone) weights resident on one GPU, ready for ``predict``."""

    def __init__(self, checkpoint, *, num_steps: int = 10, chunk_size: int = 50, device="cuda",
                 initial_noise_mode: str = "gaussian", initial_noise_scale: float = 1.0, load_backbone: bool = True,
                 weight_format: str = "bf16"):
        if weight_format not in {"bf16", "fp8"}:
            raise ValueError(f"weight_format must be 'bf16' or 'fp8' (per-row e4m3, as the reference), got {weight_format}")
        self.weight_format = weight_format
        if initial_noise_mode not in {"gaussian", "zero", "scale"}:
            raise ValueError(f"unsupported initial noise mode: {initial_noise_mode}")
        if not 1 <= chunk_size <= 64:
            raise ValueError(f"chunk_size must be in [1, 64], got {chunk_size}")
        self.num_steps, self.chunk_size = int(num_steps), int(chunk_size)
        self.initial_noise_mode, self.initial_noise_scale = initial_noise_mode, float(initial_noise_scale)
        self.device = torch.device(device)
        src = _Source(checkpoint)
        self.num_layers = _count_layers(src, EXPERT)
        if self.num_layers == 0:
            raise KeyError(f"no expert layers under {EXPERT!r} in the checkpoint")
        self._load_expert(src)
        self.backbone = None
        if load_backbone:
            bp = find_backbone_prefix(src)
            if bp is not None:
                self._load_backbone(src, bp)

    # ------------------------------------------------------------------ loading
    def _stack(self, src, prefix, name, n):
        return torch.stack([src[f"{prefix}layers.{i}.{name}"].to(self.device) for i in range(n)])

    def _load_expert(self, src):
        NL, dev = self.num_layers, self.device
        st = lambda n: self._stack(src, EXPERT, n, NL)  # noqa: E731
        pack = pi05.pack_weights_fp8 if self.weight_format == "fp8" else pi05.pack_weights
        self.packed = pack(st("self_attn.q_proj.weight"), st("self_attn.k_proj.weight"),
                           st("self_attn.v_proj.weight"), st("self_attn.o_proj.weight"),
                           st("mlp.gate_proj.weight"), st("mlp.up_proj.weight"), st("mlp.down_proj.weight"))
        f = lambda k: src[k].float().to(dev).contiguous()  # noqa: E731
        self.mods, self.mod_final = pi05.precompute_mods(
            self.num_steps, f("time_mlp_in.weight"), f("time_mlp_in.bias"), f("time_mlp_out.weight"),
            f("time_mlp_out.bias"),
            st("input_layernorm.dense.weight").float(), st("input_layernorm.dense.bias").float(),
            st("post_attention_layernorm.dense.weight").float(), st("post_attention_layernorm.dense.bias").float(),
            f(EXPERT + "norm.dense.weight"), f(EXPERT + "norm.dense.bias"))
        self.w_ain, self.b_ain = f("action_in_proj.weight"), f("action_in_proj.bias")
        self.w_aout, self.b_aout = f("action_out_proj.weight"), f("action_out_proj.bias")

    def _load_backbone(self, src, bp):
        n = _count_layers(src, bp)
        if n != self.num_layers:
            raise ValueError(f"backbone has {n} layers, the expert {self.num_layers}: each expert layer reads the "
                             "same-index backbone layer's cache")
        st = lambda name: self._stack(src, bp, name, n)  # noqa: E731
        self.backbone = {
            "packed": prefill.pack_backbone(st("self_attn.q_proj.weight"), st("self_attn.k_proj.weight"),
                                            st("self_attn.v_proj.weight"), st("self_attn.o_proj.weight"),
                                            st("mlp.gate_proj.weight"), st("mlp.up_proj.weight"),
                                            st("mlp.down_proj.weight")),
            "ln_in": st("input_layernorm.weight").float().contiguous(),
            "ln_post": st("post_attention_layernorm.weight").float().contiguous(),
        }

    # ------------------------------------------------------------------ inference
    def initial_noise(self, generator=None) -> torch.Tensor:
        x = torch.zeros(self.chunk_size, AD, dtype=torch.float32, device=self.device)
        if self.initial_noise_mode != "zero":
            x.normal_(generator=generator)
            if self.initial_noise_mode == "scale":
                x.mul_(self.initial_noise_scale)
        return x

    def predict(self, prefix_hidden=None, *, kv_rows=None, noise=None, generator=None) -> np.ndarray:
        """One action chunk [chunk_size][32] (raw, fp32).

        prefix_hidden [Lp][2048] fp32: hidden states entering backbone layer 0 -> the prefill fills
        the caches. Or kv_rows = (k_rows, v_rows) [NL][srows][256] bf16 with RoPE on interleaved
        pairs plus the prefix length Lp as kv_rows[2] -> the hand-off fills them.
        """
        dev = self.device
        if (prefix_hidden is None) == (kv_rows is None):
            raise ValueError("pass exactly one of prefix_hidden and kv_rows")
        if prefix_hidden is not None:
            if self.backbone is None:
                raise ValueError("the checkpoint has no backbone layers: pass kv_rows")
            Lp = int(prefix_hidden.shape[-2])
        else:
            Lp = int(kv_rows[2])
        Lmax = pi05.lmax_for(Lp, self.chunk_size)
        kc = torch.zeros(self.num_layers, Lmax, HD, dtype=torch.bfloat16, device=dev)
        vc = torch.zeros(self.num_layers, HD, Lmax, dtype=torch.bfloat16, device=dev)
        ksrc = vsrc = None
        srows = 0
        if prefix_hidden is not None:
            b = self.backbone
            # check_status: a prefill whose barriers expired leaves the caches unfinished; it raises
            # here (after re-initialising its workspace) before the denoise loop reads them
            prefill.prefill(b["packed"], b["ln_in"], b["ln_post"], prefix_hidden.to(dev, torch.float32).contiguous(),
                            kc, vc, check_status=True)
        else:
            ksrc, vsrc = kv_rows[0].contiguous(), kv_rows[1].contiguous()
            srows = int(ksrc.shape[-2])
        x_t = (noise.to(dev, torch.float32).clone() if noise is not None else self.initial_noise(generator))
        cos, sin = pi05.rope_table(Lp, self.chunk_size, device=dev)
        p = self.packed
        empty = torch.empty(0, device=dev)
        sc = [p.get(k, empty) for k in ("s1", "so", "s2", "s3")]
        # check_status: waits for the chunk and raises (after re-initialising the workspace) if a
        # capped wait expired, the XCD placement differed or an exchanged partial sum left the fp16
        # range, so an invalid chunk is never returned
        pi05.launch(p["w1"], p["wo"], p["w2"], p["w3"], *sc, self.mods, self.mod_final,
                    cos, sin, self.w_ain, self.b_ain, self.w_aout, self.b_aout, ksrc, vsrc, srows, kc, vc, Lp, Lmax,
                    self.num_steps, self.chunk_size, x_t, check_status=True)
        return x_t.cpu().numpy()


# ---------------------------------------------------------------- MolmoAct2
MA2_LAYER = "blocks.0.self_attn.qkv.weight"


def find_ma2_prefix(src) -> str | None:
    """The action expert's prefix P in a MolmoAct2 state dict: P + 'blocks.0.self_attn.qkv.weight'."""
    for k in sorted(src.keys()):
        if k.endswith(MA2_LAYER):
            return k[: -len(MA2_LAYER)]
    return None


class Ma2Policy:
    """MolmoAct2 action-expert weights resident on one GPU, ready for ``predict``.

    Mirrors the reference's MolmoAct2 harness (benchmarks/molmoact2/eval_numerics.py:77-133,
    eval_e2e.py:81-144) without the HF model around the expert:
      * the weights are read by module name from a state dict or ``.safetensors`` file, under the expert's
        prefix P (found as the P with P + 'blocks.0.self_attn.qkv.weight', or given): per layer l
        ``blocks.l.self_attn.qkv`` [2304][768], ``self_attn.out_proj``, ``cross_attn.q_proj``,
        ``cross_attn.out_proj`` [768][768], ``mlp.gate_proj`` / ``mlp.up_proj`` [3072][768],
        ``mlp.down_proj`` [768][3072] (weights and biases), then ``action_embed`` [768][32] and
        ``final_layer.linear`` [32][768]; gate/up rows and biases are interleaved as the reference packs
        them (eval_numerics.py:88-93);
      * the per-step modulations, the encoder context and the RoPE base come from the HF model's
        ``prepare_modulation_cache``, ``prepare_context`` and rotary module in the reference; ``predict``
        takes them as inputs, in the reference's packed layouts.
    There is no fallback: every call runs the HIP kernels through the C ABI.
    """

    def __init__(self, checkpoint, *, expert_prefix: str | None = None, num_steps: int = 10, chunk_size: int = 30,
                 action_dims: int = 6, device="cuda"):
        if not 1 <= chunk_size <= ma2.MAX_TV:
            raise ValueError(f"chunk_size must be in [1, {ma2.MAX_TV}], got {chunk_size}")
        if not 0 <= action_dims <= AD:
            raise ValueError(f"action_dims must be in [0, {AD}], got {action_dims}")
        self.num_steps, self.chunk_size, self.adim = int(num_steps), int(chunk_size), int(action_dims)
        self.device = torch.device(device)
        src = _Source(checkpoint)
        P = expert_prefix if expert_prefix is not None else find_ma2_prefix(src)
        if P is None or P + MA2_LAYER not in src:
            raise KeyError(f"no MolmoAct2 expert layers ('...{MA2_LAYER}') in the checkpoint")
        pat = re.compile(re.escape(P) + r"blocks\.(\d+)\.self_attn\.qkv\.weight$")
        self.num_layers = max(int(m.group(1)) for k in src.keys() for m in [pat.match(k)] if m) + 1
        dev, NL = self.device, self.num_layers

        def st(name, shape):
            ts = []
            for l in range(NL):
                key = f"{P}blocks.{l}.{name}"
                t = src[key]
                if tuple(t.shape) != shape:
                    raise ValueError(f"{key}: shape {tuple(t.shape)}, expected {shape}")
                ts.append(t.to(dev))
            return torch.stack(ts)

        D, FF = ma2.D, ma2.FF
        proj = (("self_attn.qkv", 3 * D, D), ("self_attn.out_proj", D, D), ("cross_attn.q_proj", D, D),
                ("cross_attn.out_proj", D, D), ("mlp.gate_proj", FF, D), ("mlp.up_proj", FF, D),
                ("mlp.down_proj", D, FF))
        w = [st(n + ".weight", (o, i)) for n, o, i in proj]
        b = [st(n + ".bias", (o,)) for n, o, i in proj]
        self.ws, self.bs = ma2.pack_weights(*w, *b)
        f = lambda k: src[P + k].float().to(dev).contiguous()  # noqa: E731
        self.w_ain, self.b_ain = f("action_embed.weight"), f("action_embed.bias")
        self.w_aout = src[P + "final_layer.linear.weight"].to(dev).to(torch.bfloat16).contiguous()
        self.b_aout = f("final_layer.linear.bias")
        if tuple(self.w_ain.shape) != (ma2.D, AD) or tuple(self.w_aout.shape) != (AD, ma2.D):
            raise ValueError(f"action_embed {tuple(self.w_ain.shape)} / final_layer.linear {tuple(self.w_aout.shape)}: "
                             f"expected ({ma2.D}, {AD}) / ({AD}, {ma2.D})")

    def initial_noise(self, generator=None) -> torch.Tensor:
        """N(0, 1) [chunk_size][32] with the dims past action_dims zeroed (eval_numerics.py:62-65)."""
        x = torch.zeros(self.chunk_size, AD, dtype=torch.float32, device=self.device)
        x.normal_(generator=generator)
        x[:, self.adim:] = 0
        return x

    def predict(self, kv_contexts, mods, mod_final, *, cross_mask=None, rope=None, noise=None,
                generator=None) -> np.ndarray:
        """One action chunk [chunk_size][32] (fp32; dims past action_dims stay as the noise left them, 0).

        kv_contexts: per layer (k, v), each [1][L][8][96] or [1][L][768] (the encoder's context, as
        ``prepare_context`` gives it), compacted to the rows ``cross_mask`` keeps (``ma2.compact_context``);
        mods [num_steps][NL][3][3][768] fp32: (scale, shift, gate) of the self-attention, cross-attention
        and MLP norms; mod_final [num_steps][2][768]: (scale, shift) of the final norm
        (eval_numerics.py:97-110); rope: (cos, sin) [chunk_size][48], default ``ma2.rope_table`` (base
        10000; the model's rotary module sets it); noise [chunk_size][32], default ``initial_noise``.
        """
        dev, NL, S, Tv = self.device, self.num_layers, self.num_steps, self.chunk_size
        if len(kv_contexts) != NL:
            raise ValueError(f"kv_contexts has {len(kv_contexts)} layers, the expert {NL}")
        mods = mods.to(dev, torch.float32).contiguous()
        mod_final = mod_final.to(dev, torch.float32).contiguous()
        if tuple(mods.shape) != (S, NL, 3, 3, ma2.D) or tuple(mod_final.shape) != (S, 2, ma2.D):
            raise ValueError(f"mods {tuple(mods.shape)} / mod_final {tuple(mod_final.shape)}: expected "
                             f"{(S, NL, 3, 3, ma2.D)} / {(S, 2, ma2.D)}")
        kctx, vtctx, Lk = ma2.compact_context([(k.to(dev), v.to(dev)) for k, v in kv_contexts], cross_mask)
        cos, sin = rope if rope is not None else ma2.rope_table(Tv, device=dev)
        cos, sin = cos.to(dev, torch.float32).contiguous(), sin.to(dev, torch.float32).contiguous()
        x_t = noise.to(dev, torch.float32).clone() if noise is not None else self.initial_noise(generator)
        if tuple(x_t.shape) != (Tv, AD):
            raise ValueError(f"noise {tuple(x_t.shape)}: expected {(Tv, AD)}")
        # check_status: waits for the chunk and raises (after re-initialising the workspace) on a capped
        # wait or an unexpected XCD placement, so an invalid chunk is never returned
        ma2.launch(self.ws, self.bs, mods, mod_final, cos, sin, self.w_ain, self.b_ain, self.w_aout, self.b_aout,
                   kctx, vtctx, Lk, int(kctx.shape[1]), Tv, self.adim, S, x_t, check_status=True)
        return x_t.cpu().numpy()
