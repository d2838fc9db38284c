"""FlashAct for MI355X: the flow-matching denoise loop of VLA action experts on gfx950.

Modules:
  pi05       -- pi0.5 (Gemma-300M-shaped) expert: ``launch`` (drop-in for src/pi05 ``mk_v6.launch``),
                packing, RoPE table, KV compaction, modulation precompute.
  synthetic  -- seeded synthetic weights and inputs of the benchmark shapes.
  build      -- builds libflashact_mi355x.so in-tree with hipcc (gfx950).
"""
__all__ = ["pi05", "synthetic", "build"]
