"""Seeded inputs of the FP8 W8A8 fixture (make_ref_vit_fp8.py) and the oracle tests that
read it.

Linear level: one fp16 weight [N, K] with a bias and one activation matrix [M, K] (fp16,
and the same values in bf16), quantised and multiplied by the reference's FP8Linear in
both of its forms (per-tensor, the default; row-wise).

Decoder level: the composition case of composition_case.py (3 layers, hidden 384, MLP
640) under the reference's two FP8 plans:
  "mixed"  models/qwen2_vl.py:61-63, apply_mixed(model) with DEFAULT_PLAN: gate_up and
           down per-tensor FP8Linear, qkv / o fp16;
  "fused"  benchmarks/compare/bench_fused_norm_fp8.py:36-40: apply_mixed with gate_up left
           fp16 and down FP8, then fuse_norm_fp8: gate_up row-wise FP8 fed by the
           post-attention norm's e4m3 rows (forward_prequant, bf16 out, bf16 silu_mul).
"""

from __future__ import annotations

import torch

SEED = 808
N, K, M = 256, 384, 24
PLANS = {
    "mixed": {"qkv": "fp16", "o": "fp16", "gate_up": "fp8", "down": "fp8"},
    "fused": {"qkv": "fp16", "o": "fp16", "gate_up": "fp16", "down": "fp8"},
}


def _g(tag: str) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(SEED * 1000 + sum(ord(c) * (i + 1) for i, c in enumerate(tag)))
    return g


def linear_case():
    """(W [N, K], bias [N], x [M, K]) as fp32 tensors holding fp16 values.  Two rows of x
    carry an outlier so that per-tensor and per-token scales differ."""
    w = (torch.randn(N, K, generator=_g("w")) * 0.05).half().float()
    b = (torch.randn(N, generator=_g("b")) * 0.1).half().float()
    x = torch.randn(M, K, generator=_g("x")).half().float()
    x[3, 17] = 9.5
    x[11, 200] = -14.0
    return w, b, x
