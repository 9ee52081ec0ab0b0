"""A small seeded vision-tower case shared by the reference fixture script
(make_ref_vit_fp8.py) and the oracle tests that read its output.

The tower: Qwen2-VL's ViT at reduced width and depth (embed 160, 2 heads of head_dim 80
as in the real tower, MLP 640, 2 blocks, 2 x 2 patch merge -> merged width 640, out 192),
14 px patches over 2 frames and 3 channels (patch_dim 1176), rotary theta 1e4.  Two
images: grid (t, h, w) = (1, 4, 6) and (2, 4, 4), i.e. three attention segments of 24,
16 and 16 patches and 14 merged rows.  Weights are Hugging Face ``visual.*`` state-dict
tensors holding fp16 values; everything is regenerated from the seed on the CPU, so the
fixture stores outputs only.
"""

from __future__ import annotations

import torch

SEED = 4242
EMBED, DEPTH, HEADS, MLP, OUT, MERGE = 160, 2, 2, 640, 192, 2
IN_CH, PATCH, TPATCH = 3, 14, 2
PATCH_DIM = IN_CH * TPATCH * PATCH * PATCH
THETA = 10000.0
GRIDS = [(1, 4, 6), (2, 4, 4)]


def _g(tag: str) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(SEED * 1000 + sum(ord(c) * (i + 1) for i, c in enumerate(tag)))
    return g


def _r(shape, std, tag, mean=0.0):
    return (mean + torch.randn(*shape, generator=_g(tag)) * std).half().float()


def state_dict():
    """fp32 tensors holding fp16 values under the checkpoint's ``visual.*`` names
    (model/qwen2_vit.py:132-147); the patch embedding in its Conv3d shape."""
    merged = EMBED * MERGE * MERGE
    sd = {"visual.patch_embed.proj.weight": _r((EMBED, IN_CH, TPATCH, PATCH, PATCH), 0.02, "pe")}
    for i in range(DEPTH):
        p = f"visual.blocks.{i}."
        for n in ("norm1", "norm2"):
            sd[p + n + ".weight"] = _r((EMBED,), 0.1, f"{n}w{i}", 1.0)
            sd[p + n + ".bias"] = _r((EMBED,), 0.1, f"{n}b{i}")
        for n, shape in (("attn.qkv", (3 * EMBED, EMBED)), ("attn.proj", (EMBED, EMBED)),
                         ("mlp.fc1", (MLP, EMBED)), ("mlp.fc2", (EMBED, MLP))):
            sd[p + n + ".weight"] = _r(shape, 0.05, f"{n}w{i}")
            sd[p + n + ".bias"] = _r((shape[0],), 0.05, f"{n}b{i}")
    sd["visual.merger.ln_q.weight"] = _r((EMBED,), 0.1, "lnw", 1.0)
    sd["visual.merger.ln_q.bias"] = _r((EMBED,), 0.1, "lnb")
    sd["visual.merger.mlp.0.weight"] = _r((merged, merged), 0.03, "m0w")
    sd["visual.merger.mlp.0.bias"] = _r((merged,), 0.05, "m0b")
    sd["visual.merger.mlp.2.weight"] = _r((OUT, merged), 0.03, "m2w")
    sd["visual.merger.mlp.2.bias"] = _r((OUT,), 0.05, "m2b")
    return sd


def pixels():
    """Flattened patches [S, PATCH_DIM] (fp16 values), S = sum of t h w over GRIDS."""
    S = sum(t * h * w for t, h, w in GRIDS)
    return _r((S, PATCH_DIM), 1.0, "pixels")
