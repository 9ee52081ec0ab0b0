"""A small seeded decoder case shared by the reference-composition fixture script
(make_ref_composition.py) and the oracle tests that read its output.

The case: a 3-layer Qwen2-shaped decoder (hidden 384, 4 query / 2 KV heads of 128,
MLP 640, vocab 1000, M-RoPE sections [16, 24, 24]) with seeded weights, two prompts
(one text-only, one with a 4-row image run between vision-start / vision-end tokens,
M-RoPE 3-D positions) prefilled one at a time into pool rows 0 and 1, then four decode
steps of both rows with fixed (teacher-forced) token ids.  Everything is regenerated from
the seed on the CPU, so the fixture stores outputs only.
"""

from __future__ import annotations

import torch

SEED = 2024
HIDDEN, LAYERS, HEADS, KV_HEADS, HEAD_DIM, INTER, VOCAB = 384, 3, 4, 2, 128, 640, 1000
EPS, THETA, SECTIONS = 1e-6, 1_000_000.0, [16, 24, 24]
IMAGE_TOKEN_ID, VISION_START_ID, VISION_END_ID = 151655, 151652, 151653
# inside the small vocabulary the prompt's special tokens take the last three ids
CASE_IMAGE_ID, CASE_VSTART_ID, CASE_VEND_ID = VOCAB - 3, VOCAB - 2, VOCAB - 1
MAX_LEN = 48
DECODE_STEPS = 4


def _g(tag: str) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(SEED * 1000 + sum(ord(c) * (i + 1) for i, c in enumerate(tag)))
    return g


def randn(shape, std, tag):
    return torch.randn(*shape, generator=_g(tag)) * std


def weights():
    """fp32 weights holding fp16 values, nn.Linear layout [out, in], fused q|k|v, gate|up."""
    qkv = (HEADS + 2 * KV_HEADS) * HEAD_DIM
    r16 = lambda t: t.half().float()
    w = {"embed": r16(randn((VOCAB, HIDDEN), 0.05, "embed")),
         "norm": r16(1.0 + randn((HIDDEN,), 0.1, "norm")), "layers": []}
    for i in range(LAYERS):
        w["layers"].append({
            "in_norm": r16(1.0 + randn((HIDDEN,), 0.1, f"in{i}")),
            "post_norm": r16(1.0 + randn((HIDDEN,), 0.1, f"post{i}")),
            "qkv_w": r16(randn((qkv, HIDDEN), 0.05, f"qkv{i}")),
            "qkv_b": r16(randn((qkv,), 0.1, f"qkvb{i}")),
            "o_w": r16(randn((HIDDEN, HEADS * HEAD_DIM), 0.05, f"o{i}")),
            "gate_up_w": r16(randn((2 * INTER, HIDDEN), 0.05, f"gu{i}")),
            "down_w": r16(randn((HIDDEN, INTER), 0.05, f"down{i}")),
        })
    return w


def prompts():
    """[(ids, image rows or None, grids)] for pool rows 0 and 1 (special tokens are
    CASE_IMAGE_ID / CASE_VSTART_ID / CASE_VEND_ID)."""
    g = _g("prompts")
    a = torch.randint(0, VOCAB - 3, (13,), generator=g).tolist()
    b_pre = torch.randint(0, VOCAB - 3, (3,), generator=g).tolist()
    b_post = torch.randint(0, VOCAB - 3, (3,), generator=g).tolist()
    # grid (t, h, w) = (1, 4, 4) -> (4/2) * (4/2) = 4 merged rows
    b = b_pre + [CASE_VSTART_ID] + [CASE_IMAGE_ID] * 4 + [CASE_VEND_ID] + b_post
    img = randn((4, HIDDEN), 0.5, "image").half().float()
    return [(a, None, []), (b, img, [(1, 4, 4)])]


def decode_ids():
    """[DECODE_STEPS][2] token ids fed to the decode steps (teacher forcing)."""
    return torch.randint(0, VOCAB, (DECODE_STEPS, 2), generator=_g("decode")).tolist()


def position_cases():
    """Token sequences for the M-RoPE position function with their image grids: a config-5
    style prompt, two adjacent images, an image run without a preceding vision-start token,
    and a vision-start that is not followed by an image."""
    I, S, E = IMAGE_TOKEN_ID, VISION_START_ID, VISION_END_ID
    return [
        ([5] * 6 + [S] + [I] * 16 + [E] + [6] * 5, [(1, 8, 8)]),
        ([1, 2, S] + [I] * 4 + [E, S] + [I] * 9 + [E, 3], [(1, 4, 4), (1, 6, 6)]),
        ([1, 2] + [I] * 4 + [3, S] + [I] * 4 + [E, 4], [(1, 4, 4), (1, 4, 4)]),
        ([7, S, 8, 9, S] + [I] * 4 + [E, 1, 2], [(1, 4, 4)]),
        ([S] + [I] * 8 + [E] + [3] * 4, [(2, 4, 4)]),
    ]
