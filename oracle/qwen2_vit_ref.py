"""CPU oracle: an fp32 restatement of omniserve's Qwen2-VL vision tower (ViT + merger).

TEST INFRASTRUCTURE ONLY.  Nothing under ``omniserver_amd/`` imports this module;
only ``tests/`` use it, as the checker of the HIP vision tower.

Follows omniserve/model/qwen2_vit.py (whole file) and kernels/vision_rope.py:19-47;
every function cites the lines it restates.  Tensors are CPU ``float32``; ``f16=True``
rounds to fp16 wherever the reference's fp16 module stores an fp16 tensor (after
every linear, LayerNorm, rotary, attention, residual add and elementwise op), so the
GPU path can be compared tightly.  Weights come as the Hugging Face ``visual.*`` state
dict (fp16 values).

How each part is pinned (tests/test_oracle_vit.py): LayerNorm and GELU against
torch's float64 library routines, QuickGELU against its closed form with the
roundings placed by hand, the rotary against complex multiplication and its
invariants, the patch positions against a per-patch loop of the window order, the
segmented attention against per-image float64 softmax attention and the
block-diagonal mask form; the composition (stage order, residuals, merger) against the
reference's own Qwen2VIT.forward run on the CPU (tests/golden/ref_vit.npz), stage by
stage and end to end.  vLLM's varlen flash attention (the reference's attention core) is
not in this image: the oracle's exact softmax stands in for it, so its rounding inside
the attention stays unpinned.
"""

from __future__ import annotations

import math
from typing import Dict, List, Sequence, Tuple

import torch

from .qwen2_ref import r16


def grids_list(grid_thw) -> List[Tuple[int, int, int]]:
    if isinstance(grid_thw, torch.Tensor):
        grid_thw = grid_thw.tolist()
    return [tuple(int(v) for v in g) for g in grid_thw]


def rot_pos_ids(grid_thw, m: int = 2) -> torch.Tensor:
    """model/qwen2_vit.py:96-105: (h, w) of every patch in merge-window order, per frame."""
    out = []
    for t, h, w in grids_list(grid_thw):
        hp = torch.arange(h).unsqueeze(1).expand(-1, w)
        hp = hp.reshape(h // m, m, w // m, m).permute(0, 2, 1, 3).flatten()
        wp = torch.arange(w).unsqueeze(0).expand(h, -1)
        wp = wp.reshape(h // m, m, w // m, m).permute(0, 2, 1, 3).flatten()
        out.append(torch.stack([hp, wp], dim=-1).repeat(t, 1))
    return torch.cat(out, 0)


def rot_cos_sin(grid_thw, head_dim: int = 80, theta: float = 10000.0, m: int = 2):
    """model/qwen2_vit.py:106-116: fp32 cos / sin [S, head_dim] (emb = cat(rpe, rpe))."""
    pos = rot_pos_ids(grid_thw, m)
    rot = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, rot, 2, dtype=torch.float32) / rot))
    max_grid = max(max(h, w) for _, h, w in grids_list(grid_thw))
    seq = torch.arange(max_grid, dtype=torch.float32)
    freqs = torch.outer(seq, inv_freq)
    rpe = freqs[pos].flatten(1)
    emb = torch.cat((rpe, rpe), dim=-1)
    return emb.cos(), emb.sin()


def cu_seqlens(grid_thw) -> List[int]:
    """model/qwen2_vit.py:124-125."""
    cu = [0]
    for t, h, w in grids_list(grid_thw):
        for _ in range(t):
            cu.append(cu[-1] + h * w)
    return cu


def layer_norm(x, w, b, eps=1e-6, f16=True):
    """nn.LayerNorm(eps=1e-6) (model/qwen2_vit.py:39-40, 87): fp32 mean / biased variance."""
    mean = x.mean(-1, keepdim=True)
    var = ((x - mean) ** 2).mean(-1, keepdim=True)
    return r16((x - mean) * torch.rsqrt(var + eps) * w + b, f16)


def linear(x, w, b=None, f16=True):
    """fp16 nn.Linear: fp32 accumulation, bias added before the single rounding."""
    y = x @ w.t()
    if b is not None:
        y = y + b
    return r16(y, f16)


def quick_gelu(x, f16=True):
    """model/qwen2_vit.py:18-19 on an fp16 tensor: 1.702 x, sigmoid, product, each rounded."""
    t = r16(x * 1.702, f16)
    s = r16(torch.sigmoid(t), f16)
    return r16(x * s, f16)


def gelu(x, f16=True):
    """F.gelu (exact erf form), model/qwen2_vit.py:128."""
    return r16(0.5 * x * (1.0 + torch.erf(x / math.sqrt(2.0))), f16)


def vision_rope(q, k, cos, sin, f16=True):
    """kernels/vision_rope.py:19-36 (= apply_rotary_vision, model/qwen2_vit.py:27-33):
    q, k [S, nh, hd]; cos, sin [S, hd] fp32 with equal halves; fp32 math, fp16 out."""
    half = q.shape[-1] // 2
    c = cos[:, None, :half]
    s = sin[:, None, :half]

    def one(x):
        x1, x2 = x[..., :half], x[..., half:]
        return r16(torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1), f16)
    return one(q), one(k)


def seg_attention(q, k, v, cu: Sequence[int], scale: float, f16=True):
    """flash_attn_varlen_func(causal=False) of model/qwen2_vit.py:58-63: exact softmax
    attention within each segment, fp32.  q, k, v [S, nh, hd] -> [S, nh, hd]."""
    out = torch.empty_like(q)
    for s0, s1 in zip(cu[:-1], cu[1:]):
        qs, ks, vs = (t[s0:s1].transpose(0, 1) for t in (q, k, v))     # [nh, L, hd]
        p = torch.softmax(qs @ ks.transpose(1, 2) * scale, dim=-1)
        out[s0:s1] = (p @ vs).transpose(0, 1)
    return r16(out, f16)


def vit_block(x, sd: Dict[str, torch.Tensor], p: str, cos, sin, cu, n_heads=16, f16=True):
    """VisionBlock.forward (model/qwen2_vit.py:66-69) with attn (:48-64)."""
    g = lambda key: sd[p + key].float()
    S, D = x.shape
    hd = D // n_heads
    h = layer_norm(x, g("norm1.weight"), g("norm1.bias"), f16=f16)
    qkv = linear(h, g("attn.qkv.weight"), g("attn.qkv.bias"), f16).view(S, 3, n_heads, hd)
    q, k = vision_rope(qkv[:, 0], qkv[:, 1], cos, sin, f16)
    o = seg_attention(q, k, qkv[:, 2], cu, hd ** -0.5, f16)
    x = r16(x + linear(o.reshape(S, D), g("attn.proj.weight"), g("attn.proj.bias"), f16), f16)
    h = layer_norm(x, g("norm2.weight"), g("norm2.bias"), f16=f16)
    f = quick_gelu(linear(h, g("mlp.fc1.weight"), g("mlp.fc1.bias"), f16), f16)
    return r16(x + linear(f, g("mlp.fc2.weight"), g("mlp.fc2.bias"), f16), f16)


def vit_forward(pixel_values, grid_thw, sd: Dict[str, torch.Tensor], n_heads=16, m=2,
                theta=10000.0, f16=True, depth=None):
    """Qwen2VIT.forward (model/qwen2_vit.py:118-129): pixel patches [S, patch_dim] ->
    merged rows [S / m^2, out_hidden]."""
    pe = sd["visual.patch_embed.proj.weight"].float()
    D = pe.shape[0]
    x = linear(pixel_values.float(), pe.reshape(D, -1), None, f16)
    cos, sin = rot_cos_sin(grid_thw, D // n_heads, theta, m)
    cu = cu_seqlens(grid_thw)
    nb = 0
    while f"visual.blocks.{nb}.norm1.weight" in sd:
        nb += 1
    for i in range(nb if depth is None else depth):
        x = vit_block(x, sd, f"visual.blocks.{i}.", cos, sin, cu, n_heads, f16)
    g = lambda key: sd["visual." + key].float()
    h = layer_norm(x, g("merger.ln_q.weight"), g("merger.ln_q.bias"), f16=f16).view(-1, D * m * m)
    h = gelu(linear(h, g("merger.mlp.0.weight"), g("merger.mlp.0.bias"), f16), f16)
    return linear(h, g("merger.mlp.2.weight"), g("merger.mlp.2.bias"), f16)
