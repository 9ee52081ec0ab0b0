"""Qwen2-VL vision tower on the gfx950 kernels: flattened pixel patches -> merged
vision rows (the rows the decoder splices in at the image tokens).

Mirrors omniserve/model/qwen2_vit.py: ``Qwen2VIT`` (:72-129, same constructor
arguments and ``forward(pixel_values, grid_thw)``), ``VisionBlock`` (:36-69) and
``load_vit_from_state_dict`` (:132-147, Hugging Face ``visual.*`` key names).  Per
block, 8 launches: LayerNorm -> qkv GEMM (+ bias) -> 2-D rotary on q / k in place ->
segmented non-causal attention (head_dim 80) -> proj GEMM (+ bias + residual, in place)
-> LayerNorm -> fc1 GEMM (+ bias + QuickGELU) -> fc2 GEMM (+ bias + residual).  Merger:
LayerNorm -> [S/4, 5120] view -> fc1 (+ bias + GELU) -> fc2 (+ bias).

Numerics follow the reference's fp16 module: fp16 storage between ops, fp32 inside
every kernel, the rotary frequencies in fp32 (inv_freq computed on the CPU in fp32, as
:107-111 requires), bias added before each linear's single rounding.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Sequence, Tuple

import torch

from ._lib import call, lib, ptr, require_cuda, stream
from .hostio import to_device

EPI_STORE, EPI_QGELU, EPI_GELU, EPI_RESID = 0, 4, 5, 6
EPI_PARTIAL = 2
_QT = 64     # queries per attention workgroup (the kernel's tile)


@dataclass
class VisionConfig:
    """Qwen2VIT constructor defaults (model/qwen2_vit.py:73-75)."""
    embed_dim: int = 1280
    depth: int = 32
    n_heads: int = 16
    in_chans: int = 3
    patch_size: int = 14
    temporal_patch_size: int = 2
    spatial_merge_size: int = 2
    mlp_ratio: int = 4
    out_hidden: int = 1536
    rope_theta: float = 10000.0
    eps: float = 1e-6

    @property
    def patch_dim(self) -> int:
        return self.in_chans * self.temporal_patch_size * self.patch_size ** 2

    @property
    def head_dim(self) -> int:
        return self.embed_dim // self.n_heads

    @property
    def mlp_dim(self) -> int:
        return self.embed_dim * self.mlp_ratio

    @property
    def merged_dim(self) -> int:
        return self.embed_dim * self.spatial_merge_size ** 2


# --------------------------------------------------------------------------- host tables
def _grids(grid_thw) -> List[Tuple[int, int, int]]:
    if isinstance(grid_thw, torch.Tensor):
        grid_thw = grid_thw.tolist()
    out = [tuple(int(v) for v in g) for g in grid_thw]
    for t, h, w in out:
        if t <= 0 or h <= 0 or w <= 0:
            raise ValueError(f"grid {(t, h, w)} must be positive")
    return out


def rot_pos_ids(grid_thw, merge: int) -> torch.Tensor:
    """int32 [S, 2] (h, w) position of every patch, patches in merge-window order and
    repeated over t (model/qwen2_vit.py:96-105)."""
    rows = []
    for t, h, w in _grids(grid_thw):
        if h % merge or w % merge:
            raise ValueError(f"grid {(t, h, w)}: h and w must be multiples of {merge}")
        hp = torch.arange(h).view(h // merge, merge, 1, 1).expand(-1, -1, w // merge, merge)
        wp = torch.arange(w).view(1, 1, w // merge, merge).expand(h // merge, merge, -1, -1)
        hp = hp.permute(0, 2, 1, 3).reshape(-1)
        wp = wp.permute(0, 2, 1, 3).reshape(-1)
        rows.append(torch.stack([hp, wp], -1).repeat(t, 1))
    return torch.cat(rows, 0).to(torch.int32)


def vision_inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """fp32 [head_dim / 4] rotary inverse frequencies, computed on the CPU in fp32 exactly
    as model/qwen2_vit.py:110-111 (rot_dim = head_dim / 2)."""
    rot = head_dim // 2
    return 1.0 / (theta ** (torch.arange(0, rot, 2, dtype=torch.float32) / rot))


def cu_seqlens(grid_thw) -> torch.Tensor:
    """int32 [n_frames + 1] patch offsets of every frame (model/qwen2_vit.py:124-125)."""
    lens = [h * w for t, h, w in _grids(grid_thw) for _ in range(t)]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    return torch.tensor(cu, dtype=torch.int32)


def query_tiles(cu: torch.Tensor) -> torch.Tensor:
    """int32 [ntiles, 2] = (first query, segment): every segment in steps of 64 queries."""
    c = cu.tolist()
    rows = [(q, s) for s in range(len(c) - 1) for q in range(c[s], c[s + 1], _QT)]
    return torch.tensor(rows, dtype=torch.int32).view(-1, 2)


# --------------------------------------------------------------------------- ops
def layer_norm_out(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, eps: float,
                   out: torch.Tensor) -> torch.Tensor:
    """nn.LayerNorm over the last dim (fp32 math, biased variance), fp16 in / out."""
    require_cuda(x, w, b, out, dtype=torch.float16)
    M, N = x.shape
    call("omni_layernorm", ptr(x), x.stride(0), ptr(w), ptr(b), M, N, float(eps), ptr(out),
         out.stride(0), stream())
    return out


def layer_norm_partials_out(parts: torch.Tensor, nparts: int, lin_bias: torch.Tensor | None,
                            x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, eps: float,
                            out: torch.Tensor) -> torch.Tensor:
    """x = fp16(x + fp16(sum of the nparts fp32 slices [S, M, N] + lin_bias)) in place (the
    split-K linear's residual add, as its finish launch would write it), then out =
    LayerNorm(x) as layer_norm_out."""
    require_cuda(parts, dtype=torch.float32)
    require_cuda(x, w, b, out, lin_bias, dtype=torch.float16)
    M, N = x.shape
    if parts.numel() < nparts * M * N:
        raise ValueError("partial buffer smaller than nparts x M x N")
    call("omni_layernorm_partials", ptr(parts), nparts, ptr(lin_bias), ptr(x), x.stride(0),
         ptr(x), x.stride(0), ptr(w), ptr(b), M, N, float(eps), ptr(out), out.stride(0),
         stream())
    return out


def vision_rope_(qkv: torch.Tensor, n_heads: int, head_dim: int, pos_hw: torch.Tensor,
                 inv_freq: torch.Tensor) -> torch.Tensor:
    """In-place 2-D rotary of the q and k heads of qkv rows (kernels/vision_rope.py:39-47)."""
    require_cuda(qkv, dtype=torch.float16)
    require_cuda(pos_hw, dtype=torch.int32)
    require_cuda(inv_freq, dtype=torch.float32)
    call("omni_vision_rope", ptr(qkv), qkv.stride(0), qkv.shape[0], n_heads, head_dim, ptr(pos_hw),
         ptr(inv_freq), stream())
    return qkv


def vit_attention_out(qkv: torch.Tensor, n_heads: int, head_dim: int, cu: torch.Tensor,
                      tiles: torch.Tensor, scale: float, out: torch.Tensor) -> torch.Tensor:
    """Non-causal attention within the segments cu (int32, device) of the rotated qkv rows."""
    require_cuda(qkv, out, dtype=torch.float16)
    require_cuda(cu, tiles, dtype=torch.int32)
    call("omni_vit_attention", ptr(qkv), qkv.stride(0), qkv.shape[0], n_heads, head_dim, ptr(cu),
         ptr(tiles), tiles.shape[0], ptr(out), out.stride(0), float(scale), stream())
    return out


class VisionLinear:
    """fp16 nn.Linear (weight [N, K], optional bias [N]) on one of two GEMMs, its weight
    packed once (omni_f16_pack) into the MFMA operand layout: ``pipe``
    (omni_f16_gemm_pipe_packed: a multi-stage LDS pipeline, N % 128 == 0, K % 128 == 0,
    K >= 256 - every linear of the blocks and the merger; it can also leave the K slices'
    fp32 sums for the next kernel, ``out_partial``) or ``tiled`` (omni_f16_gemm_tiled, K
    zero-padded to whole 128-column groups - the patch embedding's K = 1176)."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None, device,
                 path: str | None = None):
        N, K = weight.shape
        if path is None:
            path = "pipe" if N % 128 == 0 and K % 128 == 0 and K >= 256 else "tiled"
        if path not in ("pipe", "tiled"):
            raise ValueError(f"unknown GEMM path {path!r}")
        self.path = path
        self._ws = None
        self._plans: Dict[tuple, int] = {}
        w = weight.to(device=device, dtype=torch.float16).contiguous()
        self.bias = None if bias is None else bias.to(device=device, dtype=torch.float16).contiguous()
        self.N, self.K = N, K
        Kp = -(-K // 128) * 128
        if Kp != K:
            w = torch.nn.functional.pad(w, (0, Kp - K)).contiguous()
        self.w = torch.empty_like(w)
        call("omni_f16_pack", ptr(w), ptr(self.w), Kp, N, 0, stream())
        self.Kp = Kp

    def slices(self, M: int, epilogue: int = EPI_STORE, tile_rows: int = 0,
               ksplit: int = 0) -> int:
        """K slices the pipe GEMM runs for M rows (the library's plan for ksplit 0, which the
        call then makes itself; ksplit > 0 fixes them)."""
        if ksplit:
            return ksplit
        key = (M, epilogue, tile_rows)
        if key not in self._plans:
            r, c, k = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
            call("omni_packed_gemm_pipe_plan", M, self.N, self.K, 1, epilogue,
                 int(self.bias is not None and epilogue != EPI_PARTIAL), tile_rows, 0,
                 ctypes.byref(r), ctypes.byref(c), ctypes.byref(k))
            self._plans[key] = k.value
        return self._plans[key]

    def _workspace(self, need: int, device) -> torch.Tensor:
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, device=device, dtype=torch.float32)
        return self._ws

    def out(self, x: torch.Tensor, out: torch.Tensor, epilogue: int = EPI_STORE,
            res: torch.Tensor | None = None, tile_rows: int = 0,
            ksplit: int = 0) -> torch.Tensor:
        require_cuda(x, out, res, dtype=torch.float16, contiguous=False)
        if x.shape[1] != self.K:
            raise ValueError(f"input has {x.shape[1]} columns, the linear takes {self.K}")
        if x.stride(1) != 1 or out.stride(1) != 1 or (res is not None and res.stride(1) != 1):
            raise ValueError("rows must be contiguous")
        if epilogue == EPI_PARTIAL:
            raise ValueError("the partial-sum form is out_partial")
        ldr = 0 if res is None else res.stride(0)
        if self.path == "pipe":
            M = x.shape[0]
            ks = self.slices(M, epilogue, tile_rows, ksplit)
            ws = self._workspace(ks * M * self.N, x.device) if ks > 1 else None
            call("omni_f16_gemm_pipe_packed", ptr(x), x.stride(0), ptr(self.w), ptr(self.bias),
                 ptr(res), ldr, ptr(out), out.stride(0), M, self.N, self.K, epilogue, tile_rows,
                 ksplit, ptr(ws), stream())
        else:
            call("omni_f16_gemm_tiled", ptr(x), x.stride(0), self.K, ptr(self.w), ptr(self.bias),
                 ptr(res), ldr, ptr(out), out.stride(0), x.shape[0], self.N, self.Kp, epilogue,
                 stream())
        return out

    def out_partial(self, x: torch.Tensor, parts: torch.Tensor | None = None) -> Tuple[torch.Tensor, int]:
        """The K slices' fp32 sums x . W^T (no bias) into parts [S, M, N] (the linear's own
        workspace when None), for layer_norm_partials_out to finish; returns (parts, S)."""
        if self.path != "pipe":
            raise ValueError("the partial-sum form runs on the pipe GEMM")
        require_cuda(x, dtype=torch.float16, contiguous=False)
        if x.shape[1] != self.K or x.stride(1) != 1:
            raise ValueError(f"input must be rows of {self.K} contiguous columns")
        M = x.shape[0]
        S = self.slices(M, EPI_PARTIAL)
        if parts is None:
            parts = self._workspace(S * M * self.N, x.device)
        elif parts.numel() < S * M * self.N or parts.dtype != torch.float32:
            raise ValueError("partial buffer too small or not fp32")
        call("omni_f16_gemm_pipe_packed", ptr(x), x.stride(0), ptr(self.w), None, None, 0, None, 0,
             M, self.N, self.K, EPI_PARTIAL, 0, 0, ptr(parts), stream())
        return parts, S


class _Block:
    def __init__(self, sd: Dict[str, torch.Tensor], p: str, device):
        f16 = lambda k: sd[p + k].to(device=device, dtype=torch.float16).contiguous()
        self.n1w, self.n1b = f16("norm1.weight"), f16("norm1.bias")
        self.n2w, self.n2b = f16("norm2.weight"), f16("norm2.bias")
        lin = lambda k: VisionLinear(sd[p + k + ".weight"], sd[p + k + ".bias"], device)
        self.qkv, self.proj = lin("attn.qkv"), lin("attn.proj")
        self.fc1, self.fc2 = lin("mlp.fc1"), lin("mlp.fc2")


class Qwen2VIT:
    """The vision tower (model/qwen2_vit.py:72-129) on the HIP kernels."""

    def __init__(self, embed_dim=1280, depth=32, n_heads=16, in_chans=3, patch_size=14,
                 temporal_patch_size=2, spatial_merge_size=2, mlp_ratio=4, out_hidden=1536,
                 rope_theta=10000.0, device="cuda"):
        self.cfg = VisionConfig(embed_dim, depth, n_heads, in_chans, patch_size,
                                temporal_patch_size, spatial_merge_size, mlp_ratio, out_hidden,
                                rope_theta)
        if self.cfg.head_dim != 80:
            raise ValueError("the vision attention kernel is built for head_dim 80")
        self.device = torch.device(device)
        self.blocks: List[_Block] = []
        self.patch_embed = None
        self.inv_freq = vision_inv_freq(self.cfg.head_dim, rope_theta).to(self.device)

    @property
    def loaded(self) -> bool:
        return self.patch_embed is not None

    def forward(self, pixel_values: torch.Tensor, grid_thw) -> torch.Tensor:
        """pixel_values fp16 [S, patch_dim] (patches in merge-window order, as the image
        processor emits them), grid_thw [(t, h, w), ...] -> fp16 [S / merge^2, out_hidden]."""
        if not self.loaded:
            raise RuntimeError("vision tower weights not loaded (load_vit_from_state_dict)")
        cfg, dev = self.cfg, self.device
        grids = _grids(grid_thw)
        S = sum(t * h * w for t, h, w in grids)
        if pixel_values.dim() != 2 or pixel_values.shape != (S, cfg.patch_dim):
            raise ValueError(f"pixel_values must be [{S}, {cfg.patch_dim}] for grids {grids}")
        pv = pixel_values.to(device=dev, dtype=torch.float16).contiguous()
        m2 = cfg.spatial_merge_size ** 2
        pos = to_device(rot_pos_ids(grids, cfg.spatial_merge_size), torch.int32, dev)
        cu_h = cu_seqlens(grids)
        tiles = to_device(query_tiles(cu_h), torch.int32, dev)
        cu = to_device(cu_h, torch.int32, dev)
        D, nh, hd = cfg.embed_dim, cfg.n_heads, cfg.head_dim
        mk = lambda *s: torch.empty(*s, device=dev, dtype=torch.float16)
        x, h, att = mk(S, D), mk(S, D), mk(S, D)
        qkv, f = mk(S, 3 * D), mk(S, cfg.mlp_dim)
        self.patch_embed.out(pv, x)
        scale = hd ** -0.5
        # proj and fc2 leave their K slices' fp32 sums; the LayerNorm that follows each adds
        # them, the bias and the residual first (one launch where a finish launch and the
        # norm were two), with the same roundings
        np_ = max(max(b.proj.slices(S, EPI_PARTIAL), b.fc2.slices(S, EPI_PARTIAL))
                  for b in self.blocks)
        parts = torch.empty(np_ * S * D, device=dev, dtype=torch.float32)
        pend = None                      # the previous block's fc2 slices
        for blk in self.blocks:
            if pend is None:
                layer_norm_out(x, blk.n1w, blk.n1b, cfg.eps, h)
            else:
                layer_norm_partials_out(parts, pend[0], pend[1], x, blk.n1w, blk.n1b, cfg.eps, h)
            blk.qkv.out(h, qkv)
            vision_rope_(qkv, nh, hd, pos, self.inv_freq)
            vit_attention_out(qkv, nh, hd, cu, tiles, scale, att)
            _, sp = blk.proj.out_partial(att, parts)
            layer_norm_partials_out(parts, sp, blk.proj.bias, x, blk.n2w, blk.n2b, cfg.eps, h)
            blk.fc1.out(h, f, EPI_QGELU)
            _, sf = blk.fc2.out_partial(f, parts)
            pend = (sf, blk.fc2.bias)
        if pend is None:
            layer_norm_out(x, self.lnq_w, self.lnq_b, cfg.eps, h)
        else:
            layer_norm_partials_out(parts, pend[0], pend[1], x, self.lnq_w, self.lnq_b, cfg.eps, h)
        hm = h.view(S // m2, cfg.merged_dim)
        m1 = mk(S // m2, cfg.merged_dim)
        self.merger_fc1.out(hm, m1, EPI_GELU)
        out = mk(S // m2, cfg.out_hidden)
        return self.merger_fc2.out(m1, out)

    __call__ = forward


def load_vit_from_state_dict(vit: Qwen2VIT, sd: Dict[str, torch.Tensor]) -> Qwen2VIT:
    """Weights under the Hugging Face ``visual.*`` keys (model/qwen2_vit.py:132-147): the
    Conv3d patch kernel flattened to [embed_dim, patch_dim], every linear packed."""
    cfg, dev = vit.cfg, vit.device
    g = lambda k: sd["visual." + k]
    depth = 0
    while f"visual.blocks.{depth}.norm1.weight" in sd:
        depth += 1
    if depth != cfg.depth:
        raise ValueError(f"state dict holds {depth} vision blocks, the tower has {cfg.depth}")
    pe = g("patch_embed.proj.weight").reshape(cfg.embed_dim, -1)
    if pe.shape[1] != cfg.patch_dim:
        raise ValueError(f"patch kernel has {pe.shape[1]} inputs, expected {cfg.patch_dim}")
    vit.patch_embed = VisionLinear(pe, None, dev)
    vit.blocks = [_Block(sd, f"visual.blocks.{i}.", dev) for i in range(depth)]
    f16 = lambda k: g(k).to(device=dev, dtype=torch.float16).contiguous()
    vit.lnq_w, vit.lnq_b = f16("merger.ln_q.weight"), f16("merger.ln_q.bias")
    vit.merger_fc1 = VisionLinear(g("merger.mlp.0.weight"), g("merger.mlp.0.bias"), dev)
    vit.merger_fc2 = VisionLinear(g("merger.mlp.2.weight"), g("merger.mlp.2.bias"), dev)
    return vit
