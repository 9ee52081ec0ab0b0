"""Linear modules behind the reference's linear-module protocol, on gfx950 HIP kernels.

Protocol (omniserve/model/qwen2_llm.py:82-83, 120-134; kernels/mixed_precision.py:21-50):
an ``nn.Module`` with ``forward(x[..., K] fp16) -> [..., N] fp16`` installed by
``setattr`` on ``self_attn.qkv_proj/o_proj`` and ``mlp.gate_up_proj/down_proj``.

* ``GPTQLinear``   - GPTQ int4 (AutoGPTQ ``qweight [K/8, N]`` int32, ``scales [K/128, N]``
                     fp16, symmetric uint4b8, ``desc_act=False``) like ``GPTQMarlinLinear``
                     (kernels/marlin_linear.py:83-96); repacked once into this library's
                     own MFMA layout.  Bias is added after the fp16 GEMM output (:59-62).
* ``F16Linear``    - fp16 ``nn.Linear`` replacement using the packed fp16 layout.

Both run the skinny MFMA kernel (omni_w4a16_gemm / omni_f16_gemm), in blocks of at
most 64 activation rows.  ``fuse_silu=True`` (the gate_up projection) interleaves the
gate and up column tiles and emits silu(gate) * up directly: [.., 2I] -> [.., I].
"""

from __future__ import annotations

import math

import torch
from torch import nn

from ._lib import call, lib, ptr, require_cuda, stream

EPI_STORE, EPI_SILU = 0, 1
MAX_SKINNY_M = 64


def _ksplit(K: int, N: int, M: int) -> int:
    """Split-K factor for the skinny kernel: enough workgroups to cover the 256 CUs
    while keeping each wave's weight stream >= ~6 KB and the LDS tile <= 64 KB."""
    KG = K // 128
    mb = (M + 15) // 16
    # LDS: mb*16 rows x (KC + 8) halfs
    max_groups_lds = max(1, ((64 * 1024) // (mb * 16 * 2) - 8) // 128)
    ngroups = max(1, N // 128)
    ks = 1
    while ngroups * ks < 256 and ks * 2 <= KG and KG // (ks * 2) >= 3:
        ks *= 2
    while math.ceil(KG / ks) > max_groups_lds:
        ks += 1
    return min(ks, KG)


class _SkinnyBuffers:
    """Per-module split-K workspace and self-resetting counters (graph-safe)."""

    def __init__(self, N: int, K: int, device):
        self.N, self.K = N, K
        ks_max = K // 128
        self.ws = torch.empty(ks_max * MAX_SKINNY_M * N, device=device, dtype=torch.float32)
        self.counters = torch.zeros(max(1, N // 16), device=device, dtype=torch.int32)


class GPTQLinear(nn.Module):
    """W4A16 GPTQ linear: y = fp16(x . dequant(W)) (+ bias, added after rounding)."""

    def __init__(self, qweight: torch.Tensor, scales: torch.Tensor, bias=None,
                 group_size: int = 128, fuse_silu: bool = False):
        super().__init__()
        if group_size != 128:
            raise ValueError("only group_size=128 is supported")
        K = qweight.shape[0] * 8
        N = qweight.shape[1]
        if scales.shape != (K // group_size, N):
            raise ValueError(f"scales shape {tuple(scales.shape)} != {(K // group_size, N)}")
        dev = qweight.device
        require_cuda(qweight, dtype=torch.int32)
        require_cuda(scales, dtype=torch.float16)
        self.K, self.N = K, N
        self.fuse_silu = fuse_silu
        self.register_buffer("qweight_packed", torch.empty(N // 16, K // 128, 64, 4,
                                                          device=dev, dtype=torch.int32))
        self.register_buffer("scales_packed", torch.empty(N // 16, K // 128, 16,
                                                         device=dev, dtype=torch.float16))
        call("omni_gptq_repack", ptr(qweight), ptr(scales), ptr(self.qweight_packed),
             ptr(self.scales_packed), K, N, int(fuse_silu), stream())
        self.bias = None if bias is None else bias.to(device=dev, dtype=torch.float16).contiguous()
        self._buf = _SkinnyBuffers(N, K, dev)

    @property
    def out_features(self) -> int:
        return self.N // 2 if self.fuse_silu else self.N

    def forward_out(self, x2d: torch.Tensor, out: torch.Tensor, ksplit: int | None = None):
        M = x2d.shape[0]
        if M > MAX_SKINNY_M:
            for s in range(0, M, MAX_SKINNY_M):
                e = min(M, s + MAX_SKINNY_M)
                self.forward_out(x2d[s:e], out[s:e], ksplit)
            return out
        ks = ksplit or _ksplit(self.K, self.N, M)
        call("omni_w4a16_gemm", ptr(x2d), x2d.stride(0), ptr(self.qweight_packed),
             ptr(self.scales_packed), ptr(self.bias), 1, ptr(out), out.stride(0), M, self.N,
             self.K, EPI_SILU if self.fuse_silu else EPI_STORE, ks, 2, ptr(self._buf.ws),
             ptr(self._buf.counters), stream())
        return out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x2d = x.reshape(-1, self.K)
        if not x2d.is_contiguous():
            x2d = x2d.contiguous()
        require_cuda(x2d, dtype=torch.float16)
        out = torch.empty(x2d.shape[0], self.out_features, device=x.device, dtype=torch.float16)
        self.forward_out(x2d, out)
        return out.reshape(*x.shape[:-1], self.out_features)

    def dequantized(self) -> torch.Tensor:
        """W^T [K, N] fp16 as the kernels see it (columns in packed order)."""
        w = torch.empty(self.K, self.N, device=self.qweight_packed.device, dtype=torch.float16)
        call("omni_w4_dequant", ptr(self.qweight_packed), ptr(self.scales_packed), ptr(w),
             self.K, self.N, stream())
        return w


class F16Linear(nn.Module):
    """fp16 linear over the packed MFMA layout: y = fp16(x . W^T + b)."""

    def __init__(self, weight: torch.Tensor, bias=None, fuse_silu: bool = False):
        super().__init__()
        N, K = weight.shape
        dev = weight.device
        require_cuda(weight, dtype=torch.float16)
        self.K, self.N = K, N
        self.fuse_silu = fuse_silu
        self.register_buffer("weight_packed", torch.empty(N // 16, K // 32, 64, 8, device=dev,
                                                         dtype=torch.float16))
        call("omni_f16_pack", ptr(weight.contiguous()), ptr(self.weight_packed), K, N,
             int(fuse_silu), stream())
        self.bias = None if bias is None else bias.to(device=dev, dtype=torch.float16).contiguous()
        self._buf = _SkinnyBuffers(N, K, dev)

    @classmethod
    def from_linear(cls, linear: nn.Linear, fuse_silu: bool = False) -> "F16Linear":
        return cls(linear.weight.data, linear.bias, fuse_silu=fuse_silu)

    @property
    def out_features(self) -> int:
        return self.N // 2 if self.fuse_silu else self.N

    def forward_out(self, x2d: torch.Tensor, out: torch.Tensor, ksplit: int | None = None):
        M = x2d.shape[0]
        if M > MAX_SKINNY_M:
            for s in range(0, M, MAX_SKINNY_M):
                e = min(M, s + MAX_SKINNY_M)
                self.forward_out(x2d[s:e], out[s:e], ksplit)
            return out
        ks = ksplit or _ksplit(self.K, self.N, M)
        call("omni_f16_gemm", ptr(x2d), x2d.stride(0), ptr(self.weight_packed), ptr(self.bias),
             ptr(out), out.stride(0), M, self.N, self.K,
             EPI_SILU if self.fuse_silu else EPI_STORE, ks, 2, ptr(self._buf.ws),
             ptr(self._buf.counters), stream())
        return out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x2d = x.reshape(-1, self.K)
        if not x2d.is_contiguous():
            x2d = x2d.contiguous()
        require_cuda(x2d, dtype=torch.float16)
        out = torch.empty(x2d.shape[0], self.out_features, device=x.device, dtype=torch.float16)
        self.forward_out(x2d, out)
        return out.reshape(*x.shape[:-1], self.out_features)


class LMHeadArgmax(nn.Module):
    """Tied lm_head (qwen2_llm.py:167-168, 190) fused with greedy argmax
    (runners/multimodal.py:307-308): ids = argmax_n fp16(h . E[n]), lowest index on ties.
    The embedding table is stored once, packed; the token gather reads the packed form."""

    def __init__(self, embed: torch.Tensor):
        super().__init__()
        V, H = embed.shape
        dev = embed.device
        require_cuda(embed, dtype=torch.float16)
        self.V, self.H = V, H
        self.register_buffer("table_packed", torch.empty(V // 16, H // 32, 64, 8, device=dev,
                                                        dtype=torch.float16))
        call("omni_f16_pack", ptr(embed.contiguous()), ptr(self.table_packed), H, V, 0, stream())
        grid = lib().omni_lmhead_argmax_grid(V)
        self._cand_val = torch.empty(grid * MAX_SKINNY_M, device=dev, dtype=torch.float32)
        self._cand_idx = torch.empty(grid * MAX_SKINNY_M, device=dev, dtype=torch.int32)
        self._counter = torch.zeros(1, device=dev, dtype=torch.int32)

    def argmax_out(self, h2d: torch.Tensor, ids_out: torch.Tensor, logits_out=None):
        M = h2d.shape[0]
        if M > MAX_SKINNY_M:
            raise ValueError(f"lm_head argmax supports up to {MAX_SKINNY_M} rows per call")
        require_cuda(h2d, dtype=torch.float16)
        require_cuda(ids_out, dtype=torch.int64)
        call("omni_lmhead_argmax", ptr(h2d), h2d.stride(0), ptr(self.table_packed), M, self.V,
             self.H, ptr(logits_out), ptr(ids_out), ptr(self._cand_val), ptr(self._cand_idx),
             ptr(self._counter), stream())
        return ids_out

    def logits(self, h2d: torch.Tensor) -> torch.Tensor:
        """fp16 logits [M, V] (and the argmax computed alongside, discarded)."""
        out = torch.empty(h2d.shape[0], self.V, device=h2d.device, dtype=torch.float16)
        ids = torch.empty(h2d.shape[0], device=h2d.device, dtype=torch.int64)
        for s in range(0, h2d.shape[0], MAX_SKINNY_M):
            e = min(s + MAX_SKINNY_M, h2d.shape[0])
            self.argmax_out(h2d[s:e], ids[s:e], out[s:e])
        return out
