"""Linear modules behind the reference's linear-module protocol, on gfx950 HIP kernels.

Protocol (omniserve/model/qwen2_llm.py:82-83, 120-134; kernels/mixed_precision.py:21-50):
an ``nn.Module`` with ``forward(x[..., K] fp16) -> [..., N] fp16`` installed by
``setattr`` on ``self_attn.qkv_proj/o_proj`` and ``mlp.gate_up_proj/down_proj``.

* ``GPTQLinear``   - GPTQ int4 (AutoGPTQ ``qweight [K/8, N]`` int32, ``scales [K/128, N]``
                     fp16, symmetric uint4b8, ``desc_act=False``) like ``GPTQMarlinLinear``
                     (kernels/marlin_linear.py:83-96); repacked once into this library's
                     own MFMA layout.  Bias is added after the fp16 GEMM output (:59-62).
* ``F16Linear``    - fp16 ``nn.Linear`` replacement using the packed fp16 layout.
* ``LMHeadArgmax`` - tied lm_head + greedy argmax.

All run omni_w4a16_gemm / omni_f16_gemm: the skinny weight-streaming kernel for up to
64 activation rows (decode), the pipelined MFMA GEMM beyond (prefill; GPTQ at 2048 rows and
more unpacks its weights to fp16 first).  ``fuse_silu=True`` (the gate_up projection) interleaves the gate
and up column tiles and emits silu(gate) * up directly: [.., 2I] -> [.., I].
``forward_partial`` writes fp32 split-K partial sums instead of fp16 output, for a
consumer kernel (the next add+RMSNorm) that adds them in slice order.

Launch plans (workgroup shape preset, K split) come from ``PLANS`` keyed by the
weight format and shape; the decode step of the 2B decoder uses the entries below.
"""

from __future__ import annotations

import ctypes
from typing import Dict, Tuple

import torch
from torch import nn

from ._lib import call, lib, ptr, require_cuda, stream

EPI_STORE, EPI_SILU, EPI_PARTIAL = 0, 1, 2
MAX_SKINNY_M = 64

# (weight format, K, N) -> (store preset, partial preset, partial ksplit); measured on
# MI355X at M = 32 (graph-replayed launches; the fp16 entries also at M = 1 and 16).  Presets (tiles per wave, column waves,
# in-group K split): 0 = (1, 8, 2), 1 = (1, 8, 1), 2 = (1, 4, 4), 3 = (2, 4, 2);
# SiLU: 0 = (2, 4, 4), 1 = (2, 8, 1), 2 = (2, 4, 2), 3 = (2, 2, 4), 4 = (2, 3, 4), 5 = (2, 2, 8);
# 6-9 = (2, 3, 4), (2, 2, 4), (2, 4, 4), (2, 8, 1) with x staged in LDS before the weight
# stream is requested (the SiLU projection stages all of K, which otherwise queues behind
# the grid's weight loads).
PLANS: Dict[Tuple[str, int, int], Tuple[int, int, int]] = {
    ("int4", 1536, 2048): (2, 1, 7),
    ("int4", 1536, 1536): (2, 1, 12),     # o_proj: one head per K slice (attention merge)
    ("int4", 8960, 1536): (2, 1, 14),
    ("int4", 1536, 17920): (6, 2, 1),     # SiLU-fused gate_up: preset 6 = (2, 3, 4), x first
    # fp16 (two weight groups in flight per tile): swept at B = 1, 16 and 32
    ("fp16", 1536, 2048): (2, 1, 7),
    ("fp16", 1536, 1536): (2, 1, 12),
    ("fp16", 8960, 1536): (2, 3, 20),     # down: preset 3 = (2, 4, 2) x 20 K slices
    ("fp16", 1536, 17920): (4, 2, 1),     # gate_up: SiLU preset 4 = (2, 3, 4)
}


def _plan(fmt: str, K: int, N: int) -> Tuple[int, int, int]:
    if (fmt, K, N) in PLANS:
        return PLANS[(fmt, K, N)]
    ks = max(1, min(K // 128, (K // 128 + 6) // 7))
    return (2, 1, ks)


def rtn_int4(weight: torch.Tensor, group_size: int = 128):
    """Round-to-nearest symmetric int4 (uint4b8) of an fp16 weight [N, K], the quantiser
    the reference's MarlinInt4Linear calls (vLLM's quantize_weights for uint4b8, group
    ``group_size`` along K): per group and output column, in fp16,
    s = max(|max_k w| / 7, |min_k w| / 8), q = clamp(round(w / s), -8, 7) + 8.  Returns
    the AutoGPTQ tensors (qweight int32 [K/8, N], k % 8 at bits 4 (k % 8); scales fp16
    [K/group, N]) that GPTQLinear takes; the kernels then compute with fp16((q - 8) s).
    Load-time tensor work on the weight's device."""
    N, K = weight.shape
    if K % group_size or K % 8:
        raise ValueError(f"K = {K} is not a multiple of the group size {group_size}")
    w = weight.t().contiguous().to(torch.float16).view(K // group_size, group_size, N)
    mx = w.amax(1, keepdim=True)
    mn = w.amin(1, keepdim=True)
    s = torch.maximum((mx / 7.0).abs(), (mn / -8.0).abs())
    # an all-zero group has s = 0: its codes are 8 (value 0) rather than 0/0
    q = torch.round(w / torch.where(s == 0, torch.ones_like(s), s)).to(torch.int32)
    q = torch.clamp(q, -8, 7) + 8                                         # [K/g, g, N]
    q = q.view(K // 8, 8, N)
    shifts = (torch.arange(8, device=q.device, dtype=torch.int32) * 4).view(1, 8, 1)
    qweight = (q << shifts).sum(1, dtype=torch.int64).to(torch.int64)
    qweight = torch.where(qweight >= 2 ** 31, qweight - 2 ** 32, qweight).to(torch.int32)
    return qweight.contiguous(), s.view(K // group_size, N).contiguous()


_UNPACK: Dict[torch.device, torch.Tensor] = {}


def _unpack_scratch(device: torch.device, halfs: int) -> torch.Tensor:
    """The device's fp16 scratch for unpacked int4 weights (grown to the largest linear,
    kept for the process; used by one linear at a time, in stream order)."""
    buf = _UNPACK.get(device)
    if buf is None or buf.numel() < halfs:
        buf = torch.empty(halfs, device=device, dtype=torch.float16)
        _UNPACK[device] = buf
    return buf


class _Skinny(nn.Module):
    """Shared launch logic of the packed-weight linears."""

    fmt = "fp16"
    FILL_SLICES = False     # tile_ksplit's slice rule for the fp16 linears

    def _init_plan(self):
        self.store_preset, self.partial_preset, self.partial_ksplit = _plan(self.fmt, self.K, self.N)

    @property
    def out_features(self) -> int:
        return self.N // 2 if self.fuse_silu else self.N

    def partial_slices(self, ksplit: int | None = None) -> int:
        return lib().omni_gemm_slices(self.K, ksplit or self.partial_ksplit)

    def _call(self, x2d, out, partial, epilogue, ksplit, preset):
        raise NotImplementedError

    def tile_ksplit(self, M: int) -> int:
        """K split of the tiled GEMM (more than MAX_SKINNY_M rows, STORE epilogue): when its
        128 x 128 tiles would leave over half of the 256 CUs idle (e.g. a 256-token prompt's
        down projection: 24 tiles over K = 8960), the K groups are dealt to slices summed by
        a finish launch (or by the next kernel, forward_partial).  fp16 linears (FILL_SLICES)
        take as many slices as keep the tiles in one round of the CUs, each at least 2 groups
        (the pipeline's 4 stages of 64): graph-timed at M = 256, qkv 11.3 -> 9.9 us (6 slices
        against 3), o 11.4 -> 9.7 (6), down 19.2 -> 17.5 (10 against 8).  GPTQ linears keep
        up to 8 slices of at least 4 groups (their finished prefill form on the fp16
        expansion plans its own slices, omni_f16_gemm_pipe_splits, and the partial form must
        sum the same ones)."""
        if self.fuse_silu or M <= MAX_SKINNY_M:
            return 1
        tiles = -(-M // 128) * -(-self.N // 128)
        KG = self.K // 128
        if tiles >= 128 or KG < 8:
            return 1
        if self.FILL_SLICES:
            return max(1, min(KG // 2, 256 // tiles))
        return max(1, min(8, KG // 4, 256 // tiles))

    def forward_out(self, x2d: torch.Tensor, out: torch.Tensor, preset: int | None = None,
                    ksplit: int | None = None):
        """fp16 output (SiLU-fused for gate_up) into out; any number of rows (more than
        MAX_SKINNY_M rows run the library's tiled MFMA GEMM, ``preset`` then unused, split
        along K as tile_ksplit says unless ``ksplit`` is given)."""
        epi = EPI_SILU if self.fuse_silu else EPI_STORE
        M = x2d.shape[0]
        ks = self.tile_ksplit(M) if ksplit is None else ksplit
        if M > MAX_SKINNY_M and epi == EPI_STORE and ks > 1:
            ws = torch.empty(self.partial_slices(ks) * M * self.N, device=x2d.device,
                             dtype=torch.float32)
            self._call(x2d, out, ws, epi, ks, 0)
            return out
        self._call(x2d, out, None, epi, 1, self.store_preset if preset is None else preset)
        return out

    def forward_partial(self, x2d: torch.Tensor, partial: torch.Tensor,
                        ksplit: int | None = None, preset: int | None = None) -> int:
        """fp32 split-K partial sums [S][M][N] (no bias) into partial; returns S.  More than
        MAX_SKINNY_M rows run the pipelined GEMM's partial form (S = ksplit, default
        tile_ksplit(M); N % 128 == 0)."""
        if self.fuse_silu:
            raise ValueError("the SiLU-fused projection has no partial form")
        M = x2d.shape[0]
        if M > MAX_SKINNY_M:
            # the slice count forward_out's split form uses (omni_gemm_slices: slices of
            # whole 128-groups), so that the sums agree with it
            KG = self.K // 128
            ks = min(ksplit or self.tile_ksplit(M), KG)
            kc = -(-KG // ks)
            ks = -(-KG // kc)
            if partial.numel() < ks * M * self.N or partial.dtype != torch.float32:
                raise ValueError("partial buffer too small or not fp32")
            if self.N % 128 or x2d.stride(0) % 8:
                raise ValueError("the prefill partial form takes N % 128 == 0, ldx % 8 == 0")
            self._call_pipe_partial(x2d, partial, ks)
            return ks
        ks = ksplit or self.partial_ksplit
        S = self.partial_slices(ks)
        if partial.numel() < S * M * self.N or partial.dtype != torch.float32:
            raise ValueError("partial buffer too small or not fp32")
        self._call(x2d, None, partial, EPI_PARTIAL, ks,
                   self.partial_preset if preset is None else preset)
        return S

    def _prefill_fmt(self, M: int) -> int:
        """Weight format the tiled GEMM runs on at M rows: 1 packed fp16, 0 packed int4."""
        return 1

    def partial_plan(self, M: int) -> int:
        """K slices forward_partial_planned writes at M rows (more than MAX_SKINNY_M): the
        tiled GEMM's own choice for fp32 partial output, which may be the persistent 256-row
        tiles in several slices (the 2B decoder's down projection at M = 4096: 256 x 192 tiles
        in 2 slices, one item per CU)."""
        if M <= MAX_SKINNY_M or self.fuse_silu or self.N % 128 or self.K % 128:
            return 1
        key = (M, self._prefill_fmt(M))
        plans = self.__dict__.setdefault("_partial_plans", {})
        if key not in plans:
            r, c, k = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
            call("omni_packed_gemm_pipe_plan", M, self.N, self.K, key[1], EPI_PARTIAL, 0, 0, 0,
                 ctypes.byref(r), ctypes.byref(c), ctypes.byref(k))
            plans[key] = k.value
        return plans[key]

    def forward_partial_planned(self, x2d: torch.Tensor, partial: torch.Tensor) -> int:
        """fp32 partial sums [S][M][N] (no bias) into partial with S = partial_plan(M) K
        slices of whole 128-groups; returns S."""
        M = x2d.shape[0]
        if self.fuse_silu or M <= MAX_SKINNY_M:
            raise ValueError("the planned partial form takes more than MAX_SKINNY_M rows and "
                             "no SiLU-fused projection")
        if self.N % 128 or self.K % 128 or x2d.stride(0) % 8:
            raise ValueError("the planned partial form takes N, K % 128 == 0, ldx % 8 == 0")
        S = self.partial_plan(M)
        if partial.numel() < S * M * self.N or partial.dtype != torch.float32:
            raise ValueError("partial buffer too small or not fp32")
        self._call_pipe_partial(x2d, partial, 0)
        return S

    def forward_partial_attn(self, states: torch.Tensor, splits: int, n_kv: int, group: int,
                             M: int, partial: torch.Tensor, ksplit: int | None = None,
                             preset: int | None = None) -> int:
        """forward_partial with x = the merge of the decode attention's split states
        [M][n_kv][splits][group][132] (omni_decode_attention_fused, merge = 0)."""
        if self.fuse_silu:
            raise ValueError("the SiLU-fused projection has no partial form")
        if M > MAX_SKINNY_M:
            raise ValueError(f"partial sums support up to {MAX_SKINNY_M} rows")
        ks = ksplit or self.partial_ksplit
        S = self.partial_slices(ks)
        if partial.numel() < S * M * self.N or partial.dtype != torch.float32:
            raise ValueError("partial buffer too small or not fp32")
        if states.dtype != torch.float32 or states.numel() < M * n_kv * splits * group * 132:
            raise ValueError("attention state buffer too small or not fp32")
        self._call_attn(states, splits, n_kv, group, M, partial, EPI_PARTIAL, ks,
                        self.partial_preset if preset is None else preset)
        return S

    def _call_attn(self, states, splits, n_kv, group, M, partial, epilogue, ksplit, preset):
        raise NotImplementedError

    # workgroup shape of the add+RMSNorm-input form for a SiLU store preset (the same shape;
    # staging the norm first is part of that form)
    _ADDNORM_SILU_PRESET = {1: 1, 4: 4, 6: 4, 9: 1}

    def forward_addnorm(self, parts: torch.Tensor, nparts: int, residual: torch.Tensor,
                        gain: torch.Tensor, eps: float, residual_out: torch.Tensor,
                        out: torch.Tensor | None = None,
                        partial: torch.Tensor | None = None) -> int:
        """This linear on add_rms_norm's output (fused_ops.py:60-70) whose input x is the fp16
        sum of the fp32 split-K partials parts[:nparts] ([nparts][M][K], slice order): every
        workgroup forms the M rows' norm itself, so no add+RMSNorm launch runs between the
        producer and this linear, and residual_out (not residual) receives the new residual.
        One row block whose rows fit the workgroup (M (K / 8) <= its threads: M <= 2 for the 2B
        decoder's qkv).  SiLU-fused: out [M, N/2], returns 1; else the fp32 split-K partial
        sums into partial (as forward_partial), returns their count."""
        M = residual.shape[0]
        if residual_out.data_ptr() == residual.data_ptr():
            raise ValueError("residual_out must not alias residual (every workgroup reads it)")
        if parts.dtype != torch.float32 or parts.numel() < nparts * M * self.K:
            raise ValueError("partials too small or not fp32")
        if self.fuse_silu:
            if out is None:
                raise ValueError("the SiLU-fused form needs out")
            preset = self._ADDNORM_SILU_PRESET.get(self.store_preset, 4)
            self._call_addnorm(parts, nparts, residual, gain, eps, residual_out, out, None,
                               EPI_SILU, 1, preset)
            return 1
        S = self.partial_slices(self.partial_ksplit)
        if partial is None or partial.numel() < S * M * self.N or partial.dtype != torch.float32:
            raise ValueError("partial buffer too small or not fp32")
        self._call_addnorm(parts, nparts, residual, gain, eps, residual_out, None, partial,
                           EPI_PARTIAL, self.partial_ksplit, 1)
        return S

    def _call_addnorm(self, parts, nparts, residual, gain, eps, residual_out, out, partial,
                      epilogue, ksplit, preset):
        raise NotImplementedError

    def _call_pipe_partial(self, x2d, partial, ksplit):
        raise NotImplementedError

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x2d = x.reshape(-1, self.K)
        if not x2d.is_contiguous():
            x2d = x2d.contiguous()
        require_cuda(x2d, dtype=torch.float16)
        out = torch.empty(x2d.shape[0], self.out_features, device=x.device, dtype=torch.float16)
        self.forward_out(x2d, out)
        return out.reshape(*x.shape[:-1], self.out_features)


class GPTQLinear(_Skinny):
    """W4A16 GPTQ linear: y = fp16(x . dequant(W)) (+ bias, added after rounding)."""

    fmt = "int4"

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
        call("omni_gptq_repack", ptr(qweight.contiguous()), ptr(scales.contiguous()),
             ptr(self.qweight_packed), ptr(self.scales_packed), K, N, int(fuse_silu), stream())
        self.bias = None if bias is None else bias.to(device=dev, dtype=torch.float16).contiguous()
        self._init_plan()

    def _call(self, x2d, out, partial, epilogue, ksplit, preset):
        call("omni_w4a16_gemm", ptr(x2d), x2d.stride(0), ptr(self.qweight_packed),
             ptr(self.scales_packed), ptr(self.bias), 1, ptr(out),
             0 if out is None else out.stride(0), ptr(partial), x2d.shape[0], self.N, self.K,
             epilogue, ksplit, preset, stream())

    # Prefill linears run the fp16 pipelined GEMM on the fp16 values of their int4 weights
    # (fp16((q - 8) s), the values the int4 kernels dequantise to, so the outputs are the
    # same): at M = 4096 a 2B layer's four linears take 459 us in fp16 against 608 us with the
    # dequantisation in the GEMM loop (redone by every wave that reads a tile), at M = 256
    # 83 against 104 us (MI355X).  With keep_f16 the expansion (omni_w4_unpack_f16, K N fp16:
    # 2.6 GB for the 2B decoder beside its 0.7 GB of int4, on a 288 GB part) is made at the
    # first prefill of F16_ROWS rows or more and kept with the linear; decode (up to 64 rows)
    # always streams the int4 words.  Without it, from UNPACK_ROWS rows the weights are
    # unpacked into a per-device scratch on every call (~23 us per layer at 2B).  The copy is
    # of the weights as they are at that first call: a linear whose packed weights are
    # rewritten afterwards calls release_f16() (which also retires captured prefill graphs).
    UNPACK_ROWS = 2048
    F16_ROWS = 256
    keep_f16 = True

    def release_f16(self) -> None:
        """Drop the resident fp16 expansion (made again at the next large prefill).  Graphs
        captured over it would launch on freed memory: the release advances
        ``weights_epoch()``, which graph owners compare before a replay."""
        global _WEIGHTS_EPOCH
        if getattr(self, "_w16", None) is not None:
            _WEIGHTS_EPOCH += 1
        self._w16 = None

    def _prefill_fmt(self, M: int) -> int:
        if self.N % 128 or self.K < 256:
            return 0
        return 1 if (self.keep_f16 and M >= self.F16_ROWS) or M >= self.UNPACK_ROWS else 0

    def _prefill_f16(self, M: int) -> torch.Tensor | None:
        """The packed fp16 weights the prefill GEMM runs on for M rows, or None (the int4
        pipeline dequantises in its loop)."""
        if self.N % 128 or self.K < 256:
            return None
        if self.keep_f16 and M >= self.F16_ROWS:
            w16 = getattr(self, "_w16", None)
            if w16 is None:
                w16 = torch.empty(self.N * self.K, device=self.qweight_packed.device,
                                  dtype=torch.float16)
                call("omni_w4_unpack_f16", ptr(self.qweight_packed), ptr(self.scales_packed),
                     ptr(w16), self.K, self.N, stream())
                self._w16 = w16
            return w16
        if M >= self.UNPACK_ROWS:
            w16 = _unpack_scratch(self.qweight_packed.device, self.N * self.K)
            call("omni_w4_unpack_f16", ptr(self.qweight_packed), ptr(self.scales_packed),
                 ptr(w16), self.K, self.N, stream())
            return w16
        return None

    def forward_out(self, x2d: torch.Tensor, out: torch.Tensor, preset: int | None = None,
                    ksplit: int | None = None):
        M = x2d.shape[0]
        if (M > MAX_SKINNY_M and ksplit is None and x2d.data_ptr() % 16 == 0
                and x2d.stride(0) % 8 == 0 and out.data_ptr() % 8 == 0 and out.stride(0) % 4 == 0):
            w16 = self._prefill_f16(M)
            if w16 is not None:
                epi = EPI_SILU if self.fuse_silu else EPI_STORE
                ks = 1 if self.fuse_silu else lib().omni_f16_gemm_pipe_splits(M, self.N, self.K, 0)
                ws = (torch.empty(ks * M * self.N, device=x2d.device, dtype=torch.float32)
                      if ks > 1 else None)
                call("omni_packed_gemm_pipe", ptr(x2d), x2d.stride(0), ptr(w16), None, 1,
                     ptr(self.bias), 1, ptr(out), out.stride(0), M, self.N, self.K, epi, 0, ks,
                     ptr(ws), stream())
                return out
        return super().forward_out(x2d, out, preset, ksplit)

    def _call_pipe_partial(self, x2d, partial, ksplit):
        M = x2d.shape[0]
        w16 = self._prefill_f16(M)
        if w16 is not None:
            call("omni_packed_gemm_pipe", ptr(x2d), x2d.stride(0), ptr(w16), None, 1, None, 0,
                 None, 0, M, self.N, self.K, EPI_PARTIAL, 0, ksplit, ptr(partial), stream())
        else:
            call("omni_packed_gemm_pipe", ptr(x2d), x2d.stride(0), ptr(self.qweight_packed),
                 ptr(self.scales_packed), 0, None, 0, None, 0, M, self.N, self.K, EPI_PARTIAL, 0,
                 ksplit, ptr(partial), stream())

    def _call_addnorm(self, parts, nparts, residual, gain, eps, residual_out, out, partial,
                      epilogue, ksplit, preset):
        call("omni_w4a16_gemm_addnorm", ptr(parts), nparts, ptr(residual), ptr(gain), float(eps),
             ptr(residual_out), ptr(self.qweight_packed), ptr(self.scales_packed), ptr(self.bias),
             1, ptr(out), 0 if out is None else out.stride(0), ptr(partial), residual.shape[0],
             self.N, self.K, epilogue, ksplit, preset, stream())

    def _call_attn(self, states, splits, n_kv, group, M, partial, epilogue, ksplit, preset):
        call("omni_w4a16_gemm_attn", ptr(states), splits, n_kv, group, ptr(self.qweight_packed),
             ptr(self.scales_packed), ptr(self.bias), 1, None, 0, ptr(partial), M, self.N,
             self.K, epilogue, ksplit, preset, stream())

    @classmethod
    def from_linear_rtn(cls, linear, group_size: int = 128, fuse_silu: bool | None = None):
        """Round-to-nearest int4 of an fp16 linear with no calibration, the reference's
        MarlinInt4Linear (kernels/marlin_linear.py:65-80: vLLM marlin_quantize, uint4b8,
        symmetric, group 128 along K): see rtn_int4.  ``linear`` is an nn.Linear-like module
        (weight [N, K], bias) or an F16Linear (unpacked; its gate|up fusion kept)."""
        if fuse_silu is None:
            fuse_silu = bool(getattr(linear, "fuse_silu", False))
        w = linear.dense_weight() if hasattr(linear, "dense_weight") else linear.weight.data
        qweight, scales = rtn_int4(w.to(torch.float16), group_size)
        return cls(qweight, scales, getattr(linear, "bias", None), group_size, fuse_silu)

    def dequantized(self) -> torch.Tensor:
        """W^T [K, N] fp16 as the kernels see it (columns in packed order)."""
        w = torch.empty(self.K, self.N, device=self.qweight_packed.device, dtype=torch.float16)
        call("omni_w4_dequant", ptr(self.qweight_packed), ptr(self.scales_packed), ptr(w),
             self.K, self.N, stream())
        return w


class F16Linear(_Skinny):
    """fp16 linear over the packed MFMA layout: y = fp16(x . W^T + b)."""

    fmt = "fp16"
    FILL_SLICES = True

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
        self._init_plan()

    @classmethod
    def from_linear(cls, linear: nn.Linear, fuse_silu: bool = False) -> "F16Linear":
        return cls(linear.weight.data, linear.bias, fuse_silu=fuse_silu)

    def dense_weight(self) -> torch.Tensor:
        """The nn.Linear weight [N, K] fp16 back from the packed layout (element (t, s, l, e)
        of tile t is W[16 t' + l % 16, 32 s + 8 (l // 16) + e], t' the tile before the
        gate|up interleave), for building other linear kinds from this one."""
        NT, KS = self.N // 16, self.K // 32
        w = self.weight_packed.view(NT, KS, 4, 16, 8).permute(0, 3, 1, 2, 4)
        w = w.reshape(NT, 16, self.K)
        if self.fuse_silu:
            w = torch.cat([w[0::2], w[1::2]], 0)
        return w.reshape(self.N, self.K).contiguous()

    def _call(self, x2d, out, partial, epilogue, ksplit, preset):
        call("omni_f16_gemm", ptr(x2d), x2d.stride(0), ptr(self.weight_packed), ptr(self.bias),
             ptr(out), 0 if out is None else out.stride(0), ptr(partial), x2d.shape[0], self.N,
             self.K, epilogue, ksplit, preset, stream())

    def _call_pipe_partial(self, x2d, partial, ksplit):
        call("omni_packed_gemm_pipe", ptr(x2d), x2d.stride(0), ptr(self.weight_packed), None, 1,
             None, 0, None, 0, x2d.shape[0], self.N, self.K, EPI_PARTIAL, 0, ksplit, ptr(partial),
             stream())

    def _call_addnorm(self, parts, nparts, residual, gain, eps, residual_out, out, partial,
                      epilogue, ksplit, preset):
        call("omni_f16_gemm_addnorm", ptr(parts), nparts, ptr(residual), ptr(gain), float(eps),
             ptr(residual_out), ptr(self.weight_packed), ptr(self.bias), ptr(out),
             0 if out is None else out.stride(0), ptr(partial), residual.shape[0], self.N, self.K,
             epilogue, ksplit, preset, stream())

    def _call_attn(self, states, splits, n_kv, group, M, partial, epilogue, ksplit, preset):
        call("omni_f16_gemm_attn", ptr(states), splits, n_kv, group, ptr(self.weight_packed),
             ptr(self.bias), None, 0, ptr(partial), M, self.N, self.K, epilogue, ksplit, preset,
             stream())


# Advanced whenever a linear frees device memory that a captured graph may launch on
# (GPTQLinear.release_f16); the runner's prefill graphs are dropped when it moves.
_WEIGHTS_EPOCH = 0


def weights_epoch() -> int:
    return _WEIGHTS_EPOCH


class FP8Linear(nn.Module):
    """W8A8 e4m3fn linear, FP8Linear's API (kernels/fp8_linear.py:66-126), in both of its
    forms:

    * per-tensor (``rowwise=False``, the reference's default and what apply_mixed builds):
      one weight scale sw = fp16(amax |W| / 448), Wq = e4m3(fp16(W / sw)) (:87-90); the
      forward quantises x with one dynamic scale, sa = fp16(amax |x| / 448),
      xq = e4m3(fp16(x / sa)) (_quant_fp8_pertensor's eager branch, :40-41; bf16 input:
      the same in bf16) and writes the fp16 product directly, plus the fp16 bias
      (:119-125);
    * row-wise (``rowwise=True``, fuse_norm_fp8's gate_up): sw[n] = fp16(amax_k |W[n, :]| /
      448), Wq = e4m3(W / sw) (:83-86, an fp32 division); the forward quantises x per
      token (quant_fp8, :45-63) and returns bf16((xq . Wq^T) * sa * sw) cast to fp16 plus
      the bias (:115-118, 124-125); ``forward_prequant(xq, scale)`` takes rows already
      quantised by add_rms_norm_fp8 and returns the bf16 product (:99-108).

    Weights are quantised on the device at construction.  The scales are stored as an [N]
    array either way (per-tensor: the one value repeated), the form the GEMM reads."""

    fmt = "fp8"

    def __init__(self, weight: torch.Tensor, bias=None, rowwise: bool = False):
        super().__init__()
        N, K = weight.shape
        require_cuda(weight, dtype=torch.float16)
        if N % 128 or K % 128:
            raise ValueError(f"FP8Linear needs N, K multiples of 128 (got {N}, {K})")
        dev = weight.device
        self.K, self.N = K, N
        self.rowwise = bool(rowwise)
        w = weight.contiguous()
        self.register_buffer("weight_fp8", torch.empty(N, K, device=dev, dtype=torch.uint8))
        self.register_buffer("weight_scale", torch.empty(N, device=dev, dtype=torch.float32))
        if self.rowwise:
            call("omni_fp8_quant_weight_rows", ptr(w), K, ptr(self.weight_fp8),
                 ptr(self.weight_scale), N, K, stream())
        else:
            work = torch.empty(lib().omni_fp8_quant_tensor_work(N), device=dev,
                               dtype=torch.float32)
            call("omni_fp8_quant_tensor", ptr(w), K, ptr(self.weight_fp8), ptr(self.weight_scale),
                 ptr(work), N, K, 0, stream())
        self.bias = None if bias is None else bias.to(device=dev, dtype=torch.float16).contiguous()

    @classmethod
    def from_linear(cls, linear, rowwise: bool = False) -> "FP8Linear":
        """From an fp16 linear (fp8_linear.py:93-97): an nn.Linear-like module (weight
        [N, K], bias) or an F16Linear (unpacked)."""
        w = linear.dense_weight() if hasattr(linear, "dense_weight") else linear.weight.data
        return cls(w.to(torch.float16), getattr(linear, "bias", None), rowwise=rowwise)

    @property
    def out_features(self) -> int:
        return self.N

    @property
    def wq(self) -> torch.Tensor:
        """The e4m3 weight codes [N, K] (the reference's ``wq`` buffer)."""
        return self.weight_fp8.view(torch.float8_e4m3fn)

    @property
    def wscale(self) -> torch.Tensor:
        """The reference's ``wscale``: [1, N] row-wise, a 0-dim scalar per-tensor."""
        return self.weight_scale.view(1, -1) if self.rowwise else self.weight_scale[0]

    def quantize_input(self, x2d: torch.Tensor):
        """The forward's activation quantisation of fp16 or bf16 rows: (xq e4m3 bytes
        [M, K], scale fp32 [M, 1]) - per token (quant_fp8, fp8_linear.py:45-63) for the
        row-wise form, one value repeated for the per-tensor form (:40-41)."""
        M = x2d.shape[0]
        xq = torch.empty(M, self.K, device=x2d.device, dtype=torch.uint8)
        sa = torch.empty(M, 1, device=x2d.device, dtype=torch.float32)
        bf16 = x2d.dtype == torch.bfloat16
        if self.rowwise:
            fn = "omni_fp8_quant_rows_bf16" if bf16 else "omni_fp8_quant_rows"
            call(fn, ptr(x2d), x2d.stride(0), ptr(xq), ptr(sa), M, self.K, 0.0, stream())
        else:
            work = torch.empty(lib().omni_fp8_quant_tensor_work(M), device=x2d.device,
                               dtype=torch.float32)
            call("omni_fp8_quant_tensor", ptr(x2d), x2d.stride(0), ptr(xq), ptr(sa), ptr(work),
                 M, self.K, int(bf16), stream())
        return xq, sa

    # omni_fp8_gemm's output forms
    OUT_F16_VIA_BF16, OUT_BF16, OUT_F16 = 0, 1, 2

    def gemm_out(self, xq: torch.Tensor, sa: torch.Tensor, out: torch.Tensor, mode: int):
        """The scaled product into ``out`` in form ``mode``: OUT_BF16 the bf16 product plus
        bias.to(bf16) in bf16 (forward_prequant, :99-108); OUT_F16_VIA_BF16 the bf16
        product cast to fp16 plus the fp16 bias (row-wise forward, :115-118); OUT_F16 the
        fp16 product plus the fp16 bias (per-tensor forward, :119-125)."""
        M = xq.shape[0]
        call("omni_fp8_gemm", ptr(xq), ptr(sa), ptr(self.weight_fp8), ptr(self.weight_scale),
             ptr(self.bias), ptr(out), out.stride(0), M, self.N, self.K, int(mode), stream())
        return out

    def forward_prequant(self, xq: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
        if not self.rowwise:
            raise ValueError("forward_prequant needs the row-wise form (fp8_linear.py:99-103: "
                             "per-token activation scales with per-channel weight scales)")
        xq2 = xq.reshape(-1, self.K)
        if xq2.dtype == torch.float8_e4m3fn:
            xq2 = xq2.view(torch.uint8)
        xq2 = xq2.contiguous()
        out = torch.empty(xq2.shape[0], self.N, device=xq.device, dtype=torch.bfloat16)
        self.gemm_out(xq2, scale.reshape(-1).contiguous().float(), out, self.OUT_BF16)
        return out.reshape(*xq.shape[:-1], self.N)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """fp16 or bf16 x (the bf16 silu_mul output of the fused FP8 MLP route,
        qwen2_llm.py:132-134) -> fp16."""
        x2d = x.reshape(-1, self.K)
        if not x2d.is_contiguous():
            x2d = x2d.contiguous()
        require_cuda(x2d)
        if x2d.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"expected fp16 or bf16 activations, got {x2d.dtype}")
        xq, sa = self.quantize_input(x2d)
        out = torch.empty(x2d.shape[0], self.N, device=x.device, dtype=torch.float16)
        self.gemm_out(xq, sa, out, self.OUT_F16_VIA_BF16 if self.rowwise else self.OUT_F16)
        return out.reshape(*x.shape[:-1], self.N)


class LMHeadArgmax(nn.Module):
    """Tied lm_head (qwen2_llm.py:167-168, 190) fused with greedy argmax
    (runners/multimodal.py:307-308): ids = argmax_n fp16(h . E[n]), lowest index on ties.
    The embedding table is stored once, packed; the token gather reads the packed form.
    Two launches: the GEMM writes per-workgroup (max, index) candidates, a small kernel
    reduces them (and can advance the decode-step bookkeeping)."""

    def __init__(self, embed: torch.Tensor):
        super().__init__()
        V, H = embed.shape
        dev = embed.device
        require_cuda(embed, dtype=torch.float16)
        self.V, self.H = V, H
        self.register_buffer("table_packed", torch.empty(V // 16, H // 32, 64, 8, device=dev,
                                                        dtype=torch.float16))
        call("omni_f16_pack", ptr(embed.contiguous()), ptr(self.table_packed), H, V, 0, stream())
        self.grid = lib().omni_lmhead_argmax_grid(V)
        self.max_rows = lib().omni_lmhead_max_rows(H)     # rows per candidates launch
        self._cand_val = torch.empty(self.grid * MAX_SKINNY_M, device=dev, dtype=torch.float32)
        self._cand_idx = torch.empty(self.grid * MAX_SKINNY_M, device=dev, dtype=torch.int32)

    def argmax_out(self, h2d: torch.Tensor, ids_out: torch.Tensor, logits_out=None,
                   next_ids: torch.Tensor | None = None, lengths: torch.Tensor | None = None):
        """ids_out[m] = greedy token of row m; optionally also next_ids[m] = ids_out[m] and
        lengths[m] += 1 (rows < M) in the same finalize launch."""
        M = h2d.shape[0]
        if M > MAX_SKINNY_M:
            raise ValueError(f"lm_head argmax supports up to {MAX_SKINNY_M} rows per call")
        require_cuda(h2d, dtype=torch.float16)
        require_cuda(ids_out, dtype=torch.int64)
        # one candidates + finalize pair per block of rows the kernel stages at once
        rows = lambda t, s, e: None if t is None else t[s:e]
        for s in range(0, M, self.max_rows):
            e = min(M, s + self.max_rows)
            call("omni_lmhead_candidates", ptr(h2d[s:e]), h2d.stride(0), ptr(self.table_packed),
                 e - s, self.V, self.H, ptr(rows(logits_out, s, e)), ptr(self._cand_val),
                 ptr(self._cand_idx), stream())
            call("omni_argmax_finalize", ptr(self._cand_val), ptr(self._cand_idx), self.grid,
                 e - s, ptr(ids_out[s:e]), ptr(rows(next_ids, s, e)), ptr(rows(lengths, s, e)),
                 stream())
        return ids_out

    def logits(self, h2d: torch.Tensor) -> torch.Tensor:
        """fp16 logits [M, V] (the fused argmax runs alongside and is discarded)."""
        out = torch.empty(h2d.shape[0], self.V, device=h2d.device, dtype=torch.float16)
        ids = torch.empty(h2d.shape[0], device=h2d.device, dtype=torch.int64)
        for s in range(0, h2d.shape[0], MAX_SKINNY_M):
            e = min(s + MAX_SKINNY_M, h2d.shape[0])
            self.argmax_out(h2d[s:e], ids[s:e], out[s:e])
        return out
