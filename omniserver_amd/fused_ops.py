"""Fused elementwise ops with the reference's Python signatures, on gfx950 HIP.

Mirrors omniserve/kernels/fused_ops.py (rms_norm :32, add_rms_norm :60,
add_rms_norm_fp8 :94, silu_mul :122): same arguments, same return values, new
output tensors.  The ``*_out`` variants write into caller buffers (used by the
captured decode step, which must not allocate).
"""

from __future__ import annotations

import torch

from ._lib import call, ptr, require_cuda, stream


def _rows(x: torch.Tensor) -> tuple[int, int]:
    n = x.shape[-1]
    return x.numel() // n if n else 0, n


def rms_norm_out(x, weight, eps, out):
    require_cuda(x, weight, out, dtype=torch.float16)
    m, n = _rows(x)
    call("omni_rmsnorm", ptr(x), ptr(weight), ptr(out), m, n, float(eps), stream())
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """y = x * rsqrt(mean(x^2) + eps) * w (fp32 reduce, fp16 store)."""
    x = x.contiguous()
    return rms_norm_out(x, weight, eps, torch.empty_like(x))


def add_rms_norm_out(x, residual, weight, eps, out, res_out):
    require_cuda(x, residual, weight, out, res_out, dtype=torch.float16)
    m, n = _rows(x)
    call("omni_add_rmsnorm", ptr(x), ptr(residual), ptr(weight), ptr(out), ptr(res_out), m, n,
         float(eps), stream())
    return out, res_out


def add_rms_norm(x, residual, weight, eps):
    """Returns (normed, new_residual) with new_residual = fp16(residual + x)."""
    x = x.contiguous()
    residual = residual.contiguous()
    return add_rms_norm_out(x, residual, weight, eps, torch.empty_like(x),
                            torch.empty_like(residual))


def add_rms_norm_partials_out(partials, nparts: int, residual, weight, eps, out, res_out):
    """add_rms_norm where x is fp16(sum of nparts fp32 split-K partials [S, M, H])."""
    require_cuda(partials, dtype=torch.float32)
    require_cuda(residual, weight, out, res_out, dtype=torch.float16)
    m, n = _rows(residual)
    call("omni_add_rmsnorm_partials", ptr(partials), nparts, ptr(residual), ptr(weight), ptr(out),
         ptr(res_out), m, n, float(eps), stream())
    return out, res_out


def add_rms_norm_fp8(x, residual, weight, eps):
    """add_rms_norm with the normed output quantised to e4m3fn per row.

    Returns (fp8 [M, N], scale fp32 [M, 1], new_residual); scale = max(amax/448, 1e-12)."""
    x = x.contiguous()
    residual = residual.contiguous()
    require_cuda(x, residual, weight, dtype=torch.float16)
    m, n = _rows(x)
    out = torch.empty(m, n, device=x.device, dtype=torch.float8_e4m3fn)
    scale = torch.empty(m, 1, device=x.device, dtype=torch.float32)
    nres = torch.empty_like(residual)
    call("omni_add_rmsnorm_fp8", ptr(x), ptr(residual), ptr(weight), ptr(out), ptr(scale),
         ptr(nres), m, n, float(eps), stream())
    return out, scale, nres


def silu_mul_out(gate_up, out):
    """fp16 in/out, or bf16 in/out (the fp8 MLP route's gate_up.forward_prequant output)."""
    require_cuda(gate_up, out)
    if gate_up.dtype != out.dtype or gate_up.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"silu_mul takes fp16 or bf16 (got {gate_up.dtype} -> {out.dtype})")
    m, n2 = _rows(gate_up)
    fn = "omni_silu_mul_bf16" if gate_up.dtype == torch.bfloat16 else "omni_silu_mul"
    call(fn, ptr(gate_up), ptr(out), m, n2 // 2, stream())
    return out


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """gate_up [..., 2N] (gate first) -> silu(gate) * up  [..., N]."""
    gate_up = gate_up.contiguous()
    n = gate_up.shape[-1] // 2
    out = torch.empty(*gate_up.shape[:-1], n, device=gate_up.device, dtype=gate_up.dtype)
    return silu_mul_out(gate_up, out)


def embedding_out(ids, table, packed: bool, out):
    """out[t] = table[ids[t]] for a plain [V, H] or packed fp16 table."""
    require_cuda(ids, dtype=torch.int64)
    require_cuda(table, out, dtype=torch.float16)
    hidden = out.shape[-1]
    vocab = table.numel() // hidden
    call("omni_embedding", ptr(ids), ptr(table), int(packed), vocab, ptr(out), ids.numel(),
         hidden, stream())
    return out


def embed_rms_norm_out(ids, table, packed: bool, weight, eps, out, res_out):
    """Layer-0 input of the decode step: residual = E[ids]; out = rms_norm(residual)."""
    require_cuda(ids, dtype=torch.int64)
    require_cuda(table, weight, out, res_out, dtype=torch.float16)
    hidden = out.shape[-1]
    vocab = table.numel() // hidden
    call("omni_embed_rmsnorm", ptr(ids), ptr(table), int(packed), vocab, ptr(weight), ptr(out),
         ptr(res_out), ids.numel(), hidden, float(eps), stream())
    return out, res_out


def embed_rms_norm_rope_out(ids, table, packed: bool, weight, eps, out, res_out, lengths,
                            rope_delta, cos_tab, sin_tab, rope_rows):
    """embed_rms_norm_out that also writes the decode step's rotary rows [n, 128] (cos |
    sin at lengths[row] + rope_delta[row]) in the same launch."""
    require_cuda(ids, lengths, dtype=torch.int64)
    require_cuda(table, weight, out, res_out, cos_tab, sin_tab, rope_rows, dtype=torch.float16)
    hidden = out.shape[-1]
    vocab = table.numel() // hidden
    call("omni_embed_rmsnorm_rope", ptr(ids), ptr(table), int(packed), vocab, ptr(weight),
         ptr(out), ptr(res_out), ids.numel(), hidden, float(eps), ptr(lengths), ptr(rope_delta),
         ptr(cos_tab), ptr(sin_tab), cos_tab.shape[0], ptr(rope_rows), stream())
    return out, res_out
