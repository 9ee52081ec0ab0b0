"""ctypes binding of the gfx950 C ABI declared in include/omniserver_amd.h.

The shared library is built in-tree by ``python -m omniserver_amd.build``.  There
is no fallback: if it is missing or fails to load, every op raises.  torch is
imported first so the library binds to the HIP runtime torch already loaded
(both carry the soname libamdhip64.so.7) and can launch on torch's streams.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libomniserver_amd.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float

# name -> argtypes (restype is always c_int: 0 ok, <0 argument error, >0 hipError_t)
SIGNATURES = {
    "omni_rmsnorm": [_P, _P, _P, _I, _I, _F, _P],
    "omni_add_rmsnorm": [_P, _P, _P, _P, _P, _I, _I, _F, _P],
    "omni_add_rmsnorm_fp8": [_P, _P, _P, _P, _P, _P, _I, _I, _F, _P],
    "omni_add_rmsnorm_partials": [_P, _I, _P, _P, _P, _P, _I, _I, _F, _P],
    "omni_embed_rmsnorm": [_P, _P, _I, _I64, _P, _P, _P, _I, _I, _F, _P],
    "omni_embed_rmsnorm_rope": [_P, _P, _I, _I64, _P, _P, _P, _I, _I, _F, _P, _P, _P, _P, _I,
                                _P, _P],
    "omni_rope_rows": [_P, _P, _P, _P, _P, _I, _I, _I, _P, _P],
    "omni_kv_copy_slot": [_P, _I, _I, _I, _I, _I, _I, _I64, _P, _P],
    "omni_embedding": [_P, _P, _I, _I64, _P, _I, _I, _P],
    "omni_silu_mul": [_P, _P, _I, _I, _P],
    "omni_silu_mul_bf16": [_P, _P, _I, _I, _P],
    "omni_mrope_kv_write": [_P, _I, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                            _I, _I, _I, _I, _P],
    "omni_mrope_kv_write_partials": [_P, _I, _P, _I, _P, _I, _P, _P, _P, _P, _P, _I, _P, _P, _P,
                                     _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P],
    "omni_decode_attention": [_P, _I, _P, _P, _I, _I, _P, _P, _I, _I, _P, _I, _I, _I, _I, _F, _I,
                              _I, _P, _I64, _P],
    "omni_decode_attention_fused": [_P, _I, _P, _I, _P, _P, _I, _P, _I, _I, _I, _P, _P, _I, _I,
                                    _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _P, _I64, _I, _P, _P],
    "omni_fp8_quant_rows": [_P, _I, _P, _P, _I, _I, _F, _P],
    "omni_fp8_quant_rows_bf16": [_P, _I, _P, _P, _I, _I, _F, _P],
    "omni_fp8_quant_weight_rows": [_P, _I, _P, _P, _I, _I, _P],
    "omni_fp8_quant_tensor": [_P, _I, _P, _P, _P, _I, _I, _I, _P],
    "omni_fp8_quant_tensor_work": [_I],
    "omni_fp8_gemm": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    "omni_fp8_gemm_plan": [_I, _I, _I, ctypes.POINTER(_I)],
    "omni_w4a16_gemm_attn": [_P, _I, _I, _I, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _I,
                             _P],
    "omni_f16_gemm_attn": [_P, _I, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _P],
    "omni_w4a16_gemm_addnorm": [_P, _I, _P, _P, _F, _P, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I,
                                _I, _I, _I, _P],
    "omni_f16_gemm_addnorm": [_P, _I, _P, _P, _F, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I,
                              _P],
    "omni_prefill_attention_gqa": [_P, _I, _P, _P, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I,
                                   _F, _P],
    "omni_prefill_attention_gqa_halves": [_P, _I, _P, _P, _I, _I, _P, _P, _P, _I, _P, _I, _I,
                                          _I, _I, _F, _P],
    "omni_prefill_attention": [_P, _I, _P, _P, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _F,
                               _P],
    "omni_prefill_attention_split": [_P, _I, _P, _P, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I,
                                     _F, _P],
    "omni_w4a16_gemm": [_P, _I, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _I, _P],
    "omni_f16_gemm": [_P, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _P],
    "omni_f16_gemm_tiled": [_P, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _P],
    "omni_f16_gemm_pipe": [_P, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P],
    "omni_f16_gemm_pipe_splits": [_I, _I, _I, _I],
    "omni_packed_gemm_pipe": [_P, _I, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P],
    "omni_packed_gemm_pipe_plan": [_I, _I, _I, _I, _I, _I, _I, _I, ctypes.POINTER(_I),
                                   ctypes.POINTER(_I), ctypes.POINTER(_I)],
    "omni_layernorm": [_P, _I, _P, _P, _I, _I, _F, _P, _I, _P],
    "omni_layernorm_partials": [_P, _I, _P, _P, _I, _P, _I, _P, _P, _I, _I, _F, _P, _I, _P],
    "omni_f16_gemm_pipe_packed": [_P, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P],
    "omni_vision_rope": [_P, _I, _I, _I, _I, _P, _P, _P],
    "omni_vit_attention": [_P, _I, _I, _I, _I, _P, _P, _I, _P, _I, _F, _P],
    "omni_gemm_slices": [_I, _I],
    "omni_lmhead_argmax_grid": [_I],
    "omni_lmhead_max_rows": [_I],
    "omni_lmhead_candidates": [_P, _I, _P, _I, _I, _I, _P, _P, _P, _P],
    "omni_argmax_finalize": [_P, _P, _I, _I, _P, _P, _P, _P],
    "omni_lmhead_argmax_noalloc": [_P, _I, _P, _I, _I, _I, _P, _P, _P, _P, _P],
    "omni_gptq_repack": [_P, _P, _P, _P, _I, _I, _I, _P],
    "omni_f16_pack": [_P, _P, _I, _I, _I, _P],
    "omni_w4_dequant": [_P, _P, _P, _I, _I, _P],
    "omni_w4_unpack_f16": [_P, _P, _P, _I, _I, _P],
    "omni_bf16_rne_check": [_P, _P],
}

ERRORS = {-1: "invalid argument", -2: "unsupported shape"}

_lib = None


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"omniserver_amd HIP library missing at {LIB_PATH}; build it with "
                "`python -m omniserver_amd.build` (there is no CPU fallback)")
        so = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(so, name)
            fn.argtypes = argtypes
            fn.restype = _I
        _lib = so
    return _lib


_FN: dict = {}


def call(name: str, *args) -> None:
    """Invoke an entry point and raise on a non-zero return code."""
    fn = _FN.get(name)
    if fn is None:
        fn = _FN[name] = getattr(lib(), name)
    rc = fn(*args)
    if rc != 0:
        what = ERRORS.get(rc) or f"hipError_t {rc}"
        raise RuntimeError(f"{name} failed: {what}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


def stream() -> int:
    """Handle of torch's current HIP stream on the current device (captured streams
    included), read without building a Stream object (a tenth of the host time)."""
    return torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice())


def require_cuda(*tensors, dtype=None, contiguous=True) -> None:
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("omniserver_amd ops run on the GPU only (got a CPU tensor)")
        if dtype is not None and t.dtype != dtype:
            raise TypeError(f"expected {dtype}, got {t.dtype}")
        if contiguous and not t.is_contiguous():
            raise ValueError("expected a contiguous tensor")
