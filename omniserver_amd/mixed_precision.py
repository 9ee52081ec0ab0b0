"""Per-op precision of the decoder's linears, the reference's kernels/mixed_precision.py and
quantize_llm_marlin (kernels/marlin_linear.py:98-111) on this library's linear modules.

Operators are replaced by ``setattr`` on the reference's module paths
(``self_attn.qkv_proj / o_proj``, ``mlp.gate_up_proj / down_proj``), from the fp16 modules a
``Qwen2LLM.from_fp16`` model holds (F16Linear unpacks its weight for the conversion):

* ``"fp16"`` keeps the module;
* ``"fp8"``  FP8Linear in its default per-tensor form (W8A8 e4m3, one weight scale, one
  dynamic activation scale, fp16 product; kernels/fp8_linear.py:66-126 via
  FP8Linear.from_linear, mixed_precision.py:39-41);
* ``"marlin"`` round-to-nearest int4 (uint4b8, group 128) as GPTQLinear, the reference's
  MarlinInt4Linear (marlin_linear.py:65-80).

``fuse_norm_fp8`` folds gate_up's activation quantisation into the post-attention norm
(mixed_precision.py:53-73): gate_up becomes row-wise FP8 and the norm emits (e4m3 rows,
per-token scale); a gate_up that is already per-tensor FP8 is refused, as the reference
refuses it.
Hadamard rotations ("+h") and the M-adaptive "fp8a" linear are not part of this build.
"""

from __future__ import annotations

from .linear import FP8Linear, GPTQLinear

# mixed_precision.py:19: MLP on FP8, attention projections kept fp16
DEFAULT_PLAN = {"qkv": "fp16", "o": "fp16", "gate_up": "fp8", "down": "fp8"}

_ATTR = {
    "qkv": ("self_attn", "qkv_proj"),
    "o": ("self_attn", "o_proj"),
    "gate_up": ("mlp", "gate_up_proj"),
    "down": ("mlp", "down_proj"),
}


def _replace(layer, op: str, prec: str) -> int:
    """Replace one operator of one layer (mixed_precision.py:30-50); returns 1 if it was."""
    sub, attr = _ATTR[op]
    parent = getattr(layer, sub)
    lin = getattr(parent, attr)
    if prec == "fp16":
        return 0
    if prec == "fp8":
        if isinstance(lin, FP8Linear):       # already FP8 (e.g. by fuse_norm_fp8)
            return 0
        new = FP8Linear.from_linear(lin)     # per-tensor, FP8Linear's default
    elif prec == "marlin":
        if isinstance(lin, GPTQLinear):
            return 0
        new = GPTQLinear.from_linear_rtn(lin)
    else:
        raise ValueError(f"unknown precision {prec!r} (fp16, fp8 or marlin; Hadamard '+h' and "
                         f"'fp8a' are not part of this build)")
    setattr(parent, attr, new)
    return 1


def apply_mixed(model, plan: dict | None = None) -> dict:
    """Apply a per-op plan to every layer (mixed_precision.py:78-84); returns
    {op: (precision, layers replaced)}."""
    plan = plan or DEFAULT_PLAN
    counts = {op: 0 for op in plan}
    for layer in model.layers:
        for op, prec in plan.items():
            counts[op] += _replace(layer, op, prec)
    return {op: (plan[op], counts[op]) for op in plan}


def fuse_norm_fp8(model) -> int:
    """gate_up as row-wise FP8 fed straight by the post-attention norm's per-token e4m3
    output (mixed_precision.py:53-73), called on the fp16 model; returns the number of
    layers fused.  Raises ValueError, as the reference does (:69-70), for a gate_up that
    is already per-tensor FP8, and for one that is neither fp16 nor row-wise FP8 (int4)."""
    n = 0
    for layer in model.layers:
        gu = layer.mlp.gate_up_proj
        if isinstance(gu, FP8Linear):
            if not gu.rowwise:
                raise ValueError("gate_up is already per-tensor FP8; the fused norm needs a "
                                 "row-wise gate_up: call fuse_norm_fp8 before quantising")
        elif isinstance(gu, GPTQLinear):
            raise ValueError("fuse_norm_fp8 needs an fp16 (or row-wise FP8) gate_up, "
                             "not an int4 one")
        else:
            layer.mlp.gate_up_proj = FP8Linear.from_linear(gu, rowwise=True)
        layer.post_attention_layernorm.fp8_out = True
        n += 1
    return n


def quantize_llm_marlin(model, scope: str = "decoder") -> int:
    """RTN int4 of the decoder linears (marlin_linear.py:98-111): scope "decoder" all four
    per layer, "mlp" gate_up and down only.  Returns the number of linears quantised."""
    if scope not in ("decoder", "mlp"):
        raise ValueError(f"scope {scope!r} is 'decoder' or 'mlp'")
    n = 0
    for layer in model.layers:
        if scope == "decoder":
            layer.self_attn.qkv_proj = GPTQLinear.from_linear_rtn(layer.self_attn.qkv_proj)
            layer.self_attn.o_proj = GPTQLinear.from_linear_rtn(layer.self_attn.o_proj)
            n += 2
        layer.mlp.gate_up_proj = GPTQLinear.from_linear_rtn(layer.mlp.gate_up_proj)
        layer.mlp.down_proj = GPTQLinear.from_linear_rtn(layer.mlp.down_proj)
        n += 2
    return n
