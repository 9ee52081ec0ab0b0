"""Checkpoint ingest: Qwen2-VL decoder weights from ``model*.safetensors`` files.

Two layouts, the same two the reference reads:

* GPTQ int4 (``quant="gptq"``, ``gptq_dir``): the AutoGPTQ tensors per decoder linear -
  ``qweight`` int32 [K/8, N] (8 four-bit codes per word, lowest k in the low nibble),
  ``scales`` fp16 [K/128, N] - symmetric with implicit zero point 8 (uint4b8: ``qzeros``
  are not read, as kernels/marlin_linear.py:83-96 does not read them), no activation
  order.  q|k|v and gate|up are concatenated along N and the q/k/v biases along the
  output, as load_gptq_llm does (kernels/marlin_linear.py:114-143); embeddings (tied
  lm_head), the final norm and the per-layer RMSNorm gains are fp16.
* fp16 Hugging Face (``model_dir``): ``*_proj.weight`` in nn.Linear layout, fused the
  same way (model/qwen2_llm.py:193-219), with either the raw ``model.`` prefix or the
  ``model.language_model.`` prefix of newer transformers state dicts.

Files are read with ``safetensors`` (no code runs from the file).  The decoder
result is the weight dict the model builders take (``synth.gptq_decoder`` /
``synth.fp16_decoder`` layout); ``vision_state_dict`` picks the vision tower's fp16
tensors (kept fp16 in both layouts, as models/qwen2_vl.py:39-48 loads them).
"""

from __future__ import annotations

import glob
import os
from typing import Dict, List

import torch

GROUP = 128


def read_safetensors(path: str) -> Dict[str, torch.Tensor]:
    """Every tensor of ``path`` (a .safetensors file, or a directory of model*.safetensors)."""
    from safetensors.torch import load_file
    files = [path] if os.path.isfile(path) else sorted(glob.glob(os.path.join(path, "model*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no model*.safetensors under {path}")
    sd: Dict[str, torch.Tensor] = {}
    for f in files:
        sd.update(load_file(f, device="cpu"))
    return sd


def _prefix(sd: Dict[str, torch.Tensor]) -> str:
    return "model.language_model." if "model.language_model.embed_tokens.weight" in sd else "model."


def _num_layers(sd: Dict[str, torch.Tensor], P: str) -> int:
    n = 0
    while f"{P}layers.{n}.input_layernorm.weight" in sd:
        n += 1
    if n == 0:
        raise KeyError(f"no decoder layers ({P}layers.0.input_layernorm.weight missing)")
    return n


def _get(sd: Dict[str, torch.Tensor], key: str) -> torch.Tensor:
    if key not in sd:
        raise KeyError(f"checkpoint tensor {key!r} missing")
    return sd[key]


def _check_gptq(sd, lp: str, names: List[str]) -> None:
    for x in names:
        q = _get(sd, lp + x + ".qweight")
        s = _get(sd, lp + x + ".scales")
        if q.dtype != torch.int32 or q.dim() != 2:
            raise ValueError(f"{lp + x}.qweight: int32 [K/8, N] expected, got {q.dtype} {tuple(q.shape)}")
        K = q.shape[0] * 8
        if s.shape != (K // GROUP, q.shape[1]):
            raise ValueError(f"{lp + x}.scales: [{K // GROUP}, {q.shape[1]}] expected (group 128), "
                             f"got {tuple(s.shape)}")
        gi = sd.get(lp + x + ".g_idx")
        if gi is not None and not torch.equal(gi.to(torch.int64).cpu(),
                                              torch.arange(K, dtype=torch.int64) // GROUP):
            raise ValueError(f"{lp + x}.g_idx: activation-order (desc_act) checkpoints are not "
                             "supported (the reference loads desc_act=False weights only)")


def gptq_decoder_from_state_dict(sd: Dict[str, torch.Tensor]) -> Dict:
    """AutoGPTQ state dict -> the GPTQ weight dict (fused q|k|v and gate|up along N)."""
    P = _prefix(sd)
    L = _num_layers(sd, P)
    f16 = lambda t: t.to(torch.float16).contiguous()
    out = {"embed": f16(_get(sd, P + "embed_tokens.weight")), "norm": f16(_get(sd, P + "norm.weight")),
           "layers": []}
    for i in range(L):
        lp = f"{P}layers.{i}."
        _check_gptq(sd, lp, [f"self_attn.{x}_proj" for x in "qkvo"] +
                    [f"mlp.{x}_proj" for x in ("gate", "up", "down")])
        cat_n = lambda names, t: torch.cat([_get(sd, lp + n + "." + t) for n in names], dim=1).contiguous()
        qkv = [f"self_attn.{x}_proj" for x in "qkv"]
        gu = ["mlp.gate_proj", "mlp.up_proj"]
        out["layers"].append({
            "in_norm": f16(_get(sd, lp + "input_layernorm.weight")),
            "post_norm": f16(_get(sd, lp + "post_attention_layernorm.weight")),
            "qkv_q": cat_n(qkv, "qweight"), "qkv_s": f16(cat_n(qkv, "scales")),
            "qkv_b": f16(torch.cat([_get(sd, lp + n + ".bias") for n in qkv], dim=0)),
            "o_q": _get(sd, lp + "self_attn.o_proj.qweight").contiguous(),
            "o_s": f16(_get(sd, lp + "self_attn.o_proj.scales")),
            "gate_up_q": cat_n(gu, "qweight"), "gate_up_s": f16(cat_n(gu, "scales")),
            "down_q": _get(sd, lp + "mlp.down_proj.qweight").contiguous(),
            "down_s": f16(_get(sd, lp + "mlp.down_proj.scales")),
        })
    return out


def fp16_decoder_from_state_dict(sd: Dict[str, torch.Tensor]) -> Dict:
    """Hugging Face Qwen2-VL state dict -> the fp16 weight dict (load_from_hf's fusion)."""
    P = _prefix(sd)
    L = _num_layers(sd, P)
    f16 = lambda t: t.to(torch.float16).contiguous()
    out = {"embed": f16(_get(sd, P + "embed_tokens.weight")), "norm": f16(_get(sd, P + "norm.weight")),
           "layers": []}
    for i in range(L):
        lp = f"{P}layers.{i}."
        g = lambda k: _get(sd, lp + k)
        out["layers"].append({
            "in_norm": f16(g("input_layernorm.weight")),
            "post_norm": f16(g("post_attention_layernorm.weight")),
            "qkv_w": f16(torch.cat([g(f"self_attn.{x}_proj.weight") for x in "qkv"], 0)),
            "qkv_b": f16(torch.cat([g(f"self_attn.{x}_proj.bias") for x in "qkv"], 0)),
            "o_w": f16(g("self_attn.o_proj.weight")),
            "gate_up_w": f16(torch.cat([g("mlp.gate_proj.weight"), g("mlp.up_proj.weight")], 0)),
            "down_w": f16(g("mlp.down_proj.weight")),
        })
    return out


def vision_state_dict(sd: Dict[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
    """The vision tower's tensors under ``visual.*`` (either the raw ``visual.`` prefix or
    the ``model.visual.`` prefix of newer transformers state dicts); {} when absent."""
    out = {}
    for k, v in sd.items():
        if k.startswith("visual."):
            out[k] = v
        elif k.startswith("model.visual."):
            out[k[len("model."):]] = v
    return out


def gptq_state_dict_from_decoder(w: Dict, num_heads: int = 12, num_kv_heads: int = 2,
                                 head_dim: int = 128) -> Dict[str, torch.Tensor]:
    """Inverse of gptq_decoder_from_state_dict (AutoGPTQ key names, q/k/v and gate/up split
    along N): writes a GPTQ weight dict as the checkpoint layout the loader reads."""
    nq, nkv = num_heads * head_dim, num_kv_heads * head_dim
    sd = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["norm"]}
    for i, l in enumerate(w["layers"]):
        lp = f"model.layers.{i}."
        sd[lp + "input_layernorm.weight"] = l["in_norm"]
        sd[lp + "post_attention_layernorm.weight"] = l["post_norm"]
        bounds = {"q": (0, nq), "k": (nq, nq + nkv), "v": (nq + nkv, nq + 2 * nkv)}
        for x, (a, b) in bounds.items():
            sd[lp + f"self_attn.{x}_proj.qweight"] = l["qkv_q"][:, a:b].contiguous()
            sd[lp + f"self_attn.{x}_proj.scales"] = l["qkv_s"][:, a:b].contiguous()
            sd[lp + f"self_attn.{x}_proj.bias"] = l["qkv_b"][a:b].contiguous()
        sd[lp + "self_attn.o_proj.qweight"] = l["o_q"]
        sd[lp + "self_attn.o_proj.scales"] = l["o_s"]
        I = l["gate_up_q"].shape[1] // 2
        for x, (a, b) in {"gate": (0, I), "up": (I, 2 * I)}.items():
            sd[lp + f"mlp.{x}_proj.qweight"] = l["gate_up_q"][:, a:b].contiguous()
            sd[lp + f"mlp.{x}_proj.scales"] = l["gate_up_s"][:, a:b].contiguous()
        sd[lp + "mlp.down_proj.qweight"] = l["down_q"]
        sd[lp + "mlp.down_proj.scales"] = l["down_s"]
    return sd
