"""Shared test helpers: build the CPU oracle from the same synthetic weight dicts the
HIP path is built from, and compare logits the way the parity bar is stated
(fp16 logits max-abs <= 2e-2 and cosine >= 0.9999; argmax ids equal wherever the
oracle's top-1/top-2 margin is above the observed logit error)."""

from __future__ import annotations

import torch

from oracle import qwen2_ref as ref


def oracle_from_fp16(w, shape, f16=True) -> ref.Qwen2Ref:
    cfg = ref.Qwen2Config(hidden_size=shape.hidden_size, num_layers=len(w["layers"]),
                          num_heads=shape.num_heads, num_kv_heads=shape.num_kv_heads,
                          head_dim=shape.head_dim, intermediate_size=shape.intermediate_size,
                          vocab_size=shape.vocab_size)
    layers = [ref.LayerWeights(
        in_norm=l["in_norm"].float(), post_norm=l["post_norm"].float(),
        qkv_t=l["qkv_w"].float().t().contiguous(), qkv_b=l["qkv_b"].float(),
        o_t=l["o_w"].float().t().contiguous(), gate_up_t=l["gate_up_w"].float().t().contiguous(),
        down_t=l["down_w"].float().t().contiguous()) for l in w["layers"]]
    return ref.Qwen2Ref(cfg, w["embed"].float(), w["norm"].float(), layers, False, f16)


def oracle_from_gptq(w, shape, f16=True) -> ref.Qwen2Ref:
    cfg = ref.Qwen2Config(hidden_size=shape.hidden_size, num_layers=len(w["layers"]),
                          num_heads=shape.num_heads, num_kv_heads=shape.num_kv_heads,
                          head_dim=shape.head_dim, intermediate_size=shape.intermediate_size,
                          vocab_size=shape.vocab_size)
    layers = [ref.LayerWeights(
        in_norm=l["in_norm"].float(), post_norm=l["post_norm"].float(),
        qkv_t=ref.gptq_dequant(l["qkv_q"], l["qkv_s"]), qkv_b=l["qkv_b"].float(),
        o_t=ref.gptq_dequant(l["o_q"], l["o_s"]),
        gate_up_t=ref.gptq_dequant(l["gate_up_q"], l["gate_up_s"]),
        down_t=ref.gptq_dequant(l["down_q"], l["down_s"])) for l in w["layers"]]
    return ref.Qwen2Ref(cfg, w["embed"].float(), w["norm"].float(), layers, True, f16)


def compare_logits(got: torch.Tensor, exp: torch.Tensor, atol: float = 2e-2,
                   min_cos: float = 0.9999):
    got, exp = got.float().cpu(), exp.float().cpu()
    d = (got - exp).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got, exp, dim=-1).min().item()
    assert d <= atol, f"max-abs logit error {d} > {atol}"
    assert cos >= min_cos, f"cosine {cos} < {min_cos}"
    return d, cos


def check_ids(ids, exp_logits: torch.Tensor, err: float):
    """ids must equal the oracle argmax on every row whose margin exceeds 2*err."""
    exp_logits = exp_logits.float().cpu()
    ids = torch.as_tensor(ids).cpu()
    margin = ref.top2_margin(exp_logits)
    ok = margin > 2 * err + 1e-3
    want = exp_logits.argmax(-1)
    bad = (ids != want) & ok
    assert not bad.any(), f"argmax mismatch on decisive rows {bad.nonzero().flatten().tolist()}"
    return int(ok.sum())
