"""Shared test helpers: build the CPU oracle from the same synthetic weight dicts the
HIP path is built from, and compare logits the way the parity bar is stated
(fp16 logits max-abs <= 2e-2 and cosine >= 0.9999; argmax ids equal wherever the
oracle's top-1/top-2 margin is above the observed logit error)."""

from __future__ import annotations

import torch

from oracle import qwen2_ref as ref


def oracle_from_fp16(w, shape, f16=True, attn_p16=False) -> ref.Qwen2Ref:
    cfg = ref.Qwen2Config(hidden_size=shape.hidden_size, num_layers=len(w["layers"]),
                          num_heads=shape.num_heads, num_kv_heads=shape.num_kv_heads,
                          head_dim=shape.head_dim, intermediate_size=shape.intermediate_size,
                          vocab_size=shape.vocab_size)
    layers = [ref.LayerWeights(
        in_norm=l["in_norm"].float(), post_norm=l["post_norm"].float(),
        qkv_t=l["qkv_w"].float().t().contiguous(), qkv_b=l["qkv_b"].float(),
        o_t=l["o_w"].float().t().contiguous(), gate_up_t=l["gate_up_w"].float().t().contiguous(),
        down_t=l["down_w"].float().t().contiguous()) for l in w["layers"]]
    return ref.Qwen2Ref(cfg, w["embed"].float(), w["norm"].float(), layers, False, f16, attn_p16)


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


def oracle_stream_logits(orc: ref.Qwen2Ref, prompt, stream, max_len: int) -> torch.Tensor:
    """Teacher-forced oracle: the logits before each token of ``stream`` when the oracle is
    fed ``prompt`` and then the stream's own tokens (runners/multimodal.py:116-144 prefill,
    then :296-313 one decode step per token).  Row i decides token i.  Following the GPU's
    tokens, every step stays comparable past a near-tie (where the two may pick different
    tokens) instead of ending the comparison there."""
    cfg = orc.cfg
    kp = [torch.zeros(2, max_len, cfg.num_kv_heads, cfg.head_dim) for _ in orc.layers]
    vp = [torch.zeros_like(k) for k in kp]
    lengths = torch.zeros(2, dtype=torch.int64)
    L = len(prompt)
    emb = orc.embed[torch.tensor(prompt)]
    pos = torch.arange(L).view(1, -1).expand(3, -1)
    rows = [orc.prefill(emb, pos, [L], [0], kp, vp, lengths)[0]]
    for t in stream[:-1]:
        rows.append(orc.decode_step([int(t)], kp, vp, lengths)[0])
        lengths[0] += 1
    return torch.stack(rows)


def check_stream(stream, oracle_rows: torch.Tensor, cut: float, min_compared: int,
                 label: str = "") -> int:
    """Every token whose oracle top-1/top-2 margin exceeds ``cut`` (twice the measured
    logit error) must be the oracle's argmax; returns how many were compared, which must
    be at least ``min_compared``."""
    margin = ref.top2_margin(oracle_rows)
    want = oracle_rows.argmax(-1)
    compared = 0
    for i, g in enumerate(stream):
        if margin[i] > cut:
            compared += 1
            assert int(g) == int(want[i]), (
                f"{label} token {i}: got {g} want {int(want[i])} (margin {margin[i]:.4f} > {cut:.4f})")
    print(f"[gpu-test] {label}: {compared}/{len(stream)} tokens compared "
          f"(oracle margin > {cut:.4f})", flush=True)
    assert compared >= min_compared, (label, compared, min_compared)
    return compared


def record_sampled_logits(runner):
    """Wrap the runner's _sample_rows so a test sees the fp16 logits it samples from
    (prefill segment ends, the last chunk of a chunked prompt): returns the list they are
    appended to."""
    seen = []
    orig = runner._sample_rows

    def wrapped(logits, seqs):
        seen.append(logits.float().cpu().clone())
        return orig(logits, seqs)

    runner._sample_rows = wrapped
    return seen


def oracle_with_plan(w, shape, plan: dict, f16=True, norm_fp8=False) -> ref.Qwen2Ref:
    """The fp16 decoder's oracle with per-op precision applied as the reference's
    mixed_precision / quantize_llm_marlin would: "fp8" MLP linears take the FP8 route as
    apply_mixed builds them (per-tensor e4m3 weights, FP8Linear's default; with
    ``norm_fp8`` the gate_up is row-wise and fed by the post-attention norm's e4m3 rows,
    fuse_norm_fp8), "marlin" linears use the RTN int4 dequantised weights."""
    orc = oracle_from_fp16(w, shape, f16)
    for lw, src in zip(orc.layers, w["layers"]):
        lw.norm_fp8 = norm_fp8
        for op, key, attr in (("gate_up", "gate_up_w", "gate_up_t"), ("down", "down_w", "down_t"),
                              ("qkv", "qkv_w", "qkv_t"), ("o", "o_w", "o_t")):
            prec = plan.get(op, "fp16")
            if prec == "marlin":
                setattr(lw, attr, ref.gptq_dequant(*ref.rtn_int4(src[key].float())))
            elif prec == "fp8":
                if op not in ("gate_up", "down"):
                    raise ValueError("the oracle's FP8 route covers the MLP linears")
                rowwise = norm_fp8 and op == "gate_up"
                quant = ref.fp8_weight_rowwise if rowwise else ref.fp8_weight_pertensor
                setattr(lw, "fp8_" + op, quant(src[key].float()))
    if any(plan.get(op) == "marlin" for op in ("qkv", "o")):
        orc.bias_after_round = True
    return orc
