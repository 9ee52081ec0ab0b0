"""Pins the oracle's FP8 W8A8 functions and MLP routes (oracle/qwen2_ref.py) against the
reference's own modules, CPU only.

tests/golden/ref_fp8_route.npz holds what omniserve's FP8Linear (kernels/fp8_linear.py:
66-126, both weight forms), _quant_fp8_pertensor's eager branch (:40-41), apply_mixed /
fuse_norm_fp8 (kernels/mixed_precision.py:53-84), RMSNorm.forward with fp8_out and
MLP.forward (model/qwen2_llm.py:46-56, 123-134) produced on the seeded cases of
tests/golden/fp8_case.py and composition_case.py, run on the CPU by
tests/golden/make_ref_vit_fp8.py (Triton quant / norm / SiLU kernels as torch
evaluations of their formulas; row-wise _scaled_mm as fp32 accumulation times the
scales; per-tensor _scaled_mm is torch's own CPU routine).

1. Linear level, bit for bit: the weight codes and scales of both forms (the row-wise
   scale is an op on the reference's fp16 weight, so fp16-rounded), the per-tensor and
   per-token activation codes and scales (fp16 and bf16 inputs), forward with and
   without bias in both forms, forward_prequant.
2. The two FP8 plans inside the composition case's decoder: which linears become FP8 in
   which form; layer 0's gate_up, SiLU-mul and down outputs from the reference's own
   stage inputs, bit for bit (prefill and decode); the logits within the FP8 noise the
   attention's rounding seeds (the oracle's exact softmax against torch's fp16 SDPA).
3. Planted mistakes in the oracle (fp32 weight scales, the fused route's SiLU rounded to
   fp16 instead of bf16, the per-tensor activation scale taken per token, a bf16 rounding
   of the per-tensor product) each fail one of the checks above.
"""

import os
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import qwen2_ref as ref

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
sys.path.insert(0, GOLDEN)
sys.path.insert(0, HERE)
import composition_case as C  # noqa: E402
import fp8_case as P  # noqa: E402

E4M3 = torch.float8_e4m3fn


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(GOLDEN, "ref_fp8_route.npz"))


def _codes(q):
    return q.view(torch.uint8).numpy()


# ----------------------------------------------------------------------------- linear level
def linear_checks(g):
    """Every linear-level comparison; returns the names of those that differ."""
    w, b, x = P.linear_case()
    bad = []
    eq = lambda name, got, want: bad.append(name) if not np.array_equal(got, want) else None
    wt, st = ref.fp8_weight_pertensor(w)
    wr, sr = ref.fp8_weight_rowwise(w)
    eq("pt_wq", _codes(wt), g["pt_wq"])
    eq("pt_wscale", st.reshape(-1).numpy(), g["pt_wscale"])
    eq("rw_wq", _codes(wr), g["rw_wq"])
    eq("rw_wscale", sr.numpy(), g["rw_wscale"])
    xq, sa = ref.quant_fp8_pertensor(x)
    eq("pt_xq", _codes(xq), g["pt_xq"])
    eq("pt_xscale", sa.reshape(-1).numpy(), g["pt_xscale"])
    xb = ref.rbf16(x)
    xqb, sab = ref.quant_fp8_pertensor(xb, bf16=True)
    eq("pt_xq_bf16", _codes(xqb), g["pt_xq_bf16"])
    eq("pt_xscale_bf16", sab.reshape(-1).numpy(), g["pt_xscale_bf16"])
    xr, sx = ref.quant_fp8(x)
    eq("rw_xq", _codes(xr), g["rw_xq"])
    eq("rw_xscale", sx.numpy(), g["rw_xscale"])
    eq("pt_out", ref.fp8_linear_pertensor(xq, sa, wt, st, b).numpy(), g["pt_out"])
    eq("pt_out_nobias", ref.fp8_linear_pertensor(xq, sa, wt, st).numpy(), g["pt_out_nobias"])
    eq("pt_out_bf16in", ref.fp8_linear_pertensor(xqb, sab, wt, st, b).numpy(), g["pt_out_bf16in"])
    eq("rw_out", ref.fp8_linear_rowwise(xr, sx, wr, sr, b).numpy(), g["rw_out"])
    eq("rw_out_nobias", ref.fp8_linear_rowwise(xr, sx, wr, sr).numpy(), g["rw_out_nobias"])
    xrb, sxb = ref.quant_fp8(xb)
    eq("rw_out_bf16in", ref.fp8_linear_rowwise(xrb, sxb, wr, sr, b).numpy(), g["rw_out_bf16in"])
    eq("rw_prequant", ref.fp8_linear_prequant(xr, sx, wr, sr, b).numpy(), g["rw_prequant"])
    # the fp16-input forward through the dispatching helper takes the same arithmetic
    eq("fp8_linear(pt)", (ref.fp8_linear(x, (wt, st)) + 0).numpy(), g["pt_out_nobias"])
    return bad


def test_linear_level_bit_exact(golden):
    assert linear_checks(golden) == []


# ----------------------------------------------------------------------------- MLP routes
def route_oracle(plan: str, f16=True):
    """The composition case's oracle with the reference's FP8 plan applied: "mixed" =
    apply_mixed's default plan (gate_up, down per-tensor); "fused" = down per-tensor, then
    fuse_norm_fp8 (gate_up row-wise, fed by the post-attention norm's e4m3 rows)."""
    import test_oracle_composition as TC
    orc = TC._case_oracle(f16)
    for lw, l in zip(orc.layers, C.weights()["layers"]):
        lw.fp8_down = ref.fp8_weight_pertensor(l["down_w"])
        if plan == "mixed":
            lw.fp8_gate_up = ref.fp8_weight_pertensor(l["gate_up_w"])
        else:
            lw.fp8_gate_up = ref.fp8_weight_rowwise(l["gate_up_w"])
            lw.norm_fp8 = True
    return orc


def route_stage_checks(g, plan):
    """Layer 0's MLP stages from the reference's own inputs; returns the names of the
    stages whose output differs beyond one fp16 / bf16 ulp on any element."""
    lw = route_oracle(plan).layers[0]
    bad = []
    for tag in ("prefill", "decode"):
        t = lambda k: torch.tensor(g[f"{plan}_l0_{tag}_{k}"])
        want_gu, want_act, want_out = t("gate_up"), t("act"), t("mlp_out")
        if plan == "mixed":
            gu = ref.fp8_linear(t("mlp_in"), lw.fp8_gate_up)
            act = ref.silu_mul(want_gu)
            out = ref.fp8_linear(want_act, lw.fp8_down)
        else:
            mi = t("mlp_in")                       # (e4m3 rows | scale column)
            gu = ref.fp8_linear_prequant(mi[:, :-1].to(E4M3), mi[:, -1:], *lw.fp8_gate_up)
            n = want_gu.shape[-1] // 2
            g_, u_ = want_gu[:, :n], want_gu[:, n:]
            act = ref.rbf16(g_ * torch.sigmoid(g_) * u_)
            out = ref.fp8_linear(want_act, lw.fp8_down, bf16_in=True)
        for name, got, want, step in (("gate_up", gu, want_gu, 2.0 ** -7),
                                      ("act", act, want_act, 2.0 ** -7),
                                      ("mlp_out", out, want_out, 2.0 ** -10)):
            d = (got - want).abs()
            # one ulp of the stored type, and at most 1 % of the elements not bit-equal
            # (the oracle's fp32 GEMM sums in another order than the CPU library's)
            if (d > want.abs() * step + 1e-6).any() or (d > 0).float().mean() > 0.01:
                bad.append(f"{tag}:{name}")
    return bad


@pytest.mark.parametrize("plan", list(P.PLANS))
def test_plan_weight_forms(golden, plan):
    lw = route_oracle(plan).layers[0]
    for op, w in (("gate_up_proj", lw.fp8_gate_up), ("down_proj", lw.fp8_down)):
        assert int(golden[f"{plan}_{op}_rowwise"]) == int(w[1].dim() == 1), op
        assert np.array_equal(w[1].reshape(-1).numpy(), golden[f"{plan}_{op}_wscale"]), op


@pytest.mark.parametrize("plan", list(P.PLANS))
def test_route_stages_match_reference(golden, plan):
    assert route_stage_checks(golden, plan) == []


def _route_logits(plan):
    import test_oracle_composition as TC
    pre, dec, *_ = TC._run_case(route_oracle(plan))
    return pre, dec


def logits_error(g, plan):
    pre, dec = _route_logits(plan)
    err, cos_min, wrong = 0.0, 1.0, 0
    for got, want in ((pre, g[f"{plan}_prefill_logits"]), (dec, g[f"{plan}_decode_logits"])):
        want = torch.tensor(want)
        err = max(err, (got - want).abs().max().item())
        cos_min = min(cos_min, F.cosine_similarity(got.reshape(-1, C.VOCAB),
                                                   want.reshape(-1, C.VOCAB), -1).min().item())
        decisive = ref.top2_margin(want) > 0.5
        wrong += int((got.argmax(-1) != want.argmax(-1))[decisive].sum())
    return err, cos_min, wrong


@pytest.mark.parametrize("plan", list(P.PLANS))
def test_route_logits_match_reference(golden, plan):
    """Whole decoder under the plan.  The stages above agree bit for bit; what separates
    the logits is the attention (exact softmax here, torch's fp16 CPU SDPA in the
    fixture: ~5e-3 on the fp16 decoder's logits), which moves a few activations across
    e4m3 rounding boundaries and per-tensor scales by an ulp (measured 0.15-0.17 max-abs
    on logits of magnitude ~3.6, where FP8 itself moves them by 0.25-0.28 from fp16)."""
    err, cos_min, wrong = logits_error(golden, plan)
    assert err <= 0.25 and cos_min >= 0.998 and wrong == 0, (err, cos_min, wrong)


# ----------------------------------------------------------------------------- planted mistakes
def _fp32_weight_scales(mp):
    mp.setattr(ref, "fp8_weight_rowwise", lambda w: (
        (w / (w.abs().amax(1, keepdim=True) / 448.0)).to(E4M3), (w.abs().amax(1) / 448.0)))
    mp.setattr(ref, "fp8_weight_pertensor", lambda w: (
        (w / (w.abs().max() / 448.0)).to(E4M3), w.abs().max() / 448.0))


def _pertensor_scale_per_token(mp):
    def bad(x, bf16=False):
        rd = ref.rbf16 if bf16 else ref.r16
        sa = rd(x.abs().amax(-1, keepdim=True) / 448.0)
        return rd(x / sa).to(E4M3), sa
    mp.setattr(ref, "quant_fp8_pertensor", bad)


def _pertensor_bf16_product(mp):
    def bad(xq, sa, wq, sw, bias=None):
        y = ref.r16(ref.rbf16((xq.float() @ wq.float().t()) * sa * sw))
        return y if bias is None else ref.r16(y + bias)
    mp.setattr(ref, "fp8_linear_pertensor", bad)


MISTAKES = {"fp32_weight_scales": _fp32_weight_scales,
            "pertensor_scale_per_token": _pertensor_scale_per_token,
            "pertensor_bf16_product": _pertensor_bf16_product}


@pytest.mark.parametrize("mistake", list(MISTAKES))
def test_planted_mistake_is_caught(mistake, monkeypatch, golden):
    MISTAKES[mistake](monkeypatch)
    caught = linear_checks(golden)
    for plan in P.PLANS:
        caught += route_stage_checks(golden, plan)
    assert caught, f"planted mistake {mistake} passed every check"


def test_planted_fused_silu_in_fp16_is_caught(golden):
    """The fused route's silu_mul stores in its input dtype, bf16 (fused_ops.py:122-130):
    rounding it to fp16 instead changes the stage."""
    lw = route_oracle("fused").layers[0]
    want_gu = torch.tensor(golden["fused_l0_prefill_gate_up"])
    n = want_gu.shape[-1] // 2
    act16 = ref.silu_mul(want_gu)                               # fp16 rounding
    want = torch.tensor(golden["fused_l0_prefill_act"])
    assert not torch.equal(act16, want)
    assert torch.equal(ref.rbf16(want_gu[:, :n] * torch.sigmoid(want_gu[:, :n]) * want_gu[:, n:]),
                       want)
    assert lw.norm_fp8


def test_fused_norm_rejects_a_pertensor_gate_up():
    """fuse_norm_fp8 raises for a per-tensor gate_up (mixed_precision.py:69-70); the
    oracle refuses the combination the same way."""
    orc = route_oracle("mixed")
    lw = orc.layers[0]
    lw.norm_fp8 = True
    x = torch.randn(2, C.HIDDEN).half().float()
    with pytest.raises(ValueError):
        orc._post_norm_mlp(x, x, lw)
