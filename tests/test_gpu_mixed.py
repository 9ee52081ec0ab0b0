"""Per-op precision on the GPU (kernels/mixed_precision.py, quantize_llm_marlin): linears
replaced by setattr on the reference's module paths, against the oracle with the same
plan (tests/helpers.py oracle_with_plan).

* F16Linear.dense_weight returns the nn.Linear weight bit for bit (gate|up fusion undone);
  RTN int4 of it dequantises bit-exactly to the oracle's restatement (rtn_int4).
* The MLP of both reference FP8 plans stage by stage on identical inputs: each GPU stage's
  output against the oracle applied to the GPU's own input of that stage (codes and scales
  bit for bit, SiLU-mul within a last-bit exp difference, GEMM outputs within one rounding
  step plus the MFMA's reduced intermediate precision).
* One FP8-MLP decoder (fuse_norm_fp8 + gate_up / down FP8Linear, qkv / o fp16): packed
  prefill of two prompts, logits at the segment ends against the oracle's FP8 route.
* The runner with quant="mixed" (decode through forward) and quant="marlin" (RTN int4 MLP,
  the fused hipGraph step): greedy streams teacher-forced against the oracle.

FP8 bar.  e4m3 activations (3 mantissa bits) turn the last-ulp differences any two
implementations have upstream (the fp32 order of a norm's sum of squares, of a GEMM's
sums) into whole code steps for the values near a rounding boundary, and a per-tensor
scale (the reference's default form, what apply_mixed builds) moves every code of a tensor
when its one maximum moves by an ulp.  So the arithmetic is pinned stage by stage on
identical inputs (test_fp8_mlp_stages_equal_oracle: codes and scales bit for bit), and the
model-level logits - two realisations of FP8 rounding noise seeded by different last bits
- are held to the size of that noise, measured in the same test: the GPU's max-abs distance
from the fp16-faithful FP8 oracle within 1.5 x the larger of (a) the FP8 oracle's own
spread with and without its fp16 roundings and (b) FP8's own effect on the logits (the FP8
oracle against the fp16 oracle), and its cosine deficit within 2 x the larger of theirs
(measured at the runner's first step: 0.356 against 0.370 for FP8's effect, cosine 0.9952
against 0.9946; a wrong scale or code rounding moves the logits by far more, and fails the
stage test first)."""

import pytest
import torch

from oracle import qwen2_ref as ref
from tests.helpers import (check_stream, compare_logits, oracle_stream_logits, oracle_with_plan,
                           record_sampled_logits)

pytestmark = pytest.mark.gpu

FP8_MLP = {"qkv": "fp16", "o": "fp16", "gate_up": "fp8", "down": "fp8"}


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)


def test_dense_weight_and_rtn_int4(gpu):
    from omniserver_amd import synth
    from omniserver_amd.linear import F16Linear, GPTQLinear
    say("F16Linear.dense_weight and RTN int4 (gate_up fused, down, qkv with bias)")
    for (N, K, silu, bias) in ((17920, 1536, True, False), (1536, 8960, False, False),
                               (2048, 1536, False, True)):
        W = synth.randn16((N, K), 0.02, 50, f"w{N}")
        b = synth.randn16((N,), 0.02, 51, "b") if bias else None
        lin = F16Linear(W.to(gpu), None if b is None else b.to(gpu), fuse_silu=silu)
        assert torch.equal(lin.dense_weight().cpu(), W)
        q = GPTQLinear.from_linear_rtn(lin)
        assert q.fuse_silu == silu
        eq, es = ref.rtn_int4(W.float())
        if not silu:
            assert torch.equal(q.dequantized().cpu().float(), ref.gptq_dequant(eq, es.half()))
        else:
            # the fused module's columns are gate/up tiles interleaved: compare tile by tile
            deq = q.dequantized().cpu().float().view(K, N // 16, 16)
            e = ref.gptq_dequant(eq, es.half()).view(K, 2, N // 32, 16)
            assert torch.equal(deq[:, 0::2], e[:, 0]) and torch.equal(deq[:, 1::2], e[:, 1])


def _gemm_tol(e, xq, sa, wq, sw, step):
    mag = (xq.float().abs() @ wq.float().abs().t()) * sa.view(-1, 1) * sw.reshape(1, -1)
    return e.abs() * (step + 2.0 ** -10) + mag * 2.0 ** -14 + 1e-6


@pytest.mark.parametrize("plan", ["mixed", "fused"])
def test_fp8_mlp_stages_equal_oracle(gpu, plan):
    """post_attention_layernorm + MLP (qwen2_llm.py:153-154, 123-134) under the reference's
    FP8 plans: "mixed" = apply_mixed's default (gate_up, down per-tensor FP8Linear, fp16
    norm output), "fused" = down per-tensor, then fuse_norm_fp8 (row-wise gate_up fed by
    add_rms_norm_fp8, bf16 product and SiLU-mul).  Each stage runs on the GPU and is held
    to the oracle evaluated on that stage's GPU input."""
    from omniserver_amd import fused_ops as F
    from omniserver_amd import synth
    from omniserver_amd.mixed_precision import apply_mixed, fuse_norm_fp8
    from omniserver_amd.qwen2_llm import Qwen2LLM
    say(f"FP8 MLP stages, plan {plan}")
    shape = synth.DecoderShape()
    w = synth.fp16_decoder(shape, seed=23, num_layers=1)
    model = Qwen2LLM.from_fp16(w, shape, gpu, max_pos=256)
    if plan == "mixed":
        apply_mixed(model)
    else:
        apply_mixed(model, {"qkv": "fp16", "o": "fp16", "gate_up": "fp16", "down": "fp8"})
        fuse_norm_fp8(model)
    lay = model.layers[0]
    gu_lin, dn_lin = lay.mlp.gate_up_proj, lay.mlp.down_proj
    assert gu_lin.rowwise == (plan == "fused") and not dn_lin.rowwise
    src = w["layers"][0]
    gu_w = (ref.fp8_weight_rowwise if plan == "fused" else ref.fp8_weight_pertensor)(
        src["gate_up_w"].float())
    dn_w = ref.fp8_weight_pertensor(src["down_w"].float())
    assert torch.equal(gu_lin.weight_fp8.cpu(), gu_w[0].view(torch.uint8))
    assert torch.equal(dn_lin.weight_fp8.cpu(), dn_w[0].view(torch.uint8))
    M, H = 48, shape.hidden_size
    g = torch.Generator().manual_seed(24)
    o = (torch.randn(M, H, generator=g) * 0.5).half()
    res = torch.randn(M, H, generator=g).half()
    norm_out, nres = lay.post_attention_layernorm(o.to(gpu), res.to(gpu))
    _, er = ref.add_rms_norm(o.float(), res.float(), lay.post_norm.cpu().float(), 1e-6)
    assert torch.equal(nres.cpu().float(), er)
    if plan == "fused":
        xq_g, sa_g = norm_out
        eq, es, _ = ref.add_rms_norm_fp8(o.float(), res.float(), lay.post_norm.cpu().float(), 1e-6)
        same = (xq_g.cpu().view(torch.uint8) == eq.view(torch.uint8)).float().mean().item()
        assert same > 0.999 and torch.allclose(sa_g.cpu(), es, rtol=2e-6), same
        gu = gu_lin.forward_prequant(xq_g, sa_g)
        xq, sa = xq_g.cpu().view(torch.float8_e4m3fn), sa_g.cpu()
        e = ref.fp8_linear_prequant(xq, sa, *gu_w)
        step = 2.0 ** -7
    else:
        gu = gu_lin(norm_out)
        xq_g, sa_g = gu_lin.quantize_input(norm_out)
        xq, sa = ref.quant_fp8_pertensor(norm_out.cpu().float())
        assert torch.equal(xq_g.cpu(), xq.view(torch.uint8))
        assert torch.equal(sa_g.cpu().view(-1), sa.expand(M))
        e = ref.fp8_linear_pertensor(xq, sa, *gu_w)
        sa = sa.expand(M)
        step = 2.0 ** -10
    d = (gu.cpu().float() - e).abs()
    assert (d <= _gemm_tol(e, xq, sa, *gu_w, step)).all(), "gate_up"
    act = F.silu_mul(gu)
    gc = gu.cpu().float()
    n = gc.shape[-1] // 2
    e_act = gc[:, :n] * torch.sigmoid(gc[:, :n]) * gc[:, n:]
    e_act = ref.rbf16(e_act) if plan == "fused" else ref.r16(e_act)
    assert act.dtype == (torch.bfloat16 if plan == "fused" else torch.float16)
    # the device's exp and torch's may differ in the last fp32 bit: one step of the stored
    # type on a near-tie, nearly every element bit-equal
    da = (act.cpu().float() - e_act).abs()
    assert (da <= e_act.abs() * (2.0 ** -7 if plan == "fused" else 2.0 ** -10) + 2.0 ** -24).all()
    assert (da == 0).float().mean().item() > 0.999, "silu_mul"
    y = dn_lin(act)
    xq_g, sa_g = dn_lin.quantize_input(act)
    xq, sa = ref.quant_fp8_pertensor(act.cpu().float(), bf16=plan == "fused")
    assert torch.equal(xq_g.cpu(), xq.view(torch.uint8)), "down codes"
    e = ref.fp8_linear_pertensor(xq, sa, *dn_w)
    d = (y.cpu().float() - e).abs()
    assert (d <= _gemm_tol(e, xq, sa.expand(M), *dn_w, 2.0 ** -10)).all(), "down"
    torch.cuda.synchronize()


def test_fp8_mlp_decoder_prefill(gpu):
    from omniserver_amd import synth
    from omniserver_amd.linear import FP8Linear
    from omniserver_amd.kv_cache import PreallocatedKVCache
    from omniserver_amd.mixed_precision import apply_mixed, fuse_norm_fp8
    from omniserver_amd.qwen2_llm import Qwen2LLM
    say("decoder with FP8 MLP (fuse_norm_fp8 + plan), 2 layers, packed prefill 150 + 100")
    shape = synth.DecoderShape()
    w = synth.fp16_decoder(shape, seed=21, num_layers=2)
    model = Qwen2LLM.from_fp16(w, shape, gpu, max_pos=1024)
    assert fuse_norm_fp8(model) == 2
    counts = apply_mixed(model, FP8_MLP)
    assert counts["down"] == ("fp8", 2) and counts["gate_up"] == ("fp8", 0)   # already FP8
    assert model.layers[0].post_attention_layernorm.fp8_out
    assert isinstance(model.layers[1].mlp.gate_up_proj, FP8Linear)
    assert model.layers[1].mlp.gate_up_proj.rowwise and not model.layers[1].mlp.down_proj.rowwise
    assert not model.fused_decode_ready()
    # the reference refuses to fuse the norm into a per-tensor gate_up
    other = Qwen2LLM.from_fp16(w, shape, gpu, max_pos=1024)
    apply_mixed(other)
    with pytest.raises(ValueError):
        fuse_norm_fp8(other)
    del other
    wq, _ = ref.fp8_weight_rowwise(w["layers"][0]["gate_up_w"].float())
    assert torch.equal(model.layers[0].mlp.gate_up_proj.weight_fp8.cpu(), wq.view(torch.uint8))
    segs = [150, 100]
    ids = [synth.random_ids(L, shape.vocab_size, 21, f"f{L}") for L in segs]
    emb = torch.cat([w["embed"][i] for i in ids], 0)
    pos = torch.cat([torch.arange(L).view(1, -1).expand(3, -1) for L in segs], 1)
    pool = PreallocatedKVCache(2, 3, 2, 256, 128, gpu, n_heads=12)
    cache = pool.packed_prefill_cache([0, 1], segs)
    last = [segs[0] - 1, sum(segs) - 1]
    logits = model(emb.to(gpu).unsqueeze(0), pos.to(gpu).unsqueeze(1), None, cache,
                   logits_indices=last)[0]
    torch.cuda.synchronize()
    exps = []
    for plan, f16 in ((FP8_MLP, True), (FP8_MLP, False), ({}, True)):
        orc = oracle_with_plan(w, shape, plan, f16=f16, norm_fp8=bool(plan))
        kp = [torch.zeros(3, 256, 2, 128) for _ in range(2)]
        vp = [torch.zeros(3, 256, 2, 128) for _ in range(2)]
        exps.append(orc.prefill(emb.float(), pos, segs, [0, 1], kp, vp,
                                torch.zeros(3, dtype=torch.int64)))
    fp8_check(logits, exps[0], exps[1], "FP8 MLP prefill", exps[2])


def fp8_check(got, e16, e32, label, efp16=None):
    """The FP8 bar of the module docstring (e16 / e32: the FP8 oracle with / without the
    fp16 storage roundings); returns the GPU's max-abs distance from e16."""
    cos = lambda a, b: torch.nn.functional.cosine_similarity(a, b, dim=-1).min().item()
    g = got.float().cpu()
    d = (g - e16).abs().max().item()
    spread = (e16 - e32).abs().max().item()
    c, cs = cos(g, e16), cos(e16, e32)
    extra, noise, cdef = "", spread, 1 - cs
    if efp16 is not None:
        eff, ce = (e16 - efp16).abs().max().item(), cos(e16, efp16)
        noise, cdef = max(noise, eff), max(cdef, 1 - ce)
        extra = (f"; FP8's own effect (fp8 oracle vs fp16 oracle) max-abs {eff:.4f} cos "
                 f"{ce:.6f}; gpu vs fp16 oracle {(g - efp16).abs().max().item():.4f} cos "
                 f"{cos(g, efp16):.6f}")
    say(f"  {label}: gpu-fp8oracle max-abs {d:.4f} cos {c:.6f}; the FP8 oracle's own rounding "
        f"spread max-abs {spread:.4f} cos {cs:.6f}{extra}")
    assert d <= 1.5 * noise, (d, noise)
    assert 1 - c <= 2 * cdef + 1e-6, (c, cdef)
    return d


@pytest.mark.parametrize("quant", ["mixed", "marlin"])
def test_runner_quant_plans(gpu, quant):
    from omniserver_amd import synth
    from omniserver_amd.request import Request, SamplingParams, Sequence
    from omniserver_amd.runner import NativeQwenVLRunner
    say(f"runner quant={quant!r}, 3 layers, greedy, hipGraph where the step allows it")
    shape = synth.DecoderShape()
    w = synth.fp16_decoder(shape, seed=22, num_layers=3)
    runner = NativeQwenVLRunner(max_running=2, max_len=256, use_graph=True, quant=quant,
                                weights=w)
    model = runner.adapter.model
    assert model.fused_decode_ready() == (quant == "marlin")
    seen = record_sampled_logits(runner)
    prompts = [synth.random_ids(L, shape.vocab_size, 22, f"r{L}").tolist() for L in (33, 20)]
    seqs = [Sequence(Request(prompt=p, sampling=SamplingParams(max_new_tokens=7))) for p in prompts]
    for s in seqs:
        runner.tokenize(s)
    runner.prefill(seqs)
    for _ in range(6):
        runner.decode(seqs)
    plan = {"gate_up": "marlin", "down": "marlin"} if quant == "marlin" else FP8_MLP
    orc = oracle_with_plan(w, shape, plan)
    rows = [oracle_stream_logits(orc, p, s.output_token_ids, 256) for p, s in zip(prompts, seqs)]
    first = torch.stack([r[0] for r in rows])
    if quant == "mixed":
        # FP8's own spread (~0.24) exceeds nearly every top-2 margin, so instead of token
        # identity every step's logits (prefill and the 6 decode steps through forward, all
        # handed to _sample_rows) are held to the FP8 bar against the teacher-forced oracle
        o32 = oracle_with_plan(w, shape, plan, f16=False)
        rows32 = [oracle_stream_logits(o32, p, s.output_token_ids, 256)
                  for p, s in zip(prompts, seqs)]
        o16 = oracle_with_plan(w, shape, {})
        rows16 = [oracle_stream_logits(o16, p, s.output_token_ids, 256)
                  for p, s in zip(prompts, seqs)]
        assert len(seen) == 7
        err = 0.0
        for i, got in enumerate(seen):
            err = max(err, fp8_check(got, torch.stack([r[i] for r in rows]),
                                     torch.stack([r[i] for r in rows32]), f"mixed step {i}",
                                     torch.stack([r[i] for r in rows16])))
        need = 0
    else:
        err, cos = compare_logits(seen[0], first)
        say(f"  prefill logits max-abs {err:.4f}, cos {cos:.6f}")
        need = 7
    total = sum(check_stream(s.output_token_ids, r, 2 * err + 1e-3, 0, f"{quant} seq {b}")
                for b, (s, r) in enumerate(zip(seqs, rows)))
    assert total >= need, total
