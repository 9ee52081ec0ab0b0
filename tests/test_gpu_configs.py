"""BASELINE.json configs at their real sizes on the GPU, against the CPU oracle.

* config 3 (the north star): W4A16 GPTQ decoder, all 28 layers, B = 32, 2048-token
  contexts in a [33, 4096, 2, 128] pool: one decode step's logits against both oracle
  modes (fp16-faithful and exact fp32), row by row (_full_depth_check: the 2e-2 bar
  against the exact result wherever the reference's own fp16 rounding sequence meets it),
  greedy ids equal on every row whose margin exceeds twice the measured error.
* config 1: fp16 decoder, 28 layers, B = 1, a 256-token prompt, prefill then 32 greedy
  steps through the hipGraph runner; every emitted token is checked against the oracle fed
  the same tokens (teacher forcing), wherever the oracle's margin exceeds twice the
  measured prefill logit error.
* config 2: fp16 decoder, 28 layers, B = 16, contexts U[512, 2048] in a [17, 4096, 2, 128]
  pool: one decode step, checked as config 3.
* config 5: 8 image + text prompts (64 text, 256 N(0,1) vision rows, 192 text) packed into
  T = 4096 rows with 3-D M-RoPE positions, prefill (the pipelined GEMMs at M = 4096 and the
  block-diagonal causal attention) then 8 greedy int4 decode steps at B = 8, on 2 layers
  so that the oracle's T = 4096 prefill takes seconds.

Each test prints what it compared (errors, counts)."""

import pytest
import torch

from oracle import qwen2_ref as ref
from tests.helpers import (check_ids, check_stream, compare_logits, oracle_from_fp16,
                           oracle_from_gptq, oracle_stream_logits, record_sampled_logits)

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)


def _fill_pool_device(pool, lengths, seed, gpu):
    """N(0, 1) fp16 K/V prefixes generated on the device (seeded), each row up to its
    length; returns fp32 CPU copies sized to the lengths (+ room for the new token)."""
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    B = len(lengths)
    Lc = max(lengths) + 2
    kp, vp = [], []
    for l in range(pool.n_layers):
        ks = torch.zeros(B + 1, Lc, pool.n_kv_heads, pool.head_dim)
        vs = torch.zeros_like(ks)
        for b, L in enumerate(lengths):
            pool.k[l][b, :L].normal_(generator=g)
            pool.v[l][b, :L].normal_(generator=g)
            ks[b, :L] = pool.k[l][b, :L].float().cpu()
            vs[b, :L] = pool.v[l][b, :L].float().cpu()
        kp.append(ks)
        vp.append(vs)
    pool.lengths[:B] = torch.tensor(lengths, device=gpu)
    return kp, vp


def _full_depth_check(logits, out, e16, e32, label):
    """Full-depth logits against both oracle modes.  The fp16-faithful oracle (the
    reference's storage roundings, exact attention) is itself ``noise`` away from the exact
    fp32 result: at 28 layers of fp16 weights ~2e-2 on every row, with int4 weights a few
    1e-3 except on rows whose values sit near rounding boundaries.  The GPU's computation
    order (fp32 accumulation order, attention probabilities rounded to fp16 as the
    reference's flash path rounds them) is another sample of the same rounding noise, so it
    can be as far from the fp16 oracle as both are from exact.  Bar: the GPU's distance from
    the exact result within max(2e-2, 1.5 x the largest noise of the batch) on every row and
    its median over rows within 1.25 x the oracle's median noise (+1e-3): it is no noisier
    than the reference's own rounding sequence.  Cosine >= 0.9999 against both modes;
    greedy ids equal the exact argmax where its margin exceeds twice the GPU's error.  The
    distance from the fp16 oracle and the rows within 2e-2 of it are printed."""
    g = logits.float().cpu()
    d16 = (g - e16).abs().max(1).values
    d32 = (g - e32).abs().max(1).values
    noise = (e16 - e32).abs().max(1).values
    cos = lambda a, b: torch.nn.functional.cosine_similarity(a, b, dim=-1).min().item()
    c16, c32 = cos(g, e16), cos(g, e32)
    bar = max(2e-2, 1.5 * noise.max().item())
    say(f"{label}: max-abs gpu-f16oracle {d16.max():.4f} (rows within 2e-2: "
        f"{int((d16 <= 2e-2).sum())}/{len(d16)}), gpu-f32 {d32.max():.4f} (median "
        f"{d32.median():.4f}), f16oracle-f32 {noise.max():.4f} (median {noise.median():.4f}); "
        f"cos {c16:.6f} / {c32:.6f}")
    assert c16 >= 0.9999 and c32 >= 0.9999, (c16, c32)
    assert (d32 <= bar).all(), (d32.max().item(), bar)
    assert d32.median() <= 1.25 * noise.median() + 1e-3, (d32.median(), noise.median())
    decisive = check_ids(out, e32, d32.max().item())
    say(f"{label}: greedy ids equal on {decisive}/{len(d16)} decisive rows")
    return decisive


def _one_step(gpu, model, pool, orc, lengths, ids, label):
    n = len(lengths)
    out = torch.empty(n, dtype=torch.int64, device=gpu)
    logits = torch.empty(n, model.cfg.vocab_size, dtype=torch.float16, device=gpu)
    model.decode_greedy(ids.to(gpu), pool.view(n, None), out, logits)
    torch.cuda.synchronize()
    return out, logits


def test_config3_full_step(gpu):
    from omniserver_amd import synth
    from omniserver_amd.kv_cache import PreallocatedKVCache
    from omniserver_amd.qwen2_llm import Qwen2LLM
    B, ctx = 32, 2048
    say(f"config 3: int4, 28 layers, B={B}, ctx {ctx}, pool [{B + 1}, 4096, 2, 128]")
    shape = synth.DecoderShape()
    w = synth.gptq_decoder(shape, seed=0)
    model = Qwen2LLM.from_gptq(w, shape, gpu, max_pos=8192)
    pool = PreallocatedKVCache(28, B + 1, 2, 4096, 128, gpu, n_heads=12)
    lengths = [ctx] * B
    kp, vp = _fill_pool_device(pool, lengths, 31, gpu)
    ids = synth.random_ids(B, shape.vocab_size, 0, "c3ids")
    out, logits = _one_step(gpu, model, pool, None, lengths, ids, "config 3")
    lens = torch.tensor(lengths + [0])
    e32 = oracle_from_gptq(w, shape, f16=False).decode_step(
        ids.tolist(), [k.clone() for k in kp], [v.clone() for v in vp], lens.clone())
    orc = oracle_from_gptq(w, shape, f16=True)
    del w
    e16 = orc.decode_step(ids.tolist(), kp, vp, lens.clone())
    # the new K/V rows of the first layer (before any depth has accumulated) and the last
    dk0 = (pool.k[0][:B, ctx].float().cpu() - kp[0][:B, ctx]).abs().max().item()
    assert dk0 <= 2e-2, dk0
    for l in (0, 27):
        dk = (pool.k[l][:B, ctx].float().cpu() - kp[l][:B, ctx]).abs().max().item()
        dv = (pool.v[l][:B, ctx].float().cpu() - vp[l][:B, ctx]).abs().max().item()
        say(f"config 3: layer {l} new K/V rows max-abs {dk:.4f} / {dv:.4f}")
    decisive = _full_depth_check(logits, out, e16, e32, "config 3")
    assert decisive >= B // 2


def test_config1_greedy_32_steps(gpu):
    from omniserver_amd import synth
    from omniserver_amd.request import Request, SamplingParams, Sequence
    from omniserver_amd.runner import NativeQwenVLRunner
    say("config 1: fp16, 28 layers, B=1, 256-token prompt, 32 greedy steps (hipGraph runner)")
    shape = synth.DecoderShape()
    w = synth.fp16_decoder(shape, seed=1)
    prompt = synth.random_ids(256, shape.vocab_size, 1, "c1").tolist()
    runner = NativeQwenVLRunner(max_running=1, max_len=1024, use_graph=True, weights=w)
    seen = record_sampled_logits(runner)
    seq = Sequence(Request(prompt=prompt, sampling=SamplingParams(max_new_tokens=33)))
    runner.tokenize(seq)
    runner.prefill([seq])
    for _ in range(32):
        runner.decode([seq])
    stream = seq.output_token_ids
    assert len(stream) == 33
    del runner
    torch.cuda.empty_cache()
    orc = oracle_from_fp16(w, shape, f16=True)
    rows = oracle_stream_logits(orc, prompt, stream, 320)
    err, cos = compare_logits(seen[0], rows[0:1])
    say(f"config 1: prefill logits max-abs {err:.4f} (bar 2e-2), cos {cos:.6f}")
    check_stream(stream, rows, 2 * err + 1e-3, 24, "config 1 greedy stream")


def test_config2_ragged_step(gpu):
    from omniserver_amd import synth
    from omniserver_amd.kv_cache import PreallocatedKVCache
    from omniserver_amd.qwen2_llm import Qwen2LLM
    B = 16
    lengths = synth.context_lengths(B, 512, 2048, 2).tolist()
    say(f"config 2: fp16, 28 layers, B={B}, contexts U[512, 2048] {lengths[:4]}..")
    shape = synth.DecoderShape()
    w = synth.fp16_decoder(shape, seed=1)
    model = Qwen2LLM.from_fp16(w, shape, gpu, max_pos=8192)
    pool = PreallocatedKVCache(28, B + 1, 2, 4096, 128, gpu, n_heads=12)
    kp, vp = _fill_pool_device(pool, lengths, 32, gpu)
    ids = synth.random_ids(B, shape.vocab_size, 2, "c2ids")
    out, logits = _one_step(gpu, model, pool, None, lengths, ids, "config 2")
    lens = torch.tensor(lengths + [0])
    e32 = oracle_from_fp16(w, shape, f16=False).decode_step(
        ids.tolist(), [k.clone() for k in kp], [v.clone() for v in vp], lens.clone())
    e16 = oracle_from_fp16(w, shape, f16=True).decode_step(ids.tolist(), kp, vp, lens.clone())
    del w
    decisive = _full_depth_check(logits, out, e16, e32, "config 2")
    assert decisive >= B // 2


def test_config5_packed_prefill_and_decode(gpu):
    from omniserver_amd import synth
    from omniserver_amd.positions import IMAGE_TOKEN_ID, VISION_START_TOKEN_ID
    from omniserver_amd.request import Request, SamplingParams, Sequence, VisionInput
    from omniserver_amd.runner import NativeQwenVLRunner
    B, layers, steps = 8, 2, 8
    say(f"config 5: int4, {layers} layers, 8 x [64 text | 256 image rows | 192 text] packed "
        f"prefill T={512 * B}, then {steps} greedy steps at B={B}")
    shape = synth.DecoderShape()
    w = synth.gptq_decoder(shape, seed=5, num_layers=layers)
    prompts, rows = [], []
    for b in range(B):
        ids = (synth.random_ids(63, shape.vocab_size, 5, f"c5a.{b}").tolist()
               + [VISION_START_TOKEN_ID] + [IMAGE_TOKEN_ID] * 256
               + synth.random_ids(192, shape.vocab_size, 5, f"c5b.{b}").tolist())
        prompts.append(ids)
        rows.append(synth.randn16((256, shape.hidden_size), 1.0, 5, f"c5v.{b}"))
    runner = NativeQwenVLRunner(max_running=B, max_len=1024, use_graph=True, quant="gptq",
                                weights=w)
    seen = record_sampled_logits(runner)
    seqs = [Sequence(Request(prompt=p, sampling=SamplingParams(max_new_tokens=steps + 1),
                             images=[VisionInput(r.to(gpu), (1, 32, 32))]))
            for p, r in zip(prompts, rows)]
    for s in seqs:
        runner.tokenize(s)
    runner.prefill(seqs)
    k_gpu = [runner.pool.k[l][:B, :512].float().cpu() for l in range(layers)]
    for _ in range(steps):
        runner.decode(seqs)
    streams = [s.output_token_ids for s in seqs]

    # oracle: the same packed prefill (positions from the reference's rule), then decode
    # steps fed the GPU's tokens
    orc = oracle_from_gptq(w, shape, f16=True)
    embs, poss, deltas = [], [], []
    for ids, r in zip(prompts, rows):
        pos, d = ref.mrope_position_ids(ids, [(1, 32, 32)], image_token_id=IMAGE_TOKEN_ID,
                                        vision_start_id=VISION_START_TOKEN_ID)
        e = orc.embed[torch.tensor(ids)].clone()
        e[torch.tensor(ids) == IMAGE_TOKEN_ID] = r.float()
        embs.append(e)
        poss.append(pos)
        deltas.append(int(d))
    assert deltas == [-240] * B          # t = 64, h/w = 64 + 0..15, text resumes at 80
    kp = [torch.zeros(B + 1, 512 + steps + 2, 2, 128) for _ in range(layers)]
    vp = [torch.zeros_like(k) for k in kp]
    lens = torch.zeros(B + 1, dtype=torch.int64)
    lg = orc.prefill(torch.cat(embs, 0), torch.cat(poss, 1), [512] * B, list(range(B)), kp, vp, lens)
    err, cos = compare_logits(seen[0], lg)
    say(f"config 5: prefill logits max-abs {err:.4f}, cos {cos:.6f}")
    for l in range(layers):
        dk = (k_gpu[l] - kp[l][:B, :512]).abs().max().item()
        assert dk <= 2e-2, (l, dk)
    cut = 2 * err + 1e-3
    oracle_rows = [[lg[b]] for b in range(B)]
    delta = torch.tensor(deltas + [0])
    for i in range(steps):
        lg = orc.decode_step([streams[b][i] for b in range(B)], kp, vp, lens, delta)
        lens[:B] += 1
        for b in range(B):
            oracle_rows[b].append(lg[b])
    total = 0
    for b in range(B):
        total += check_stream(streams[b], torch.stack(oracle_rows[b]), cut, 0, f"config 5 seq {b}")
    say(f"config 5: {total}/{B * (steps + 1)} tokens compared")
    assert total >= B * (steps + 1) // 2
