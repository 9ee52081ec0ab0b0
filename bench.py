"""Decode-step benchmark of the Qwen2-VL-2B text decoder on one MI355X.

Workload (the north-star configuration): W4A16 GPTQ
decoder (all q/k/v/o/gate/up/down int4 symmetric, group 128, codes U{0..15},
zero point 8, scales |N(0,0.02)|/7; fp16 embeddings / lm_head), batch 32, each
sequence with a 2048-token context already in the KV pool [32(+1), 4096, 2, 128]
fp16 (N(0,1) values), greedy decode, one new token per sequence per step.  Random
seeded weights of the real architecture (no checkpoints offline).

A step is one ``NativeQwenVLRunner.decode`` call (hipGraph replay of the whole
28-layer step + lm_head/argmax, the H2D of token ids when needed, the D2H of the
new ids).  ``value`` = 32 * steps / wall time of the timed steps.

The JSON line also carries:
* ``roofline`` for the dominant kernel (the split-K decode attention: ~63% of the
  step's algorithmic bytes): algorithmic bytes per launch / its mean duration,
  timed with HIP events on the stream it runs on, against 8 TB/s;
* ``step_roofline``: algorithmic bytes per step / ms_per_step against 8 TB/s;
* ``b1``: the metric's B = 1 case (same int4 weights, one sequence at ctx 2048);
* ``baseline_configs``: BASELINE.json configs[0], [1], [4] with their own shapes (fp16
  B = 1 prefill + decode, fp16 B = 16 decode, multimodal packed prefill + B = 8 decode);
* ``fp8_gemm``: BASELINE.json configs[3], the FP8 W8A8 linears of one decoder layer at
  M = 8192 (achieved dense TFLOP/s against the 5.0 PFLOP/s fp8 MFMA peak);
* ``vit``: the vision tower on one 448 x 448 image (TFLOP/s against the fp16 peak);
* ``cpu_baseline``: the fp32 CPU restatement (oracle/) of the same step, timed on
  this host on a bounded sample with torch using every host core (os.cpu_count()),
  the CPU model name alongside.

``roofline`` is one kernel's fraction (``scope``: "kernel"); the whole step's
fraction, the one the >= 60 % target is stated for, is ``step_roofline.frac``.

Usage: python bench.py [--gpus 1] [--steps 128] [--warmup 3] [--no-cpu] [--no-fp8]
       [--no-vit] [--no-b1] [--no-configs] [--vit-only] [--pmc-probe]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

PEAK_HBM = 8.0e12  # MI355X HBM3E, bytes/s
PEAK_FP8 = 5.0e15  # MI355X dense fp8 MFMA, FLOP/s
PEAK_FP16 = 2.5e15  # MI355X dense fp16 MFMA, FLOP/s

H, I, NL, NH, NKV, HD, V = 1536, 8960, 28, 12, 2, 128, 151936
LINEARS = [(H, (NH + 2 * NKV) * HD), (NH * HD, H), (H, 2 * I), (I, H)]   # (K, N)
KV_TOKEN_BYTES = NL * 2 * NKV * HD * 2                                  # 28672 B / token


def weight_bytes(quant: str) -> int:
    """Algorithmic weight bytes per decode step (each weight read once)."""
    if quant == "gptq":
        lin = sum(K * N // 2 + (K // 128) * N * 2 for K, N in LINEARS)
    else:
        lin = sum(2 * K * N for K, N in LINEARS)
    bias = 2 * LINEARS[0][1]
    return NL * (lin + bias) + 2 * H * (2 * NL + 1) + 2 * V * H


def step_bytes(quant: str, ctx_lens) -> int:
    """Algorithmic HBM bytes of one decode step with the given pre-step context lengths:
    weights once, attended KV rows once (incl. the new token), new KV rows written once,
    embedding rows and ids.  Activations/logits are excluded (fusible)."""
    B = len(ctx_lens)
    kv_read = sum(int(L) + 1 for L in ctx_lens) * KV_TOKEN_BYTES
    return weight_bytes(quant) + kv_read + B * KV_TOKEN_BYTES + B * H * 2 + B * 16


def attn_launch_bytes(ctx_lens) -> int:
    """Algorithmic bytes of one fused decode-attention launch (one layer) for pre-step
    context lengths L: K and V rows [0, L) of both KV heads read, the new K/V row written,
    the fp16 qkv row (+ bias) in and the attention output out."""
    B = len(ctx_lens)
    kv = sum(int(L) for L in ctx_lens) * 2 * NKV * HD * 2 + B * 2 * NKV * HD * 2
    qkv = B * (NH + 2 * NKV) * HD * 2 + (NH + 2 * NKV) * HD * 2
    return kv + qkv + B * NH * HD * 2


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_config3(device, batch: int = 32, ctx: int = 2048, max_len: int = 4096, seed: int = 0,
                  w=None):
    from omniserver_amd import synth
    from omniserver_amd.request import Request, SamplingParams, Sequence
    from omniserver_amd.runner import NativeQwenVLRunner

    shape = synth.DecoderShape()
    if w is None:
        t0 = time.time()
        w = synth.gptq_decoder(shape, seed=seed)
        log(f"synthetic int4 weights generated in {time.time() - t0:.1f}s")
    runner = NativeQwenVLRunner(max_running=batch, max_len=max_len, use_graph=True,
                                quant="gptq", weights=w)
    pool = runner.pool
    g = torch.Generator(device=device)
    g.manual_seed(seed + 1)
    for l in range(NL):
        for kv in (0, 1):
            pool.storage[l, kv, :batch, :ctx].normal_(generator=g)
    seqs = []
    for b in range(batch):
        ids = synth.random_ids(ctx, shape.vocab_size, seed, f"ctx{b}").tolist()
        s = Sequence(Request(prompt=ids, sampling=SamplingParams(max_new_tokens=1 << 30)))
        runner.tokenize(s)
        s.request.sampling.stop_token_ids.clear()      # fixed-length decode
        seqs.append(s)
    runner.attach_prefilled(seqs, [ctx] * batch)
    torch.cuda.synchronize()
    log(f"config3 runner ready (pool {tuple(pool.storage.shape)})")
    return runner, seqs, w, shape


def time_kernel(fn, reps: int) -> float:
    """Mean duration (s) of fn() over reps launches, HIP events on the current stream."""
    st = torch.cuda.current_stream()
    fn()
    st.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        fn()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / 1e3 / reps


def attention_launch_time(runner, B: int, reps: int) -> tuple[float, int]:
    """Mean duration (s) of one decode-attention launch at the current context: the 28
    layers' launches (each over its own layer's K/V, so nothing is served from cache)
    captured in a HIP graph and replayed ``reps`` times between HIP events on the stream
    the kernels run on."""
    model = runner.adapter.model
    cfg = model.cfg
    dev = runner.pool.storage.device
    view = runner.pool.view(B, runner._rope_delta)
    bufs = model.decode_buffers(B, dev)
    Sq = model.layers[0].qkv_proj.forward_partial(bufs["h"], bufs["qpart"])
    view.rope_rows(model.rope_cos, model.rope_sin, bufs["rope"])   # as the step's first launch

    def launches():
        for i, layer in enumerate(model.layers):
            view.attend_fused(bufs["qpart"], Sq, layer.qkv_proj.bias, layer.qkv_proj.fmt == "int4",
                              i, model.scale, model.rope_cos, model.rope_sin, cfg.mrope_section,
                              rope_rows=bufs["rope"])

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launches()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launches()
    g.replay()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(st)
    for _ in range(reps):
        g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    n = reps * len(model.layers)
    return e0.elapsed_time(e1) / 1e3 / n, n


def pmc_probe(runner, seqs, B: int) -> None:
    """Kernel launches for rocprofv3 counter runs (--pmc), each its own dispatch record,
    in this order (the summaries key dispatches by it):
      1. one eager decode step of the config-3 model at B rows (embedding + layer-0 norm,
         then per layer: qkv, attention, o_proj, add+RMSNorm, gate_up + SiLU, down,
         add+RMSNorm; lm_head candidates, argmax) and then
      2. the same step for one row (B = 1), both at the bench context (K/V written past
         the valid lengths only, which are not advanced);
      3. a plain 256 MiB device copy: the byte-counter calibration;
      4. BASELINE.json configs[3]'s four FP8 linears at M = 8192 (qkv, o, gate_up, down);
      5. layer 0's four int4 linears at M = 4096 (config 5's packed prefill: each unpacks
         its weights to fp16, then the pipelined MFMA GEMM; the down projection as the
         prefill runs it at 4096 rows, fp32 partial sums in the GEMM's planned K slices).
    Prints no JSON line."""
    from omniserver_amd.linear import FP8Linear
    model = runner.adapter.model
    dev = runner.pool.storage.device
    runner.decode(seqs)                       # graph captured and one step taken
    runner.settle()
    torch.cuda.synchronize()
    for n in (B, 1):
        ids = torch.tensor([s.last_token_id() for s in seqs[:n]], dtype=torch.int64, device=dev)
        out = torch.empty(n, dtype=torch.int64, device=dev)
        model.decode_greedy(ids, runner.pool.view(n, runner._rope_delta), out)
        torch.cuda.synchronize()
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    for K, N in LINEARS:
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).half()
        x = torch.randn(8192, K, generator=g, device=dev).half()
        lin = FP8Linear(w, rowwise=True)
        xq, sa = lin.quantize_input(x)
        y = torch.empty(8192, N, device=dev, dtype=torch.float16)
        torch.cuda.synchronize()
        lin.gemm_out(xq, sa, y, FP8Linear.OUT_F16_VIA_BF16)
        torch.cuda.synchronize()
        del w, x, lin, xq, y
    lay = model.layers[0]
    for lin in (lay.qkv_proj, lay.o_proj, lay.gate_up_proj, lay.down_proj):
        x = torch.randn(4096, lin.K, generator=g, device=dev).half()
        torch.cuda.synchronize()
        if lin is lay.down_proj and model.prefill_down_partials_ok(4096):
            part = torch.empty(lin.partial_plan(4096) * 4096 * lin.N, device=dev,
                               dtype=torch.float32)
            lin.forward_partial_planned(x, part)
        else:
            y = torch.empty(4096, lin.out_features, device=dev, dtype=torch.float16)
            lin.forward_out(x, y)
        torch.cuda.synchronize()
    log(f"pmc probe: eager decode steps at B={B} and 1 (ctx {int(runner.pool.lengths[0])}), "
        f"one 256 MiB copy, 4 FP8 linears at M=8192, 4 int4 linears at M=4096")


def traffic_from_profiles(kernel: str):
    """HBM bytes per launch of ``kernel`` measured with rocprofv3 byte counters and
    calibrated against a plain copy (profiles/traffic.json, written from the runs its
    "commands" field lists), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        k = t["kernels"][kernel]
        return int(k["fetch_bytes"] + k["write_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def mfma_from_profiles(prefix: str) -> dict | None:
    """MFMA busy % per linear from rocprofv3 counters (profiles/traffic.json "mfma", written
    from the runs its "commands" list): {linear: busy %} for the GEMMs whose key starts with
    ``prefix``, or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            g = json.load(f)["mfma"]["gemms"]
        return {k.split()[-1]: v["mfma_busy_pct"] for k, v in g.items() if k.startswith(prefix)}
    except (OSError, KeyError, ValueError):
        return None


def fp8_layer_gemms(device, M: int = 8192, reps: int = 10) -> dict:
    """the FP8 e4m3fn W8A8 linears of one decoder layer on a packed
    8 x 1024-token prefill (M = 8192): QKV 1536->2048, O 1536->1536, gate/up 1536->17920,
    down 8960->1536.  Weights N(0, 0.02) quantised per output channel, activations N(0, 1)
    quantised per token; the timed region is the fp8 MFMA GEMM (fp32 accumulate, bf16 ->
    fp16 epilogue) with inputs resident in HBM, the median of five timed repetitions of
    ``reps`` launches after 0.1 s of untimed passes over the layer.  Achieved dense TFLOP/s
    against the MI355X fp8 peak (5.0 PFLOP/s)."""
    from omniserver_amd.linear import FP8Linear
    shapes = [("qkv", 1536, 2048), ("o", 1536, 1536), ("gate_up", 1536, 17920),
              ("down", 8960, 1536)]
    g = torch.Generator(device=device)
    g.manual_seed(4)
    ops = []
    for name, K, N in shapes:
        lin = FP8Linear((torch.randn(N, K, device=device, generator=g) * 0.02).half(),
                        rowwise=True)
        x = torch.randn(M, K, device=device, generator=g).half()
        xq, sa = lin.quantize_input(x)
        out = torch.empty(M, N, device=device, dtype=torch.float16)
        ops.append((name, 2.0 * M * N * K,
                    lambda lin=lin, xq=xq, sa=sa, out=out:
                        lin.gemm_out(xq, sa, out, FP8Linear.OUT_F16_VIA_BF16)))
        del x
    # Untimed passes over the whole layer for 0.1 s, then each shape's median of five timed
    # repetitions: the first pass runs on freshly allocated buffers and ramping clocks (its
    # layer time, reported as first_pass_us, is 2-4 % above the steady state on MI355X, and
    # ~10 ms of passes do not close the gap), as a prefill's first layer would; the timed
    # repetitions are the steady state of a running prefill.
    first = sum(time_kernel(f, reps) for _, _, f in ops)
    t_end = time.perf_counter() + 0.1
    while time.perf_counter() < t_end:
        for _, _, f in ops:
            time_kernel(f, reps)
    per, tot_s, tot_f = {}, 0.0, 0.0
    for name, fl, f in ops:
        t = statistics.median(time_kernel(f, reps) for _ in range(5))
        per[name] = {"us": round(t * 1e6, 1), "tflops": round(fl / t / 1e12, 1)}
        tot_s += t
        tot_f += fl
    del ops
    return {"workload": f"one layer's W8A8 linears at M={M}", "gflop": round(tot_f / 1e9, 1),
            "us": round(tot_s * 1e6, 1), "achieved": round(tot_f / tot_s / 1e12, 1),
            "peak": PEAK_FP8 / 1e12, "unit": "TFLOP/s", "frac": round(tot_f / tot_s / PEAK_FP8, 4),
            "first_pass_us": round(first * 1e6, 1),
            "per_shape": per,
            "mfma_busy_pct_counters": mfma_from_profiles("fp8 W8A8 M=8192")}


def decode_b1(device, w, ctx: int = 2048, steps: int = 64) -> dict:
    """The metric's B = 1 case: the same int4 decoder and weights, one sequence at a 2048-token
    context (pool [1, 4096, 2, 128] fp16), greedy hipGraph steps; algorithmic bytes per step
    (weights once + the sequence's KV) against the 8 TB/s HBM peak."""
    runner, seqs, _, _ = build_config3(device, 1, ctx, w=w)
    for _ in range(3):
        runner.decode(seqs)
    torch.cuda.synchronize()
    ahead = runner.steps_ahead()
    ctx0 = int(runner.pool.lengths[0]) - ahead
    t0 = time.perf_counter()
    for _ in range(steps):
        runner.decode(seqs)
    torch.cuda.synchronize()
    per = (time.perf_counter() - t0) / steps
    runner.settle()
    g = runner._graphs[1][0]
    st = torch.cuda.current_stream()
    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    r0.record(st)
    for _ in range(16):
        g.replay()
    r1.record(st)
    torch.cuda.synchronize()
    nbytes = sum(step_bytes("gptq", [ctx0 + s]) for s in range(steps)) / steps
    out = {"workload": f"int4 decode B=1, ctx {ctx}", "ms_per_step": round(per * 1e3, 4),
           "tok_per_s": round(1.0 / per, 1), "graph_replay_ms": round(r0.elapsed_time(r1) / 16, 4),
           "bytes_per_step": int(nbytes), "achieved_GBps": round(nbytes / per / 1e9, 1),
           "frac": round(nbytes / per / PEAK_HBM, 4)}
    del runner, seqs
    torch.cuda.empty_cache()
    return out


def _timed_decode(runner, seqs, steps: int, warmup: int = 3):
    """(wall ms per step, graph replay ms, pre-step contexts) of `steps` greedy decode steps."""
    for _ in range(warmup):
        runner.decode(seqs)
    torch.cuda.synchronize()
    B = len(seqs)
    ahead = runner.steps_ahead()
    ctx0 = [L - ahead for L in runner.pool.lengths[:B].cpu().tolist()]
    t0 = time.perf_counter()
    for _ in range(steps):
        runner.decode(seqs)
    torch.cuda.synchronize()
    per = (time.perf_counter() - t0) / steps
    runner.settle()
    g = runner._graphs[B][0]
    st = torch.cuda.current_stream()
    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    r0.record(st)
    for _ in range(8):
        g.replay()
    r1.record(st)
    torch.cuda.synchronize()
    return per * 1e3, r0.elapsed_time(r1) / 8, ctx0


def _decode_line(quant, per_ms, replay_ms, ctx0, steps):
    B = len(ctx0)
    nbytes = sum(step_bytes(quant, [L + s for L in ctx0]) for s in range(steps)) / steps
    return {"ms_per_step": round(per_ms, 4), "tok_per_s": round(B / per_ms * 1e3, 1),
            "graph_replay_ms": round(replay_ms, 4), "bytes_per_step": int(nbytes),
            "frac": round(nbytes / (per_ms / 1e3) / PEAK_HBM, 4)}


def _prefill_ms(r, make_seqs, reps: int, idle_s: float = 0.0):
    """Median wall time (ms) of ``reps`` prefills of make_seqs() on runner r, each into a
    freshly freed pool; returns (median ms, the last prefill's sequences).  The wall time
    includes the prefill's host-side input preparation (tokens, image rows, M-RoPE positions,
    the upload).  The requests themselves are made before the timed loop, as a serving
    engine's queue holds them: their synthetic vision rows are host-side random draws that
    would otherwise leave the GPU idle for tens of ms before every timed prefill, and MI355X
    lowers its clocks within a few ms of idle (configs[4]'s graph replay after 0.5 / 1 / 5 /
    20 ms of host idle: 12.4 / 12.45 / 13.5 / 14.1 ms).  Consecutive prefills are then
    separated by the pool's frees alone, as in serving, where prefills run between decode
    steps; ``idle_s`` > 0 instead times each prefill after that long idle (reported beside).
    The loop starts once the host's thread pools, still spinning after the set-up's CPU work
    (synthetic weights, packing), have gone idle, behind one untimed prefill (the first use of
    the prefill kernels, or a layout's graph capture)."""
    seqs = make_seqs()
    r.prefill(seqs)
    torch.cuda.synchronize()
    batches = [make_seqs() for _ in range(reps + 1)]
    time.sleep(0.5)
    ts = []
    for i, nxt in enumerate(batches):
        for s_ in seqs:
            r.free(s_)
        seqs = nxt
        torch.cuda.synchronize()
        if idle_s:
            time.sleep(idle_s)
        t1 = time.perf_counter()
        r.prefill(seqs)
        torch.cuda.synchronize()
        if i:
            ts.append((time.perf_counter() - t1) * 1e3)
    return sorted(ts)[len(ts) // 2], seqs


def _prefill_eager_ms(r, make_seqs, reps: int):
    """_prefill_ms with the runner's prefill graphs off: every prefill runs eagerly, as the
    first prefill of a segment layout does (a serving engine rarely repeats a layout)."""
    keep = r.prefill_graph_layouts
    r.prefill_graph_layouts = 0
    try:
        ms, seqs = _prefill_ms(r, make_seqs, reps)
    finally:
        r.prefill_graph_layouts = keep
    for s_ in seqs:
        r.free(s_)
    return ms


def _f16_expansion(r) -> dict:
    """The GPTQ linears' resident fp16 expansions the int4 prefill runs on: their bytes, and
    the device time of making them all again (omni_w4_unpack_f16, CUDA events around the
    launches into a scratch buffer), which the first large prefill pays once."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd.linear import GPTQLinear
    lins = [m for m in r.adapter.model.modules() if isinstance(m, GPTQLinear)]
    nbytes = sum(2 * m.N * m.K for m in lins if getattr(m, "_w16", None) is not None)
    buf = torch.empty(max(m.N * m.K for m in lins), device=r.device, dtype=torch.float16)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for m in lins:
        call("omni_w4_unpack_f16", ptr(m.qweight_packed), ptr(m.scales_packed), ptr(buf), m.K,
             m.N, stream())
    e1.record()
    torch.cuda.synchronize()
    del buf
    int4 = sum(m.qweight_packed.numel() * 4 + m.scales_packed.numel() * 2 for m in lins)
    return {"prefill_f16_resident_bytes": int(nbytes), "int4_weight_bytes": int(int4),
            "prefill_f16_unpack_ms": round(e0.elapsed_time(e1), 3)}


def _config1_runner(w16):
    """configs[0]'s runner and prompt maker: fp16, batch 1, a 256-token prompt."""
    from omniserver_amd import synth
    from omniserver_amd.request import Request, SamplingParams, Sequence
    from omniserver_amd.runner import NativeQwenVLRunner
    shape = synth.DecoderShape()
    r = NativeQwenVLRunner(max_running=1, max_len=1024, use_graph=True, weights=w16)
    mk = lambda: [Sequence(Request(prompt=synth.random_ids(256, shape.vocab_size, 1, "c1").tolist(),
                                   sampling=SamplingParams(max_new_tokens=1 << 30)))]
    return r, mk


def _config5_runner(device, w_int4, B: int = 8):
    """configs[4]'s runner and prompt maker: int4, 8 x [63 text, <|vision_start|>, 256 vision
    rows (grid 1 x 32 x 32), 192 text] packed into T = 4096 rows."""
    from omniserver_amd import synth
    from omniserver_amd.positions import IMAGE_TOKEN_ID, VISION_START_TOKEN_ID
    from omniserver_amd.request import Request, SamplingParams, Sequence, VisionInput
    from omniserver_amd.runner import NativeQwenVLRunner
    shape = synth.DecoderShape()
    r = NativeQwenVLRunner(max_running=B, max_len=4096, use_graph=True, quant="gptq", weights=w_int4)

    def mk():
        ss = []
        for b in range(B):
            ids = (synth.random_ids(63, shape.vocab_size, 5, f"c5a.{b}").tolist()
                   + [VISION_START_TOKEN_ID] + [IMAGE_TOKEN_ID] * 256
                   + synth.random_ids(192, shape.vocab_size, 5, f"c5b.{b}").tolist())
            rows = synth.randn16((256, shape.hidden_size), 1.0, 5, f"c5v.{b}").to(device)
            ss.append(Sequence(Request(prompt=ids, sampling=SamplingParams(max_new_tokens=1 << 30),
                                       images=[VisionInput(rows, (1, 32, 32))])))
        return ss
    return r, mk


def _prefill_flops(T: int, B: int, L: int) -> float:
    """Dense FLOPs of a packed prefill of B segments of L tokens (T = B L): the four linears
    per layer (2 T K N) and the causal attention (QK^T and PV over L (L + 1) / 2 pairs)."""
    lin = sum(2.0 * T * K * N for K, N in LINEARS) * NL
    att = NL * B * 4.0 * (L * (L + 1) / 2) * NH * HD
    return lin + att


def prefill_only(device) -> dict:
    """configs[0]'s and configs[4]'s prefills alone (median of 5 / 3 after a warm-up), for
    profiling the prefill path: ``python bench.py --prefill-only``."""
    from omniserver_amd import synth
    shape = synth.DecoderShape()
    r, mk = _config1_runner(synth.fp16_decoder(shape, seed=1))
    c1e = _prefill_eager_ms(r, mk, 5)
    c1, _ = _prefill_ms(r, mk, 5)
    del r
    torch.cuda.empty_cache()
    r, mk = _config5_runner(device, synth.gptq_decoder(shape, seed=0))
    c5e = _prefill_eager_ms(r, mk, 3)
    c5, _ = _prefill_ms(r, mk, 3)
    fl = _prefill_flops(4096, 8, 512)
    return {"metric": "prefill ms (BASELINE configs[0] and [4])", "config1_prefill_ms": round(c1, 3),
            "config1_prefill_eager_ms": round(c1e, 3),
            "config5_prefill_ms": round(c5, 3), "config5_prefill_eager_ms": round(c5e, 3),
            "config5_prefill_tflops": round(fl / (c5 * 1e-3) / 1e12, 1),
            "config5_prefill_frac_fp16_peak": round(fl / (c5 * 1e-3) / PEAK_FP16, 4),
            **_f16_expansion(r)}


def baseline_configs(device, w_int4) -> dict:
    """BASELINE.json configs[0], [1] and [4] end to end with their own shapes (configs[2] is the
    headline line, configs[3] the fp8_gemm object): seeded synthetic weights, hipGraph
    decode, decode rates against the HBM peak, the packed prefill against the fp16 MFMA
    peak."""
    from omniserver_amd import synth
    from omniserver_amd.request import Request, SamplingParams, Sequence
    from omniserver_amd.runner import NativeQwenVLRunner
    shape = synth.DecoderShape()
    mk = lambda ids, **kw: Sequence(Request(prompt=ids, sampling=SamplingParams(max_new_tokens=1 << 30), **kw))
    out = {}
    t0 = time.time()
    w16 = synth.fp16_decoder(shape, seed=1)
    log(f"synthetic fp16 weights generated in {time.time() - t0:.1f}s")

    # fp16, batch 1, 256-token prompt, 32 new tokens (prefill: median of 5)
    r, mk1 = _config1_runner(w16)
    eager_ms = _prefill_eager_ms(r, mk1, 5)
    pre_ms, seqs = _prefill_ms(r, mk1, 5)
    per, rep, ctx0 = _timed_decode(r, seqs, 32)
    out["config1"] = {"workload": "fp16 decoder, B=1, 256-token prompt, 32 greedy steps",
                      "prefill_ms": round(pre_ms, 3), "prefill_eager_ms": round(eager_ms, 3),
                      "prefill_note": "prefill_ms: graph replay of a captured segment layout; "
                                      "prefill_eager_ms: every prefill eager (a new layout)",
                      **_decode_line("fp16", per, rep, ctx0, 32)}
    del r, seqs

    # fp16, batch 16, contexts U[512, 2048], pool [16, 4096], 64 steps
    B = 16
    lens = synth.context_lengths(B, 512, 2048, 2).tolist()
    r = NativeQwenVLRunner(max_running=B, max_len=4096, use_graph=True, weights=w16)
    g = torch.Generator(device=device)
    g.manual_seed(3)
    for l in range(NL):
        for kv in (0, 1):
            for b, L in enumerate(lens):
                r.pool.storage[l, kv, b, :L].normal_(generator=g)
    seqs = [mk(synth.random_ids(4, shape.vocab_size, 2, f"c2.{b}").tolist()) for b in range(B)]
    for s_ in seqs:
        r.tokenize(s_)
    r.attach_prefilled(seqs, lens)
    per, rep, ctx0 = _timed_decode(r, seqs, 64)
    out["config2"] = {"workload": "fp16 decoder, B=16, contexts U[512, 2048], 64 greedy steps",
                      **_decode_line("fp16", per, rep, ctx0, 64)}
    del r, seqs, w16
    torch.cuda.empty_cache()

    # int4, 8 x [64 text, 256 vision rows (grid 1 x 32 x 32), 192 text] packed
    # prefill (T = 4096, block-diagonal causal; median of 3), then 128 greedy steps at B = 8
    B = 8
    r, mk5 = _config5_runner(device, w_int4, B)
    eager5 = _prefill_eager_ms(r, mk5, 3)
    idle5, seqs = _prefill_ms(r, mk5, 3, idle_s=0.02)
    for s_ in seqs:
        r.free(s_)
    pre_ms5, seqs = _prefill_ms(r, mk5, 3)
    pre = pre_ms5 * 1e-3
    T = 512 * B
    fl = _prefill_flops(T, B, 512)
    per, rep, ctx0 = _timed_decode(r, seqs, 128)
    out["config5"] = {"workload": "int4 decoder, 8 x 512-token image+text prompts: packed prefill "
                                  "(T = 4096), then 128 greedy steps at B = 8",
                      "prefill_ms": round(pre * 1e3, 3), "prefill_eager_ms": round(eager5, 3),
                      "prefill_after_idle_ms": round(idle5, 3),
                      "prefill_tok_per_s": round(T / pre, 1),
                      "prefill_tflops": round(fl / pre / 1e12, 1),
                      "prefill_frac_fp16_peak": round(fl / pre / PEAK_FP16, 4),
                      "prefill_eager_frac_fp16_peak": round(fl / (eager5 * 1e-3) / PEAK_FP16, 4),
                      "prefill_note": "the int4 linears' prefill GEMMs run on a resident fp16 "
                                      "expansion of their weights, made at the first prefill of "
                                      ">= 256 rows (prefill_f16_unpack_ms, outside the timed "
                                      "prefills) and kept (prefill_f16_resident_bytes beside "
                                      "int4_weight_bytes); decode streams the int4 words; "
                                      "prefill_after_idle_ms: each prefill after 20 ms of GPU "
                                      "idle (the clocks drop within a few ms of idle)",
                      **_f16_expansion(r),
                      "prefill_gemm_mfma_busy_pct_counters": mfma_from_profiles("int4 prefill M=4096"),
                      **_decode_line("gptq", per, rep, ctx0, 128)}
    del r, seqs
    torch.cuda.empty_cache()
    return out


def vit_flops(grids, cfg) -> float:
    """Dense FLOPs of one vision-tower forward (model/qwen2_vit.py:118-129): the patch
    embedding (K = 1176), per block the four linears and the two attention products within
    each frame, the merger's two linears."""
    D, I, M = cfg.embed_dim, cfg.mlp_dim, cfg.merged_dim
    S = sum(t * h * w for t, h, w in grids)
    attn = sum(t * 4.0 * (h * w) ** 2 * D for t, h, w in grids)
    block = 2.0 * S * D * (3 * D + D + 2 * I) + attn
    merger = 2.0 * (S // 4) * M * (M + cfg.out_hidden)
    return 2.0 * S * cfg.patch_dim * D + cfg.depth * block + merger


def vit_tower(device, grid=(1, 32, 32), reps: int = 5) -> dict:
    """The vision tower (all 32 blocks + merger, seeded synthetic fp16 weights) on one
    448 x 448 image (32 x 32 patches -> 256 rows), pixels resident in HBM.  Achieved dense
    TFLOP/s against the MI355X fp16 MFMA peak (2.5 PFLOP/s)."""
    from omniserver_amd import synth
    from omniserver_amd.vit import Qwen2VIT, VisionConfig, load_vit_from_state_dict
    cfg = VisionConfig()
    tower = load_vit_from_state_dict(Qwen2VIT(device=device), synth.vision_tower(cfg, seed=5))
    pv = synth.pixel_patches([grid], cfg.patch_dim, 6).to(device)
    # untimed forwards for 0.1 s first, so the timed ones run at the clocks of a busy GPU
    t_end = time.perf_counter() + 0.1
    while time.perf_counter() < t_end:
        tower(pv, [grid])
        torch.cuda.synchronize()
    t = time_kernel(lambda: tower(pv, [grid]), reps)
    fl = vit_flops([grid], cfg)
    return {"workload": f"vision tower, 32 blocks + merger, one image grid {list(grid)} "
                        f"({grid[0] * grid[1] * grid[2]} patches)",
            "gflop": round(fl / 1e9, 1), "ms": round(t * 1e3, 3),
            "achieved": round(fl / t / 1e12, 1), "peak": PEAK_FP16 / 1e12, "unit": "TFLOP/s",
            "frac": round(fl / t / PEAK_FP16, 4)}


def cpu_model() -> str:
    """The host CPU's model name (what lscpu prints as 'Model name')."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(runner, seqs, w, shape, budget_s: float = 12.0, max_steps: int = 20) -> dict:
    """fp32 CPU restatement (oracle) of the same decode step on this host's cores."""
    from oracle import qwen2_ref as ref
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    t0 = time.time()
    cfg = ref.Qwen2Config()
    layers = [ref.LayerWeights(
        in_norm=l["in_norm"].float(), post_norm=l["post_norm"].float(),
        qkv_t=ref.gptq_dequant(l["qkv_q"], l["qkv_s"]), qkv_b=l["qkv_b"].float(),
        o_t=ref.gptq_dequant(l["o_q"], l["o_s"]),
        gate_up_t=ref.gptq_dequant(l["gate_up_q"], l["gate_up_s"]),
        down_t=ref.gptq_dequant(l["down_q"], l["down_s"])) for l in w["layers"]]
    orc = ref.Qwen2Ref(cfg, w["embed"].float(), w["norm"].float(), layers, True, f16=False)
    B = len(seqs)
    lengths = runner.pool.lengths[:B].cpu()
    Lmax = int(lengths.max()) + max_steps + 4      # room for the warm-up and timed tokens
    kp = [runner.pool.k[l][:B, :Lmax].float().cpu() for l in range(NL)]
    vp = [runner.pool.v[l][:B, :Lmax].float().cpu() for l in range(NL)]
    lengths = torch.cat([lengths, torch.zeros(1, dtype=torch.int64)])
    log(f"cpu baseline: oracle built in {time.time() - t0:.1f}s, {threads} threads")
    ids = [s.last_token_id() for s in seqs]
    orc.decode_step(ids, kp, vp, lengths)          # warm-up
    lengths[:B] += 1
    n, t1 = 0, time.perf_counter()
    while True:
        orc.decode_step(ids, kp, vp, lengths)
        lengths[:B] += 1
        n += 1
        el = time.perf_counter() - t1
        if el >= budget_s or n >= max_steps:
            break
    per = el / n
    return {"value": round(B / per, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "torch_threads": torch.get_num_threads(),
            "ms_per_step": round(per * 1e3, 1),
            "sample": f"{n} decode steps (after 1 warm-up) of the same B={B}, ctx~{int(lengths[0])} "
                      f"int4 config, all 28 layers, fp32 oracle (weights dequantised once)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--ctx", type=int, default=2048)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-fp8", action="store_true",
                    help="skip the FP8 W8A8 GEMM leg (BASELINE.json configs[3])")
    ap.add_argument("--no-vit", action="store_true", help="skip the vision-tower leg")
    ap.add_argument("--no-b1", action="store_true", help="skip the B = 1 decode leg")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip BASELINE.json configs[0], [1], [4] (fp16 B=1 / B=16, multimodal)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="time only configs[0]'s and configs[4]'s prefills (one JSON object)")
    ap.add_argument("--vit-only", action="store_true",
                    help="time only the vision tower (one JSON object) and exit")
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--kernel-steps", type=int, default=10,
                    help="replays of the 28-launch attention graph timed for the roofline")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="for rocprofv3 --pmc: eager decode steps at B and 1, a plain 256 MiB "
                         "device copy (the byte-counter calibration), the FP8 and int4 prefill "
                         "linears (see pmc_probe); prints no JSON line")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(data-parallel sharding by sequence is a design note, not implemented)",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.vit_only:
        print(json.dumps(vit_tower(dev)), flush=True)
        return
    if args.prefill_only:
        print(json.dumps(prefill_only(dev)), flush=True)
        return

    runner, seqs, w, shape = build_config3(dev, args.batch, args.ctx)
    B = len(seqs)
    if args.pmc_probe:
        pmc_probe(runner, seqs, B)
        return

    for _ in range(args.warmup):
        runner.decode(seqs)
    torch.cuda.synchronize()

    # the runner may hold the next step enqueued ahead (already run by the synchronize):
    # the first timed step's contexts are the lengths before it
    ahead = runner.steps_ahead()
    ctx_before = [L - ahead for L in runner.pool.lengths[:B].cpu().tolist()]
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(st)
    for _ in range(args.steps):
        runner.decode(seqs)
    e1.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dev_ms = e0.elapsed_time(e1) / args.steps
    ms = wall * 1e3 / args.steps
    tok_s = B * args.steps / wall

    # device time of the step alone: the captured graph replayed back to back (no D2H,
    # no host bookkeeping between steps)
    runner.settle()
    g = runner._graphs[B][0]
    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    r0.record(st)
    for _ in range(8):
        g.replay()
    r1.record(st)
    torch.cuda.synchronize()
    replay_ms = r0.elapsed_time(r1) / 8

    # algorithmic bytes per step, averaged over the timed steps (contexts grow by 1/step)
    avg_step_bytes = sum(step_bytes("gptq", [L + s for L in ctx_before])
                         for s in range(args.steps)) / args.steps

    # dominant kernel: decode attention (all 28 layers of eager steps at the current context)
    model = runner.adapter.model
    bufs = model.decode_buffers(B, dev)
    ctx_now = runner.pool.lengths[:B].cpu().tolist()
    t_attn, n_attn = attention_launch_time(runner, B, args.kernel_steps)
    a_bytes = attn_launch_bytes(ctx_now)
    achieved = a_bytes / t_attn
    # second-largest stream: the gate_up W4A16 GEMM with the fused SiLU
    lay = model.layers[0]
    t_gu = time_kernel(lambda: lay.gate_up_proj.forward_out(bufs["h"], bufs["act"]),
                       args.kernel_reps)
    gu_bytes = H * 2 * I // 2 + (H // 128) * 2 * I * 2 + B * H * 2 + B * I * 2

    out = {
        "metric": "decode tok/s + ms/step, Qwen2-VL-2B LLM shape, B=1/32 int4; % HBM roofline",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": "Qwen2-VL-2B text decoder, W4A16 GPTQ int4 g128 (lm_head/embed fp16), "
                        f"greedy decode B={B}, ctx {args.ctx} (pool [{B},{runner.pool.max_len},2,128] "
                        "fp16, N(0,1) prefix), hipGraph step",
            "batch": B, "context": args.ctx, "max_len": runner.pool.max_len,
            "weights": "int4 codes U{0..15} zp 8, scales |N(0,0.02)|/7, seeded",
            "parallelism": "single GPU",
        },
        "roofline": {
            "scope": "kernel (the step's fraction is step_roofline.frac)",
            "bound": "hbm",
            "kernel": "decode_attn_kernel (qkv partials + bias + M-RoPE + KV write + split GQA "
                      "decode attention, states out), graph of the 28 layers' launches",
            "achieved": round(achieved / 1e9, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM, 4),
            "traffic": traffic_from_profiles("decode_attn_kernel"),
            "launch_us": round(t_attn * 1e6, 2), "launches": n_attn, "bytes_per_launch": a_bytes,
        },
        "step_roofline": {
            "bytes_per_step": int(avg_step_bytes),
            "achieved": round(avg_step_bytes / (ms / 1e3) / 1e9, 1), "unit": "GB/s",
            "frac": round(avg_step_bytes / (ms / 1e3) / PEAK_HBM, 4),
            "device_ms_per_step": round(dev_ms, 4),
            "device_frac": round(avg_step_bytes / (dev_ms / 1e3) / PEAK_HBM, 4),
            "graph_replay_ms": round(replay_ms, 4),
        },
        "kernels": {
            "gate_up_w4a16_silu_us": round(t_gu * 1e6, 2),
            "gate_up_GBps": round(gu_bytes / t_gu / 1e9, 1),
        },
        "b1": None,
        "baseline_configs": None,
        "fp8_gemm": None,
        "vit": None,
        "cpu_baseline": None,
    }
    if not args.no_b1:
        try:
            out["b1"] = decode_b1(dev, w, args.ctx)
        except Exception as e:  # report, never fail the decode line on this leg
            out["b1"] = {"error": repr(e)}
    if not args.no_configs:
        try:
            out["baseline_configs"] = baseline_configs(dev, w)
        except Exception as e:  # report, never fail the decode line on this leg
            out["baseline_configs"] = {"error": repr(e)}
    if not args.no_fp8:
        try:
            out["fp8_gemm"] = fp8_layer_gemms(dev)
        except Exception as e:  # report, never fail the decode line on this leg
            out["fp8_gemm"] = {"error": repr(e)}
    if not args.no_vit:
        try:
            out["vit"] = vit_tower(dev)
        except Exception as e:  # report, never fail the decode line on this leg
            out["vit"] = {"error": repr(e)}
    if not args.no_cpu:
        try:
            out["cpu_baseline"] = cpu_baseline(runner, seqs, w, shape)
        except Exception as e:  # report, never fail the GPU line on the CPU leg
            out["cpu_baseline"] = {"error": repr(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
