"""Vision tower on the GPU against the CPU oracle (oracle/qwen2_vit_ref.py).

Kernel by kernel (LayerNorm, 2-D rotary, segmented attention, the tiled GEMM's
epilogues incl. the zero-padded K of the patch embedding), then the whole tower at
reduced and at full depth.  Tolerances are stated per test: the kernels accumulate in
fp32 in another order than the oracle, so an fp16 rounding may land one ulp apart, and
the attention rounds its probabilities to fp16 for the MFMA (as flash attention does).
"""

import pytest
import torch

from oracle import qwen2_vit_ref as vref

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)


def f16(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(torch.float16)


def rel_err(got, want):
    got, want = got.float().cpu(), want.float().cpu()
    return (got - want).abs().max().item() / max(want.abs().max().item(), 1e-6)


@pytest.mark.parametrize("rows", [1, 7, 300])
def test_layernorm(gpu, rows):
    from omniserver_amd import vit
    say(f"layernorm rows={rows}")
    N = 1280
    x = f16((rows, N), 1, 2.0)
    w = (1 + 0.1 * f16((N,), 2).float()).half()
    b = f16((N,), 3, 0.1)
    out = torch.empty(rows, N, device=gpu, dtype=torch.float16)
    vit.layer_norm_out(x.to(gpu), w.to(gpu), b.to(gpu), 1e-6, out)
    want = vref.layer_norm(x.float(), w.float(), b.float(), 1e-6)
    d = (out.cpu().float() - want).abs()
    # one fp16 ulp of each value (fp32 sums in another order)
    assert (d <= want.abs() * 2.0 ** -10 + 1e-3).all(), d.max().item()


@pytest.mark.parametrize("grids", [[(1, 4, 6)], [(1, 8, 8), (2, 2, 2), (1, 6, 4)]])
def test_vision_rope(gpu, grids):
    from omniserver_amd import vit
    say(f"vision_rope grids={grids}")
    nh, hd = 16, 80
    S = sum(t * h * w for t, h, w in grids)
    qkv = f16((S, 3 * nh * hd), 4)
    dev = qkv.to(gpu)
    vit.vision_rope_(dev, nh, hd, vit.rot_pos_ids(grids, 2).to(gpu),
                     vit.vision_inv_freq(hd, 10000.0).to(gpu))
    got = dev.cpu().view(S, 3, nh, hd)
    cos, sin = vref.rot_cos_sin(grids, hd)
    x = qkv.float().view(S, 3, nh, hd)
    eq, ek = vref.vision_rope(x[:, 0], x[:, 1], cos, sin)
    for g, e in ((got[:, 0], eq), (got[:, 1], ek)):
        d = (g.float() - e).abs()
        assert (d <= e.abs() * 2.0 ** -10 + 2.0 ** -20).all(), d.max().item()
    assert torch.equal(got[:, 2], qkv.view(S, 3, nh, hd)[:, 2])          # v untouched


@pytest.mark.parametrize("lens", [[4], [64], [100], [4, 64, 37, 200], [1024], [16, 16, 16, 16]])
def test_vit_attention(gpu, lens):
    from omniserver_amd import vit
    say(f"vit_attention segments={lens}")
    nh, hd = 16, 80
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    S = cu[-1]
    qkv = f16((S, 3 * nh * hd), 5)
    cu_t = torch.tensor(cu, dtype=torch.int32)
    tiles = vit.query_tiles(cu_t)
    out = torch.full((S, nh * hd), float("nan"), device=gpu, dtype=torch.float16)
    vit.vit_attention_out(qkv.to(gpu), nh, hd, cu_t.to(gpu), tiles.to(gpu), hd ** -0.5, out)
    x = qkv.float().view(S, 3, nh, hd)
    want = vref.seg_attention(x[:, 0], x[:, 1], x[:, 2], cu, hd ** -0.5).reshape(S, nh * hd)
    got = out.cpu().float()
    assert not torch.isnan(got).any()
    assert (got - want).abs().max().item() <= 4e-3


# (M, N, K, epilogue, bias): the tower's shapes (patch embed K = 1176 padded to 1280)
GEMM_CASES = [(300, 1280, 1176, 0, False), (300, 3840, 1280, 0, True), (257, 5120, 1280, 4, True),
              (64, 1280, 5120, 6, True), (75, 5120, 5120, 5, True), (75, 1536, 5120, 0, True),
              (5, 1280, 1280, 6, True), (1, 3840, 1280, 0, True), (1024, 1280, 5120, 6, True)]
# (path, tile_rows, ksplit): the pipelined GEMM at both tile heights, without and with
# K slices (0 = its own choice), the packed tiled GEMM
PATHS = [("pipe", 128, 1), ("pipe", 256, 1), ("pipe", 128, 0), ("pipe", 256, 3), ("tiled", 0, 0)]


@pytest.mark.parametrize("path,tile_rows,ksplit", PATHS)
@pytest.mark.parametrize("M,N,K,epi,has_bias", GEMM_CASES)
def test_gemm_epilogues(gpu, M, N, K, epi, has_bias, path, tile_rows, ksplit):
    from omniserver_amd import vit
    if path == "pipe" and K % 128:
        pytest.skip("the pipelined GEMM takes K % 128 == 0 (the patch embedding uses the tiled one)")
    if path == "pipe" and K // 64 // max(ksplit, 1) < 4:
        pytest.skip("slices below 4 K steps")
    say(f"gemm {path}/{tile_rows}/ks{ksplit} M={M} N={N} K={K} epi={epi}")
    x = f16((M, K), 6)
    w = f16((N, K), 7, 0.02)
    b = f16((N,), 8, 0.02) if has_bias else None
    res = f16((M, N), 9)
    lin = vit.VisionLinear(w, b, gpu, path=path)
    out = res.to(gpu).clone() if epi == vit.EPI_RESID else torch.empty(M, N, device=gpu,
                                                                        dtype=torch.float16)
    lin.out(x.to(gpu), out, epi, res=out if epi == vit.EPI_RESID else None, tile_rows=tile_rows,
            ksplit=ksplit)
    h = vref.linear(x.float(), w.float(), None if b is None else b.float())
    if epi == vit.EPI_QGELU:
        want = vref.quick_gelu(h)
    elif epi == vit.EPI_GELU:
        want = vref.gelu(h)
    elif epi == vit.EPI_RESID:
        want = vref.r16(res.float() + h)
    else:
        want = h
    d = (out.cpu().float() - want).abs()
    # the fp32 sum may round to the neighbouring fp16 value (and that ulp carries through
    # the elementwise epilogue)
    tol = 2.0 ** -9 * (want.abs() + h.abs()) + 1e-3 * want.abs().max().item()
    assert (d <= tol).all(), d.max().item()


def _tower(gpu, depth, seed):
    from omniserver_amd import synth, vit
    cfg = vit.VisionConfig(depth=depth)
    sd = synth.vision_tower(cfg, seed=seed, depth=depth)
    tower = vit.load_vit_from_state_dict(vit.Qwen2VIT(depth=depth, device=gpu), sd)
    return cfg, sd, tower


def test_vit_tower_two_blocks(gpu):
    from omniserver_amd import synth
    say("vit tower depth 2, three images")
    cfg, sd, tower = _tower(gpu, 2, 11)
    grids = [(1, 8, 8), (1, 4, 6), (2, 2, 4)]
    pv = synth.pixel_patches(grids, cfg.patch_dim, 12)
    got = tower(pv.to(gpu), grids).cpu().float()
    want = vref.vit_forward(pv.float(), grids, sd)
    assert got.shape == want.shape == (16 + 6 + 4, 1536)
    cos = torch.nn.functional.cosine_similarity(got, want, dim=-1).min().item()
    e = rel_err(got, want)
    say(f"depth 2: max rel err {e:.2e}, min cos {cos:.6f}")
    assert e <= 1e-2 and cos >= 0.9999


def test_vit_tower_full_depth(gpu):
    from omniserver_amd import synth
    say("vit tower depth 32, 16x16 patches")
    cfg, sd, tower = _tower(gpu, 32, 13)
    grids = [(1, 16, 16)]
    pv = synth.pixel_patches(grids, cfg.patch_dim, 14)
    got = tower(pv.to(gpu), grids).cpu().float()
    want = vref.vit_forward(pv.float(), grids, sd)
    cos = torch.nn.functional.cosine_similarity(got, want, dim=-1).min().item()
    e = rel_err(got, want)
    say(f"depth 32: max rel err {e:.2e}, min cos {cos:.6f}")
    assert e <= 3e-2 and cos >= 0.999


def test_runner_pixel_inputs_match_oracle(gpu):
    """Image+text requests given as pixel patches (PixelInput) go through the adapter's
    vision tower (models/qwen2_vl.py:96-97, runners/multimodal.py:124-126): the greedy
    streams equal those of the same requests given the tower's rows as VisionInput, and the
    packed prefill's logits with the tower's rows equal the oracle's with the vision
    oracle's rows (splice at the image tokens, M-RoPE positions)."""
    from tests.helpers import check_ids, compare_logits, oracle_from_gptq
    from omniserver_amd import synth
    from omniserver_amd.kv_cache import PreallocatedKVCache
    from omniserver_amd.positions import IMAGE_TOKEN_ID, VISION_START_TOKEN_ID
    from omniserver_amd.request import PixelInput, Request, SamplingParams, Sequence, VisionInput
    from omniserver_amd.runner import NativeQwenVLRunner
    from omniserver_amd.vit import VisionConfig
    from oracle import qwen2_ref as ref
    say("runner with pixel inputs (vision depth 2, gptq decoder 2 layers)")
    shape = synth.DecoderShape()
    w = synth.gptq_decoder(shape, seed=21, num_layers=2)
    vsd = synth.vision_tower(VisionConfig(), seed=22, depth=2)
    grids = [(1, 8, 8), (1, 4, 6)]
    prompts, pixels = [], []
    for s, g in enumerate(grids):
        n_img = g[0] * g[1] * g[2] // 4
        prompts.append(synth.random_ids(7 + s, shape.vocab_size, 21, f"a{s}").tolist()
                       + [VISION_START_TOKEN_ID] + [IMAGE_TOKEN_ID] * n_img
                       + synth.random_ids(5, shape.vocab_size, 21, f"b{s}").tolist())
        pixels.append(synth.pixel_patches([g], VisionConfig().patch_dim, 23 + s))

    def run(images_of):
        r = NativeQwenVLRunner(max_running=2, max_len=128, use_graph=True, quant="gptq",
                               weights=w, vision=vsd)
        seqs = [Sequence(Request(prompt=p, images=images_of(r, i),
                                 sampling=SamplingParams(max_new_tokens=16)))
                for i, p in enumerate(prompts)]
        r.prefill(seqs)
        for _ in range(5):
            r.decode(seqs)
        return r, [s.output_token_ids for s in seqs]

    runner, pix = run(lambda r, i: [PixelInput(pixels[i].to(gpu), grids[i])])
    _, rows = run(lambda r, i: [VisionInput(r.adapter.vision(pixels[i].to(gpu), [grids[i]]),
                                            grids[i])])
    assert pix == rows and all(len(t) == 6 for t in pix)

    # packed prefill logits of both prompts: tower rows (GPU) vs vision-oracle rows (CPU)
    from oracle import qwen2_vit_ref as vr
    ad = runner.adapter
    emb_g, emb_o, pos_all, segs = [], [], [], []
    for p, g, pv in zip(prompts, grids, pixels):
        ids = torch.tensor(p)
        mask = ids == IMAGE_TOKEN_ID
        eg = ad.embed_tokens(ids.to(gpu))
        eg[mask.to(gpu)] = ad.vision_embed([PixelInput(pv.to(gpu), g)])
        eo = w["embed"][ids].float()
        eo[mask] = vr.vit_forward(pv.float(), [g], vsd)
        pos, _ = ad.prefill_positions(p, [g])
        emb_g.append(eg)
        emb_o.append(eo)
        pos_all.append(pos)
        segs.append(len(p))
    pos = torch.cat(pos_all, 1)
    pool = PreallocatedKVCache(2, 3, 2, 128, 128, gpu, n_heads=12)
    last = (torch.tensor(segs).cumsum(0) - 1).tolist()
    logits = ad.llm(torch.cat(emb_g).unsqueeze(0), pos.to(gpu).unsqueeze(1), None,
                    pool.packed_prefill_cache([0, 1], segs), logits_indices=last)[0]
    kp = [torch.zeros(3, 128, 2, 128) for _ in range(2)]
    vp = [torch.zeros(3, 128, 2, 128) for _ in range(2)]
    exp = oracle_from_gptq(w, shape).prefill(torch.cat(emb_o), pos, segs, [0, 1], kp, vp,
                                             torch.zeros(3, dtype=torch.int64))
    err, cos = compare_logits(logits, exp)
    check_ids(torch.tensor([t[0] for t in pix]), exp, err)
    say(f"  prefill logits vs oracle: max-abs {err:.2e} cos {cos:.6f}")


@pytest.mark.parametrize("M,N,K,epi,bias", [(300, 3840, 1280, 0, True), (257, 5120, 1280, 4, True),
                                            (75, 5120, 5120, 5, True), (1024, 1280, 5120, 6, True),
                                            (64, 1280, 1280, 6, False)])
def test_packed_equals_rows_layout(gpu, M, N, K, epi, bias):
    """omni_f16_gemm_pipe_packed (the tower's linears, packed weights) equals
    omni_f16_gemm_pipe on the nn.Linear-layout weight bit for bit, at the same tile height
    and K slices (the same k order per output), every epilogue."""
    from omniserver_amd import vit
    from omniserver_amd._lib import call, ptr, stream
    say(f"packed vs row-layout pipe GEMM M={M} N={N} K={K} epi={epi}")
    x, w = f16((M, K), 31).to(gpu), f16((N, K), 32, 0.02).to(gpu)
    b = f16((N,), 33, 0.02).to(gpu) if bias else None
    res = f16((M, N), 34).to(gpu)
    lin = vit.VisionLinear(w, b, gpu)
    for tile_rows, ks in ((128, 1), (256, 2), (128, 3)):
        if K // 128 // ks < 2:
            continue
        ws = torch.empty(ks * M * N, device=gpu, dtype=torch.float32)
        outs = []
        for packed in (True, False):
            o = res.clone() if epi == vit.EPI_RESID else torch.empty(M, N, device=gpu, dtype=torch.float16)
            name = "omni_f16_gemm_pipe_packed" if packed else "omni_f16_gemm_pipe"
            call(name, ptr(x), K, ptr(lin.w if packed else w), ptr(b), ptr(o) if epi == vit.EPI_RESID else None,
                 N, ptr(o), N, M, N, K, epi, tile_rows, ks, ptr(ws), stream())
            outs.append(o.cpu())
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), (tile_rows, ks)


@pytest.mark.parametrize("M,N,K,bias", [(1024, 1280, 5120, True), (1024, 1280, 1280, True),
                                        (300, 1280, 1280, False), (7, 1280, 5120, True)])
def test_layernorm_partials(gpu, M, N, K, bias):
    """proj / fc2 leaving their K slices (out_partial, the library's plan) and the next
    LayerNorm adding them (layer_norm_partials_out: slices in order, the bias before the fp16
    rounding, the residual after) equal the same GEMM finished with the residual epilogue at
    the same slice count followed by the plain LayerNorm, bit for bit: the new residual rows
    and the normalised rows."""
    from omniserver_amd import vit
    say(f"layernorm over partials M={M} N={N} K={K} bias={bias}")
    x, w = f16((M, K), 41).to(gpu), f16((N, K), 42, 0.02).to(gpu)
    b = f16((N,), 43, 0.02).to(gpu) if bias else None
    res = f16((M, N), 44).to(gpu)
    g, gb = (1.0 + 0.1 * f16((N,), 45)).to(gpu), f16((N,), 46, 0.1).to(gpu)
    lin = vit.VisionLinear(w, b, gpu)
    parts, S = lin.out_partial(x, torch.empty(16 * M * N, device=gpu, dtype=torch.float32))
    r2, h2 = res.clone(), torch.empty(M, N, device=gpu, dtype=torch.float16)
    vit.layer_norm_partials_out(parts, S, lin.bias, r2, g, gb, 1e-6, h2)
    r1, h1 = res.clone(), torch.empty(M, N, device=gpu, dtype=torch.float16)
    lin.out(x, r1, vit.EPI_RESID, res=r1, ksplit=S)
    vit.layer_norm_out(r1, g, gb, 1e-6, h1)
    torch.cuda.synchronize()
    say(f"  {S} slices")
    assert torch.equal(r1.cpu(), r2.cpu()) and torch.equal(h1.cpu(), h2.cpu())
    # and against the oracle's x + linear, then LayerNorm
    want_r = vref.r16(res.cpu().float() + vref.linear(x.cpu().float(), w.cpu().float(),
                                                       None if b is None else b.cpu().float()))
    assert (r2.cpu().float() - want_r).abs().max().item() <= 2e-3 * max(1.0, want_r.abs().max().item())


@pytest.mark.parametrize("M,epi,bias", [(1024, 4, True), (1024, 0, True), (1024, 5, True),
                                         (1024, 6, True), (1024, 0, False), (1000, 4, True),
                                         (1000, 6, True)])
def test_n160_tiles_equal_128_column_tiles(gpu, M, epi, bias):
    """The vision tower's fc1 shape (1024 x 1280 -> 5120, and a ragged 1000 rows) on the
    library's own plan (128 x 160 tiles, one per CU) equals the forced 256 x 128 tiles bit for
    bit, every biased epilogue (the same K order per output and the same epilogue
    arithmetic); rows past M untouched."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd import vit
    import ctypes
    from omniserver_amd._lib import lib
    K, N = 1280, 5120
    r, c, k = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    lib().omni_packed_gemm_pipe_plan(M, N, K, 1, epi, int(bias), 0, 0, ctypes.byref(r), ctypes.byref(c), ctypes.byref(k))
    assert (r.value, c.value, k.value) == (128, 160, 1)
    say(f"n160 tiles M={M} epi={epi} bias={bias}")
    x, w = f16((M, K), 51).to(gpu), f16((N, K), 52, 0.02).to(gpu)
    b = f16((N,), 53, 0.02).to(gpu) if bias else None
    res = f16((M, N), 54).to(gpu)
    lin = vit.VisionLinear(w, b, gpu)
    outs = []
    for tile_rows in (0, 256):
        # one spare row past M: the tiles' ragged last rows must not store there
        o = torch.full((M + 1, N), float("nan"), device=gpu, dtype=torch.float16)
        if epi == vit.EPI_RESID:
            o[:M] = res
        call("omni_f16_gemm_pipe_packed", ptr(x), K, ptr(lin.w), ptr(b), ptr(o) if epi == vit.EPI_RESID else None,
             N, ptr(o), N, M, N, K, epi, tile_rows, 1, None, stream())
        outs.append(o.cpu())
    torch.cuda.synchronize()
    assert not torch.isnan(outs[0][:M]).any() and torch.isnan(outs[0][M]).all()
    assert torch.equal(outs[0][:M], outs[1][:M])
