"""Pins the CPU oracle (oracle/qwen2_ref.py) without trusting its own formulas.

The reference ships no golden vectors, fixtures or known-answer tests for this path
(its checks compare against HF weights on a CUDA GPU), so each oracle function is
pinned by something independent of how it is written:

  rms_norm / add_rms_norm   float64 numpy closed form; residual rounding = numpy fp16 add
  add_rms_norm_fp8          scale closed form; dequantised codes within one e4m3 step;
                            the row maximum maps to exactly +-448
  silu_mul                  float64 numpy closed form
  apply_mrope (t = h = w)   textbook RoPE as a complex rotation of (x_d, x_{d+64}) by
                            p * fp16(1/theta^(2d/128)) (the .half() module's buffer)
  apply_mrope (3-D)         each section follows only its own axis (dims [0,16)+[64,80) ->
                            t, [16,40)+[80,104) -> h, [40,64)+[104,128) -> w)
  mrope_position_ids        text-only = arange / delta 0; BASELINE.json config-5 closed form
                            (image t=64, h=w=64+0..15, text resumes at 80, delta -240);
                            two images; product implementation equal
  gptq pack/dequant         bit-level brute force with Python ints; round trip
  decode_attention          float64 brute-force softmax loops; the fp16-probability option
                            exact where every probability is a power of two
  prefill_attention         brute force; last token of a segment == decode over it
  fp8 linear                torch._scaled_mm (library GEMM) on the same fp8 operands;
                            both FP8Linear forms and the FP8 MLP routes against the
                            reference's own modules: tests/test_oracle_fp8.py
  rounding points           torch fp16 / bf16 CPU ops evaluating the reference's expressions:
                            the GPTQ bias add (marlin_linear.py:62), forward_prequant's bias
                            (fp8_linear.py:106-107), apply_mrope (qwen2_llm.py:64-72)
  decode_step / prefill     append consistency: prefill(p[:L]) + decode(p[L]) gives the
                            logits prefill(p[:L+1]) gives at its last position
  greedy                    lowest index wins ties
"""

import math

import numpy as np
import pytest
import torch

from oracle import qwen2_ref as ref


def rnd(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * std


# ----------------------------------------------------------------------------- norms
def test_rms_norm_closed_form():
    x = rnd((5, 64), 1).half().float()
    w = (1 + 0.1 * rnd((64,), 2)).half().float()
    y = ref.rms_norm(x, w, 1e-6, f16=False)
    xn = x.double().numpy()
    e = xn / np.sqrt((xn ** 2).mean(-1, keepdims=True) + 1e-6) * w.double().numpy()
    assert np.abs(y.numpy() - e).max() < 1e-5


def test_add_rms_norm_residual_is_fp16_sum():
    x = rnd((4, 96), 3).half()
    r = rnd((4, 96), 4).half()
    _, nr = ref.add_rms_norm(x.float(), r.float(), torch.ones(96), 1e-6)
    e = (x.numpy().astype(np.float16) + r.numpy().astype(np.float16)).astype(np.float32)
    assert np.array_equal(nr.numpy(), e)


def test_add_rms_norm_fp8():
    x = rnd((6, 128), 5).half().float()
    r = rnd((6, 128), 6).half().float()
    q, s, nr = ref.add_rms_norm_fp8(x, r, torch.ones(128), 1e-6)
    y = ref.rms_norm(nr, torch.ones(128), 1e-6, f16=False)
    assert torch.allclose(s.view(-1), y.abs().amax(-1) / 448.0, rtol=1e-6)
    deq = q.float() * s
    assert ((deq - y).abs() <= 2.0 ** -4 * y.abs() + s * 2.0 ** -9).all()
    assert (q.float().abs().amax(-1) == 448.0).all()


def test_silu_mul_closed_form():
    gu = rnd((3, 20), 7, 3.0)
    y = ref.silu_mul(gu, f16=False).numpy()
    g, u = gu[:, :10].double().numpy(), gu[:, 10:].double().numpy()
    assert np.abs(y - g / (1 + np.exp(-g)) * u).max() < 1e-5


# ----------------------------------------------------------------------------- rope
def test_mrope_equals_textbook_rope_when_axes_agree():
    cfg = ref.Qwen2Config()
    T, nh = 7, 3
    pos = torch.tensor([0, 1, 5, 100, 1023, 4000, 77])
    q = rnd((1, nh, T, 128), 8)
    k = rnd((1, 1, T, 128), 9)
    cos, sin = ref.rope_cos_sin(pos.view(1, 1, T).expand(3, 1, T), cfg, f16=False)
    qr, kr = ref.apply_mrope(q, k, cos, sin, cfg.mrope_section, f16=False)
    # the deployed module's inverse frequencies: the fp16 rounding of 1/theta^(2j/128)
    inv = (1.0 / (1e6 ** (np.arange(0, 128, 2) / 128.0))).astype(np.float16).astype(np.float64)
    for x, xr in ((q, qr), (k, kr)):
        xn = x.double().numpy()
        z = xn[..., :64] + 1j * xn[..., 64:]
        ang = pos.double().numpy()[:, None] * inv[None, :]
        rot = z * np.exp(1j * ang)[None, None]
        e = np.concatenate([rot.real, rot.imag], -1)
        assert np.abs(xr.double().numpy() - e).max() < 2e-3   # fp32 angle rounding at p~4000


def test_mrope_sections_follow_their_axis():
    cfg = ref.Qwen2Config()
    q = rnd((1, 1, 1, 128), 10)
    k = rnd((1, 1, 1, 128), 11)
    base = torch.tensor([10, 10, 10]).view(3, 1, 1)
    c0, s0 = ref.rope_cos_sin(base, cfg, f16=False)
    q0, _ = ref.apply_mrope(q, k, c0, s0, cfg.mrope_section, f16=False)
    spans = {0: list(range(0, 16)) + list(range(64, 80)),
             1: list(range(16, 40)) + list(range(80, 104)),
             2: list(range(40, 64)) + list(range(104, 128))}
    for axis in range(3):
        p = base.clone()
        p[axis] = 37
        c, s = ref.rope_cos_sin(p, cfg, f16=False)
        q1, _ = ref.apply_mrope(q, k, c, s, cfg.mrope_section, f16=False)
        changed = set((q1 != q0).view(-1).nonzero().view(-1).tolist())
        assert changed == set(spans[axis]), axis


def test_mrope_positions_text_only():
    pos, d = ref.mrope_position_ids(list(range(10)), [])
    assert torch.equal(pos, torch.arange(10).view(1, -1).expand(3, -1)) and d == 0


def test_mrope_positions_config5_closed_form():
    # 63 text tokens, <|vision_start|>, 256 image tokens, 192 text tokens (the vision-start
    # token is the 64th text token: positions.py:27-30 counts an image only after one)
    ids = [5] * 63 + [151652] + [151655] * 256 + [6] * 192
    pos, d = ref.mrope_position_ids(ids, [(1, 32, 32)])
    assert torch.equal(pos[:, :64], torch.arange(64).view(1, -1).expand(3, -1))
    img = pos[:, 64:320]
    assert (img[0] == 64).all()
    assert torch.equal(img[1], 64 + torch.arange(16).repeat_interleave(16))
    assert torch.equal(img[2], 64 + torch.arange(16).repeat(16))
    assert torch.equal(pos[:, 320:], (80 + torch.arange(192)).view(1, -1).expand(3, -1))
    assert d == 272 - 512 == -240


def test_mrope_positions_two_images_and_product_agree():
    from omniserver_amd.positions import mrope_positions
    S, I = 151652, 151655
    ids = [1, S] + [I] * 4 + [S] + [I] * 9 + [4, 5]
    grids = [(1, 4, 4), (1, 6, 6)]
    pos, d = ref.mrope_position_ids(ids, grids)
    # image 1 at positions 2..3, vision-start at 4, image 2 at 5..7, text at 8, 9
    assert pos[:, 6].tolist() == [4, 4, 4]
    assert pos[:, 7:16].max().item() == 7
    assert pos[:, 16:].tolist() == [[8, 9]] * 3 and d == 10 - 18
    p2, d2 = mrope_positions(ids, grids)
    assert torch.equal(pos, p2) and d == d2


def test_mrope_positions_random_layouts_agree():
    """The product's positions (cached per-grid offsets, running maximum) equal the oracle's
    on random layouts: 0-3 images of t = 1-2 frames and even h, w, text of any length
    before, between and after (none too), a stray image token without a vision-start, and
    prompts given as lists or int64 arrays."""
    from omniserver_amd.positions import mrope_positions
    S, I = 151652, 151655
    g = np.random.default_rng(7)
    for case in range(60):
        ids, grids = [], []
        for _ in range(int(g.integers(0, 4))):
            ids += [int(x) for x in g.integers(0, 1000, int(g.integers(0, 6)))]
            t, h, w = int(g.integers(1, 3)), 2 * int(g.integers(1, 5)), 2 * int(g.integers(1, 5))
            ids += [S] + [I] * (t * (h // 2) * (w // 2))
            grids.append((t, h, w))
        ids += [int(x) for x in g.integers(0, 1000, int(g.integers(0, 6)))]
        if case % 7 == 3:
            ids += [I]                                   # no vision-start before it: text
        if not ids:
            ids = [1]
        pos, d = ref.mrope_position_ids(ids, grids)
        for arg in (ids, np.asarray(ids, dtype=np.int64)):
            p2, d2 = mrope_positions(arg, grids)
            assert torch.equal(pos, p2) and d == d2, case


def test_mrope_positions_image_without_vision_start_is_text():
    """positions.py:27-30 counts images by vision-start tokens followed by an image token:
    a prompt whose image run has none gets 1-D text positions."""
    from omniserver_amd.positions import mrope_positions
    ids = [1, 2] + [151655] * 4 + [3]
    for pos, d in (ref.mrope_position_ids(ids, [(1, 4, 4)]), mrope_positions(ids, [(1, 4, 4)])):
        assert torch.equal(pos, torch.arange(7).view(1, -1).expand(3, -1)) and d == 0


# ----------------------------------------------------------------------------- int4
def test_gptq_pack_dequant_bit_level():
    K, N = 256, 3
    g = torch.Generator().manual_seed(12)
    codes = torch.randint(0, 16, (K, N), generator=g)
    qw = ref.gptq_pack(codes)
    assert torch.equal(ref.gptq_unpack(qw), codes)
    scales = (rnd((K // 128, N), 13).abs() * 0.003).half()
    W = ref.gptq_dequant(qw, scales)
    for k in (0, 1, 7, 8, 127, 128, 255):
        for n in range(N):
            word = int(qw[k // 8, n]) & 0xFFFFFFFF
            q = (word >> (4 * (k % 8))) & 0xF
            s = float(scales[k // 128, n])
            e = float(np.float16(np.float32((q - 8)) * np.float32(s)))
            assert float(W[k, n]) == e


# ----------------------------------------------------------------------------- attention
def _brute_attention(q, K, V, scale):
    s = [sum(q[d] * K[j][d] for d in range(len(q))) * scale for j in range(len(K))]
    m = max(s)
    p = [math.exp(x - m) for x in s]
    z = sum(p)
    return [sum(p[j] * V[j][d] for j in range(len(K))) / z for d in range(len(V[0]))]


def test_decode_attention_brute_force():
    n, nh, nkv, hd, ML = 2, 4, 2, 8, 16
    q = rnd((n, nh, hd), 14)
    kp = rnd((3, ML, nkv, hd), 15)
    vp = rnd((3, ML, nkv, hd), 16)
    rows, L = torch.tensor([2, 0]), torch.tensor([5, 11])
    out = ref.decode_attention(q, kp, vp, rows, L, 0.3, f16=False)
    for b in range(n):
        for h in range(nh):
            g = h // (nh // nkv)
            e = _brute_attention(q[b, h].tolist(), kp[rows[b], :L[b], g].tolist(),
                                 vp[rows[b], :L[b], g].tolist(), 0.3)
            assert np.allclose(out[b, h].numpy(), e, atol=1e-5)


def test_prefill_attention_causal_and_consistent_with_decode():
    nh, nkv, hd = 4, 2, 8
    segs = [5, 3]
    T = sum(segs)
    q, k, v = rnd((T, nh, hd), 17), rnd((T, nkv, hd), 18), rnd((T, nkv, hd), 19)
    out = ref.prefill_attention(q, k, v, segs, 0.25, f16=False)
    # token 3 of segment 0 sees keys 0..3 only
    for h in range(nh):
        g = h // 2
        e = _brute_attention(q[3, h].tolist(), k[:4, g].tolist(), v[:4, g].tolist(), 0.25)
        assert np.allclose(out[3, h].numpy(), e, atol=1e-5)
    # last token of segment 1 == decode attention over segment 1
    kp = torch.zeros(1, 8, nkv, hd)
    vp = torch.zeros(1, 8, nkv, hd)
    kp[0, :3], vp[0, :3] = k[5:], v[5:]
    d = ref.decode_attention(q[7:8], kp, vp, torch.tensor([0]), torch.tensor([3]), 0.25, f16=False)
    assert torch.allclose(out[7], d[0], atol=1e-6)


def test_attention_fp16_probabilities_option():
    """The flash-rounding option of both attentions (p16): where every unnormalised
    probability exp(s - max) is a power of two (scores integer multiples of ln 2) the fp16
    rounding is exact and the result equals the exact softmax; on generic scores it moves
    each output by at most one fp16 rounding of each probability (relative 2^-11 of the
    sum of |p v|)."""
    L, hd = 9, 128
    ln2 = math.log(2.0)
    # q = e_0 * c, k_j = e_0 * (-j ln2 / c) / scale: scores s_j = -j ln 2
    scale, c = 0.25, 2.0
    q = torch.zeros(1, 1, hd)
    q[0, 0, 0] = c
    k = torch.zeros(1, L + 1, 1, hd)
    for j in range(L):
        k[0, j, 0, 0] = -j * ln2 / (c * scale)
    v = rnd((1, L + 1, 1, hd), 60)
    ex = ref.decode_attention(q, k, v, torch.tensor([0]), torch.tensor([L]), scale, f16=False)
    p16 = ref.decode_attention(q, k, v, torch.tensor([0]), torch.tensor([L]), scale, f16=False,
                               p16=True)
    assert torch.allclose(ex, p16, rtol=1e-6, atol=1e-7)
    # generic scores: within one fp16 rounding per probability
    q2 = rnd((3, 4, hd), 61, 0.3)
    k2 = rnd((3, 40, 2, hd), 62)
    v2 = rnd((3, 40, 2, hd), 63)
    lens = torch.tensor([40, 17, 1])
    a = ref.decode_attention(q2, k2, v2, torch.arange(3), lens, 0.1, f16=False)
    b = ref.decode_attention(q2, k2, v2, torch.arange(3), lens, 0.1, f16=False, p16=True)
    bound = 2.0 ** -11 * 4.0         # |v| <~ 4: sum_j p_j |v_j| <= max |v|
    assert (a - b).abs().max().item() <= bound and not torch.equal(a, b)
    # the prefill form: the last query of a segment is the decode form over it
    qs, ks, vs = rnd((6, 4, hd), 64, 0.3), rnd((6, 2, hd), 65), rnd((6, 2, hd), 66)
    pf = ref.prefill_attention(qs, ks, vs, [6], 0.1, f16=False, p16=True)
    kp = torch.zeros(1, 6, 2, hd)
    vp = torch.zeros(1, 6, 2, hd)
    kp[0], vp[0] = ks, vs
    dc = ref.decode_attention(qs[5:6], kp, vp, torch.tensor([0]), torch.tensor([6]), 0.1,
                              f16=False, p16=True)
    assert torch.allclose(pf[5], dc[0], atol=1e-6)


# ----------------------------------------------------------------------------- fp8
def test_fp8_linear_matches_scaled_mm():
    x = rnd((16, 64), 20).half().float()
    w = rnd((32, 64), 21, 0.02).half().float()
    wq, sw = ref.fp8_weight_rowwise(w)
    xq, sa = ref.quant_fp8(x)
    y = ref.fp8_linear_rowwise(xq, sa, wq, sw, out_f16=False)
    # the library fp8 GEMM (per-tensor unit scales, fp32 out) on the same e4m3 operands,
    # then the row / column scales and the bf16 rounding of the reference's epilogue
    one = torch.tensor(1.0)
    try:
        acc = torch._scaled_mm(xq, wq.t(), scale_a=one, scale_b=one, out_dtype=torch.float32)
    except (RuntimeError, NotImplementedError) as err:
        pytest.skip(f"CPU _scaled_mm unavailable: {err}")
    e = (acc * sa.view(-1, 1) * sw.view(1, -1)).to(torch.bfloat16).float()
    assert torch.allclose(y, e, atol=0, rtol=2 ** -7)
    # scales follow the closed forms; the weight's is an op on the reference's fp16 tensor
    assert torch.equal(sw, (w.half().abs().amax(1) / 448.0).float())
    assert torch.allclose(sa.view(-1), x.abs().amax(1) / 448.0)


# ----------------------------------------------------------------------------- rounding points
def test_gptq_bias_added_after_the_fp16_output():
    """_MarlinBase.forward returns ``out + self.bias`` on the fp16 GEMM output
    (marlin_linear.py:59-62): two roundings, evaluated here by torch's fp16 add."""
    x = rnd((9, 256), 30).half().float()
    w = rnd((256, 64), 31, 0.05).half().float()
    b = rnd((64,), 32, 0.5).half()
    y = ref.linear(x, w, b.float(), bias_after_round=True)
    want = (x @ w).half() + b
    assert torch.equal(y, want.float())
    # and it is a different rounding from the fp16 nn.Linear's single one on some outputs
    assert not torch.equal(y, ref.linear(x, w, b.float(), bias_after_round=False))


def test_fp8_prequant_bias_in_bf16():
    """forward_prequant adds bias.to(bf16) to the bf16 _scaled_mm output (fp8_linear.py:106-107)."""
    x = rnd((8, 128), 33).half().float()
    w = rnd((64, 128), 34, 0.02).half().float()
    b = rnd((64,), 35, 0.3).half()
    wq, sw = ref.fp8_weight_rowwise(w)
    xq, sa = ref.quant_fp8(x)
    y = ref.fp8_linear_prequant(xq, sa, wq, sw, b.float())
    prod = ((xq.float() @ wq.float().t()) * sa * sw.view(1, -1)).to(torch.bfloat16)
    assert torch.equal(y, (prod + b.to(torch.bfloat16)).float())


def test_apply_mrope_fp16_expression():
    """apply_mrope's ``(q * cos) + (rotate_half(q) * sin)`` on fp16 tensors
    (qwen2_llm.py:64-72, cos/sin cast to fp16 at :181) evaluated by torch's fp16 ops."""
    cfg = ref.Qwen2Config()
    q = rnd((1, 3, 5, 128), 36).half()
    k = rnd((1, 2, 5, 128), 37).half()
    pos = torch.tensor([[[0, 9, 300, 2047, 4095]], [[0, 8, 301, 2000, 4000]],
                        [[0, 7, 302, 1999, 4001]]])
    cos, sin = ref.rope_cos_sin(pos, cfg)
    qr, kr = ref.apply_mrope(q.float(), k.float(), cos, sin, cfg.mrope_section)
    sec = cfg.mrope_section * 2
    c16 = torch.cat([m[i % 3] for i, m in enumerate(cos.half().split(sec, -1))], -1).unsqueeze(1)
    s16 = torch.cat([m[i % 3] for i, m in enumerate(sin.half().split(sec, -1))], -1).unsqueeze(1)
    rot = lambda x: torch.cat((-x[..., 64:], x[..., :64]), -1)
    assert torch.equal(qr, ((q * c16) + (rot(q) * s16)).float())
    assert torch.equal(kr, ((k * c16) + (rot(k) * s16)).float())


# ----------------------------------------------------------------------------- model
def _tiny(f16=False, seed=22):
    cfg = ref.Qwen2Config(hidden_size=256, num_layers=2, num_heads=2, num_kv_heads=1,
                          head_dim=128, intermediate_size=384, vocab_size=500)
    H, I = cfg.hidden_size, cfg.intermediate_size
    qkv = (cfg.num_heads + 2 * cfg.num_kv_heads) * cfg.head_dim
    layers = [ref.LayerWeights(
        in_norm=torch.ones(H), post_norm=torch.ones(H),
        qkv_t=rnd((H, qkv), seed + 10 * i, 0.05), qkv_b=rnd((qkv,), seed + 10 * i + 1, 0.05),
        o_t=rnd((cfg.num_heads * cfg.head_dim, H), seed + 10 * i + 2, 0.05),
        gate_up_t=rnd((H, 2 * I), seed + 10 * i + 3, 0.05),
        down_t=rnd((I, H), seed + 10 * i + 4, 0.05)) for i in range(cfg.num_layers)]
    return ref.Qwen2Ref(cfg, rnd((cfg.vocab_size, H), seed + 99, 0.05), torch.ones(H), layers,
                        False, f16)


def test_decode_after_prefill_equals_longer_prefill():
    orc = _tiny()
    cfg = orc.cfg
    prompt = torch.randint(0, cfg.vocab_size, (13,), generator=torch.Generator().manual_seed(23))
    L = 12

    def pool():
        return ([torch.zeros(2, 32, 1, 128) for _ in range(2)],
                [torch.zeros(2, 32, 1, 128) for _ in range(2)], torch.zeros(2, dtype=torch.int64))

    kp, vp, lens = pool()
    orc.prefill(orc.embed[prompt[:L]], torch.arange(L).view(1, -1).expand(3, -1), [L], [0], kp, vp,
                lens)
    assert lens[0] == L
    dec = orc.decode_step([int(prompt[L])], kp, vp, lens)
    kp2, vp2, lens2 = pool()
    full = orc.prefill(orc.embed[prompt], torch.arange(L + 1).view(1, -1).expand(3, -1), [L + 1],
                       [0], kp2, vp2, lens2)
    assert torch.allclose(dec, full, atol=1e-4)
    # and the pools agree on the first L+1 positions
    for l in range(2):
        assert torch.allclose(kp[l][0, :L + 1], kp2[l][0, :L + 1], atol=1e-5)


def test_packed_prefill_equals_separate_prefills():
    orc = _tiny()
    g = torch.Generator().manual_seed(24)
    p1 = torch.randint(0, 500, (7,), generator=g)
    p2 = torch.randint(0, 500, (4,), generator=g)

    def run(prompts, slots):
        kp = [torch.zeros(3, 16, 1, 128) for _ in range(2)]
        vp = [torch.zeros(3, 16, 1, 128) for _ in range(2)]
        lens = torch.zeros(3, dtype=torch.int64)
        emb = torch.cat([orc.embed[p] for p in prompts])
        pos = torch.cat([torch.arange(len(p)).view(1, -1).expand(3, -1) for p in prompts], 1)
        return orc.prefill(emb, pos, [len(p) for p in prompts], slots, kp, vp, lens)

    both = run([p1, p2], [0, 1])
    assert torch.allclose(both[0], run([p1], [0])[0], atol=1e-5)
    assert torch.allclose(both[1], run([p2], [1])[0], atol=1e-5)


def test_greedy_lowest_index_on_ties():
    lg = torch.tensor([[1.0, 3.0, 3.0, 2.0], [5.0, 5.0, 5.0, 5.0]])
    assert ref.greedy(lg) == [1, 0]


def test_golden_fixture_reproduced():
    """The committed fixture (tests/golden/make_golden.py) is what the oracle computes."""
    import json
    import os
    import sys
    gdir = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    sys.path.insert(0, gdir)
    import make_golden
    want = json.load(open(os.path.join(gdir, "decode_fp16_2layer.json")))
    got = make_golden.generate()
    assert got["prompts"] == want["prompts"]
    for g, w in zip(got["steps"], want["steps"]):
        for b in range(2):
            if w["margin"][b] > 1e-3:
                assert g["tokens"][b] == w["tokens"][b]
        assert np.allclose(g["top5_logits"], w["top5_logits"], atol=1e-3)


# ----------------------------------------------------------------------------- RTN int4
def _rtn_brute(w16: np.ndarray, group: int):
    """Python-scalar restatement of the RTN rule on fp16 values: per group and column the
    scale max(|max/7|, |min/-8|) in fp16 arithmetic, the quotient w/s rounded to fp16 (the
    reference divides fp16 tensors), then round half to even and clamp to [-8, 7]."""
    K, N = w16.shape
    codes = np.zeros((K, N), dtype=np.int64)
    scales = np.zeros((K // group, N), dtype=np.float16)
    for gi in range(K // group):
        for n in range(N):
            col = w16[gi * group:(gi + 1) * group, n]
            mx, mn = col.max(), col.min()
            s = max(abs(np.float16(mx / np.float16(7))), abs(np.float16(mn / np.float16(-8))))
            scales[gi, n] = s
            for i, v in enumerate(col):
                q = 0 if s == 0 else round(float(np.float16(v / s)))
                codes[gi * group + i, n] = min(max(q, -8), 7) + 8
    return codes, scales


def test_rtn_int4_brute_force_and_bounds():
    """marlin_linear.py:65-80 (vLLM quantize_weights, uint4b8): the oracle's codes and
    scales equal a scalar brute force; every dequantised weight is within s/2 of its fp16
    value (plus the fp16 rounding of the product); the dominating extreme of each group
    maps to code 15 (max/7 side) or 0 (min/-8 side); an all-zero group gives code 8."""
    N, K, G = 6, 256, 128
    w = (rnd((N, K), 40) * 0.02).half()
    w[2, :128] = 0                                   # an all-zero group
    qw, s = ref.rtn_int4(w.float(), G)
    codes = ref.gptq_unpack(qw)
    bc, bs = _rtn_brute(w.t().numpy().astype(np.float16), G)
    assert np.array_equal(codes.numpy(), bc)
    assert np.array_equal(s.numpy().astype(np.float16), bs)
    deq = ref.gptq_dequant(qw, s.half(), G)                       # [K, N]
    wt = w.t().float()
    srep = s.repeat_interleave(G, 0)
    assert ((deq - wt).abs() <= srep / 2 + wt.abs() * 2.0 ** -10 + 1e-8).all()
    for gi in range(K // G):
        for n in range(N):
            col = wt[gi * G:(gi + 1) * G, n]
            cc = codes[gi * G:(gi + 1) * G, n]
            if col.abs().max() == 0:
                assert (cc == 8).all()
                continue
            up = col.max().item() / 7 >= -col.min().item() / 8
            assert cc[col.argmax()] == 15 if up else cc[col.argmin()] == 0
