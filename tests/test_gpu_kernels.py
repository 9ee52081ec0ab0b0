"""Kernel-level parity of the HIP path against the CPU oracle (GPU tests).

Each test feeds the same seeded fp16 inputs to the HIP kernel (through the C ABI
via omniserver_amd's thin wrappers) and to oracle/qwen2_ref.py, and compares:
bit-exact for integer/byte/index work and for the fp16-rounding-specified ops
(M-RoPE, embedding gather, int4 dequant, KV writes), tolerance for reductions.
"""

import math

import pytest
import torch

from oracle import qwen2_ref as ref

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)


def f16(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(torch.float16)


# ----------------------------------------------------------------------------- norms
@pytest.mark.parametrize("rows", [1, 5, 32, 257])
def test_add_rmsnorm(gpu, rows):
    from omniserver_amd import fused_ops as F
    say(f"add_rmsnorm rows={rows}")
    H = 1536
    x, r = f16((rows, H), 1), f16((rows, H), 2)
    w = (1.0 + 0.1 * f16((H,), 3).float()).to(torch.float16)
    y, nr = F.add_rms_norm(x.to(gpu), r.to(gpu), w.to(gpu), 1e-6)
    ey, er = ref.add_rms_norm(x.float(), r.float(), w.float(), 1e-6)
    assert torch.equal(nr.cpu().float(), er)                 # residual add: exact fp16
    d = (y.cpu().float() - ey).abs()
    assert d.max().item() <= 2e-3 * max(1.0, ey.abs().max().item())
    assert (d > 0).float().mean().item() < 0.02              # almost all bit-equal


def test_rmsnorm_and_embed(gpu):
    from omniserver_amd import fused_ops as F
    say("rmsnorm / embedding gather (plain + packed) / embed_rmsnorm")
    V, H = 4096, 1536
    table = f16((V, H), 7, 0.02)
    ids = torch.tensor([0, 5, 4095, 17, 1000], dtype=torch.int64)
    w = torch.ones(H, dtype=torch.float16)
    y = F.rms_norm(table[ids].to(gpu), w.to(gpu), 1e-6)
    ey = ref.rms_norm(table[ids].float(), w.float(), 1e-6)
    assert (y.cpu().float() - ey).abs().max().item() <= 2e-3 * ey.abs().max().item()

    from omniserver_amd.linear import LMHeadArgmax
    lm = LMHeadArgmax(table.to(gpu))
    out = torch.empty(len(ids), H, device=gpu, dtype=torch.float16)
    F.embedding_out(ids.to(gpu), lm.table_packed, True, out)
    assert torch.equal(out.cpu(), table[ids])
    out2 = torch.empty_like(out)
    F.embedding_out(ids.to(gpu), table.to(gpu), False, out2)
    assert torch.equal(out2.cpu(), table[ids])
    h = torch.empty_like(out)
    res = torch.empty_like(out)
    F.embed_rms_norm_out(ids.to(gpu), lm.table_packed, True, w.to(gpu), 1e-6, h, res)
    assert torch.equal(res.cpu(), table[ids])
    assert torch.equal(h.cpu(), y.cpu())
    # the decode step's first launch also writes each row's rotary row: the cos | sin table
    # rows at lengths + delta (clamped), bit-equal to indexing the tables
    from omniserver_amd.qwen2_llm import rope_tables
    cos, sin = rope_tables(ref.Qwen2Config(), 512, gpu)
    lens = torch.tensor([0, 37, 511, 600, 200], dtype=torch.int64)
    delta = torch.tensor([0, -5, 3, 0, -300], dtype=torch.int64)
    rows = torch.empty(len(ids), 128, device=gpu, dtype=torch.float16)
    h2, res2 = torch.empty_like(out), torch.empty_like(out)
    F.embed_rms_norm_rope_out(ids.to(gpu), lm.table_packed, True, w.to(gpu), 1e-6, h2, res2,
                              lens.to(gpu), delta.to(gpu), cos, sin, rows)
    assert torch.equal(h2.cpu(), h.cpu()) and torch.equal(res2.cpu(), res.cpu())
    pos = (lens + delta).clamp(0, 511)
    assert torch.equal(rows.cpu(), torch.cat([cos.cpu()[pos], sin.cpu()[pos]], 1))


def test_add_rmsnorm_fp8(gpu):
    from omniserver_amd import fused_ops as F
    say("add_rmsnorm_fp8")
    M, H = 64, 1536
    x, r = f16((M, H), 11), f16((M, H), 12)
    w = torch.ones(H, dtype=torch.float16)
    q, s, nr = F.add_rms_norm_fp8(x.to(gpu), r.to(gpu), w.to(gpu), 1e-6)
    eq, es, er = ref.add_rms_norm_fp8(x.float(), r.float(), w.float(), 1e-6)
    assert torch.equal(nr.cpu().float(), er)
    assert torch.allclose(s.cpu(), es, rtol=1e-5, atol=0)
    qd, eqd = q.cpu().float(), eq.float()
    mism = (q.cpu().view(torch.uint8) != eq.view(torch.uint8)).float().mean().item()
    assert mism < 0.01
    # any mismatch is one e4m3 step: relative difference <= 2^-3
    assert ((qd - eqd).abs() <= 0.125 * eqd.abs() + 2.0 ** -9).all()


def test_silu_mul(gpu):
    from omniserver_amd import fused_ops as F
    say("silu_mul")
    gu = f16((7, 2 * 8960), 21, 2.0)
    y = F.silu_mul(gu.to(gpu)).cpu().float()
    ey = ref.silu_mul(gu.float())
    d = (y - ey).abs()
    assert d.max().item() <= 1e-3 * max(1.0, ey.abs().max().item())


# ----------------------------------------------------------------------------- rope + kv
@pytest.mark.parametrize("T", [1, 3, 32])
def test_mrope_kv_write_decode(gpu, T):
    """Decode form: positions = lengths[row] + rope_delta[row] on all three axes;
    rotated K and raw V land at pool[row, lengths[row]].  Bit-exact vs the oracle."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd.qwen2_llm import rope_tables
    say(f"mrope_kv_write decode T={T}")
    cfg = ref.Qwen2Config()
    nh, nkv, hd = 12, 2, 128
    P, ML = T + 1, 64
    qkv = f16((T, (nh + 2 * nkv) * hd), 31)
    lengths = torch.randint(0, 40, (P,), generator=torch.Generator().manual_seed(2))
    delta = torch.randint(-5, 6, (P,), generator=torch.Generator().manual_seed(3))
    cos, sin = rope_tables(cfg, 256, gpu)
    kc = torch.zeros(P, ML, nkv, hd, dtype=torch.float16, device=gpu)
    vc = torch.zeros_like(kc)
    g = qkv.to(gpu)
    lg, dg = lengths.to(gpu), delta.to(gpu)   # kept alive until the kernel has run
    call("omni_mrope_kv_write", ptr(g), g.stride(0), None, ptr(lg), ptr(dg), ptr(cos),
         ptr(sin), 256, ptr(kc), ptr(vc), None, None, P, ML, T, nh, nkv, hd, 16, 24, 24,
         stream())
    torch.cuda.synchronize()
    pos = (lengths[:T] + delta[:T]).clamp(min=0)
    c, s = ref.rope_cos_sin(pos.view(1, 1, T).expand(3, 1, T), cfg)
    q = qkv[:, :nh * hd].float().view(T, nh, hd).transpose(0, 1).unsqueeze(0)
    k = qkv[:, nh * hd:(nh + nkv) * hd].float().view(T, nkv, hd).transpose(0, 1).unsqueeze(0)
    qr, kr = ref.apply_mrope(q, k, c, s, cfg.mrope_section)
    out = g.cpu().float()
    assert torch.equal(out[:, :nh * hd].view(T, nh, hd), qr[0].transpose(0, 1))
    assert torch.equal(out[:, nh * hd:(nh + nkv) * hd].view(T, nkv, hd), kr[0].transpose(0, 1))
    kcc, vcc = kc.cpu().float(), vc.cpu().float()
    v = qkv[:, (nh + nkv) * hd:].float().view(T, nkv, hd)
    for t in range(T):
        assert torch.equal(kcc[t, lengths[t]], kr[0, :, t])
        assert torch.equal(vcc[t, lengths[t]], v[t])
    # nothing else written
    assert (kcc != 0).sum().item() == (kr[0] != 0).sum().item()


def test_mrope_3d_positions(gpu):
    """Prefill form with distinct t/h/w position ids (image tokens): bit-exact."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd.qwen2_llm import rope_tables
    say("mrope 3-D positions")
    cfg = ref.Qwen2Config()
    nh, nkv, hd = 12, 2, 128
    ids = [1] * 4 + [151655] * 16 + [2] * 3
    pos, delta = ref.mrope_position_ids(ids, [(1, 8, 8)])
    T = len(ids)
    qkv = f16((T, (nh + 2 * nkv) * hd), 41)
    cos, sin = rope_tables(cfg, 64, gpu)
    g = qkv.to(gpu)
    pg = pos.contiguous().to(gpu)
    call("omni_mrope_kv_write", ptr(g), g.stride(0), ptr(pg), None, None, ptr(cos), ptr(sin),
         64, None, None, None, None, 0, 0, T, nh, nkv, hd, 16, 24, 24, stream())
    torch.cuda.synchronize()
    c, s = ref.rope_cos_sin(pos.view(3, 1, T), cfg)
    q = qkv[:, :nh * hd].float().view(T, nh, hd).transpose(0, 1).unsqueeze(0)
    k = qkv[:, nh * hd:(nh + nkv) * hd].float().view(T, nkv, hd).transpose(0, 1).unsqueeze(0)
    qr, kr = ref.apply_mrope(q, k, c, s, cfg.mrope_section)
    out = g.cpu().float()
    assert torch.equal(out[:, :nh * hd].view(T, nh, hd), qr[0].transpose(0, 1))
    assert torch.equal(out[:, nh * hd:(nh + nkv) * hd].view(T, nkv, hd), kr[0].transpose(0, 1))


# ----------------------------------------------------------------------------- attention
@pytest.mark.parametrize("lengths,waves,splits", [
    ([1], 4, 1), ([7], 4, 3), ([33, 64, 100], 4, 1), ([300, 5, 1000], 8, 4), ([2048] * 4, 8, 2),
    ([1, 2, 3, 4095], 4, 16), ([31, 32, 33, 65], 8, 1), ([2049] * 3, 4, 8),
])
def test_decode_attention(gpu, lengths, waves, splits):
    from omniserver_amd._lib import call, ptr, stream
    say(f"decode_attention lengths={lengths} waves={waves} splits={splits}")
    n = len(lengths)
    nh, nkv, hd, ML = 12, 2, 128, 4096
    P = n + 1
    kp = f16((P, ML, nkv, hd), 51)
    vp = f16((P, ML, nkv, hd), 52)
    q = f16((n, nh * hd), 53)
    L = torch.tensor(lengths, dtype=torch.int64)
    out = torch.empty(n, nh, hd, device=gpu, dtype=torch.float16)
    scale = hd ** -0.5
    kg, vg, qg, Lg = kp.to(gpu), vp.to(gpu), q.to(gpu), L.to(gpu)
    ws = torch.empty(n * nkv * splits * 6 * 132, device=gpu, dtype=torch.float32)
    call("omni_decode_attention", ptr(qg), nh * hd, ptr(kg), ptr(vg), P, ML, None, ptr(Lg), 0, 0,
         ptr(out), n, nh, nkv, hd, scale, waves, splits, ptr(ws), ws.numel(), stream())
    torch.cuda.synchronize()
    e = ref.decode_attention(q.float().view(n, nh, hd), kp.float(), vp.float(),
                             torch.arange(n), L, scale)
    d = (out.cpu().float() - e).abs().max().item()
    assert d <= 4e-3, d


@pytest.mark.parametrize("segs", [[1], [5, 16, 17], [256], [100, 37, 512], [33, 64, 511, 2]])
def test_prefill_attention(gpu, segs):
    """Both prefill attention kernels against the oracle, and equal to each other bit for bit
    (query blocks of 16 / 32 tokens; the shared-tile kernel adds only fully masked tiles for
    a block's first rows, which change nothing)."""
    from omniserver_amd.attention import QBLOCK_GQA, query_blocks
    from omniserver_amd._lib import call, ptr, stream
    say(f"prefill_attention segs={segs}")
    nh, nkv, hd, ML = 12, 2, 128, 1024
    P = len(segs)
    T = sum(segs)
    q = f16((T, nh * hd), 61)
    k = f16((T, nkv, hd), 62)
    v = f16((T, nkv, hd), 63)
    kp = torch.zeros(P, ML, nkv, hd, dtype=torch.float16)
    vp = torch.zeros_like(kp)
    slot, pos = [], []
    off = 0
    for s, Ls in enumerate(segs):
        kp[s, :Ls] = k[off:off + Ls]
        vp[s, :Ls] = v[off:off + Ls]
        slot += [s] * Ls
        pos += list(range(Ls))
        off += Ls
    slot_t = torch.tensor(slot, dtype=torch.int64, device=gpu)
    kvl = torch.tensor(pos, dtype=torch.int64, device=gpu) + 1
    qb = query_blocks(segs, gpu)
    out = torch.empty(T, nh, hd, device=gpu, dtype=torch.float16)
    qg, kg, vg = q.to(gpu), kp.to(gpu), vp.to(gpu)
    call("omni_prefill_attention", ptr(qg), nh * hd, ptr(kg), ptr(vg), P, ML, ptr(slot_t),
         ptr(kvl), ptr(qb), qb.shape[0], ptr(out), nh * hd, nh, nkv, hd, hd ** -0.5, stream())
    qb32 = query_blocks(segs, gpu, QBLOCK_GQA)
    out32 = torch.full_like(out, float("nan"))
    call("omni_prefill_attention_gqa", ptr(qg), nh * hd, ptr(kg), ptr(vg), P, ML, ptr(slot_t),
         ptr(kvl), ptr(qb32), qb32.shape[0], ptr(out32), nh * hd, nh, nkv, hd, hd ** -0.5,
         stream())
    outs = torch.full_like(out, float("nan"))
    call("omni_prefill_attention_split", ptr(qg), nh * hd, ptr(kg), ptr(vg), P, ML, ptr(slot_t),
         ptr(kvl), ptr(qb), qb.shape[0], ptr(outs), nh * hd, nh, nkv, hd, hd ** -0.5, stream())
    outh = torch.full_like(out, float("nan"))
    call("omni_prefill_attention_gqa_halves", ptr(qg), nh * hd, ptr(kg), ptr(vg), P, ML,
         ptr(slot_t), ptr(kvl), ptr(qb32), qb32.shape[0], ptr(outh), nh * hd, nh, nkv, hd,
         hd ** -0.5, stream())
    torch.cuda.synchronize()
    e = ref.prefill_attention(q.float().view(T, nh, hd), k.float(), v.float(), segs, hd ** -0.5)
    d = (out.cpu().float() - e).abs().max().item()
    assert d <= 4e-3, d
    assert torch.equal(out.cpu(), out32.cpu())
    # key tiles split over four waves: P rounded to fp16 against each wave's own maximum
    ds = (outs.cpu().float() - e).abs().max().item()
    assert ds <= 4e-3, ds
    # key tiles split between two wave groups: the same, plus the second group's normalised
    # output rounded to fp16 before the merge
    dh = (outh.cpu().float() - e).abs().max().item()
    assert dh <= 4e-3, dh


@pytest.mark.parametrize("ctx,chunk", [((40, 300), (16, 7)), ((2048,), (256,)),
                                       ((97, 1023, 5), (33, 16, 5))])
def test_prefill_attention_append(gpu, ctx, chunk):
    """The append form (a chunk of chunk[s] new tokens at the end of a context of ctx[s]
    keys: token i of the chunk sees keys [0, ctx - chunk + i + 1)) for every prefill kernel
    (16-token blocks for the per-head ones, 32 for the shared-tile ones), against the
    oracle's per-token attention over the same pool rows."""
    from omniserver_amd.attention import QBLOCK_GQA, query_blocks
    from omniserver_amd._lib import call, ptr, stream
    say(f"prefill_attention append ctx={ctx} chunk={chunk}")
    nh, nkv, hd, ML = 12, 2, 128, 2048
    P = len(ctx)
    T = sum(chunk)
    kp = f16((P, ML, nkv, hd), 64)
    vp = f16((P, ML, nkv, hd), 65)
    q = f16((T, nh * hd), 66)
    slot, kvl = [], []
    for s, (Lk, Lq) in enumerate(zip(ctx, chunk)):
        slot += [s] * Lq
        kvl += [Lk - Lq + i + 1 for i in range(Lq)]
    qb16 = query_blocks(chunk, gpu)
    slot_t = torch.tensor(slot, dtype=torch.int64, device=gpu)
    kvl_t = torch.tensor(kvl, dtype=torch.int64, device=gpu)
    qg, kg, vg = q.to(gpu), kp.to(gpu), vp.to(gpu)
    e = ref.decode_attention(q.float().view(T, nh, hd), kp.float(), vp.float(),
                             torch.tensor(slot), torch.tensor(kvl), hd ** -0.5)
    qb32 = query_blocks(chunk, gpu, QBLOCK_GQA)
    for fn in ("omni_prefill_attention", "omni_prefill_attention_split",
               "omni_prefill_attention_gqa", "omni_prefill_attention_gqa_halves"):
        qb = qb32 if "gqa" in fn else qb16
        out = torch.full((T, nh, hd), float("nan"), device=gpu, dtype=torch.float16)
        call(fn, ptr(qg), nh * hd, ptr(kg), ptr(vg), P, ML, ptr(slot_t), ptr(kvl_t), ptr(qb),
             qb.shape[0], ptr(out), nh * hd, nh, nkv, hd, hd ** -0.5, stream())
        torch.cuda.synchronize()
        d = (out.cpu().float() - e).abs().max().item()
        assert d <= 4e-3, (fn, d)


# ----------------------------------------------------------------------------- linears
def _gptq(K, N, seed):
    from omniserver_amd.synth import gptq_random
    return gptq_random(K, N, seed, "t")


@pytest.mark.parametrize("K,N", [(1536, 2048), (8960, 1536), (1536, 256)])
def test_w4_dequant_bit_exact(gpu, K, N):
    from omniserver_amd.linear import GPTQLinear
    say(f"int4 dequant K={K} N={N}")
    qw, sc = _gptq(K, N, 71)
    lin = GPTQLinear(qw.to(gpu), sc.to(gpu))
    w = lin.dequantized().cpu().float()
    e = ref.gptq_dequant(qw, sc)
    assert torch.equal(w, e)


@pytest.mark.parametrize("M", [1, 16, 32, 48, 64])
@pytest.mark.parametrize("K,N,bias,silu", [
    (1536, 2048, True, False), (1536, 1536, False, False), (8960, 1536, False, False),
    (1536, 17920, False, True),
])
def test_w4a16_gemm(gpu, M, K, N, bias, silu):
    from omniserver_amd.linear import GPTQLinear
    say(f"w4a16 M={M} K={K} N={N} bias={bias} silu={silu}")
    qw, sc = _gptq(K, N, 72 + K + N)
    b = f16((N,), 73, 0.02) if bias else None
    x = f16((M, K), 74)
    lin = GPTQLinear(qw.to(gpu), sc.to(gpu), None if b is None else b.to(gpu), fuse_silu=silu)
    W = ref.gptq_dequant(qw, sc)
    if silu:
        e = ref.silu_mul(ref.linear(x.float(), W))
    else:
        e = ref.linear(x.float(), W, None if b is None else b.float(), bias_after_round=True)
    tol = 2e-3 * max(1.0, e.abs().max().item())
    xg = x.to(gpu)
    presets = [None, 1, 4, 6, 7, 9] if silu else [0, 1, 2, 3]
    outs = {}
    for pr in presets:
        out = torch.empty(M, lin.out_features, device=gpu, dtype=torch.float16)
        lin.forward_out(xg, out, preset=pr)
        outs[pr] = out.cpu()
        d = (out.cpu().float() - e).abs().max().item()
        assert d <= tol, (pr, d, tol)
    if silu:
        # x staged before (6, 7, 9) or after (4, 3, 1) the weights are requested: same sums
        assert torch.equal(outs[4], outs[6]) and torch.equal(outs[1], outs[9])
    if not silu:
        # split-K partial sums (fp32, no bias): their slice-ordered sum is the GEMM
        e32 = x.float() @ W
        for ks in (2, 5):
            for pr in (0, 1):
                part = torch.empty(ks * M * N, device=gpu, dtype=torch.float32)
                S = lin.forward_partial(xg, part, ks, pr)
                got = part[:S * M * N].view(S, M, N).sum(0).cpu()
                d = (got - e32).abs().max().item()
                assert d <= 1e-3 * max(1.0, e32.abs().max().item()), (ks, pr, d)


@pytest.mark.parametrize("fmt", ["int4", "fp16"])
@pytest.mark.parametrize("M", [65, 300])
@pytest.mark.parametrize("K,N,bias,silu", [
    (1536, 2048, True, False), (8960, 1536, False, False), (1536, 17920, False, True),
    # N % 128 != 0: the tiled kernel instead of the pipelined one
    (256, 48, True, False), (1536, 2064, True, False), (1536, 17952, False, True),
])
def test_tiled_gemm(gpu, fmt, M, K, N, bias, silu):
    """Prefill-size linears (M > 64) run an MFMA GEMM (the pipelined one for N % 128 == 0,
    else the tiled one): within tolerance of the oracle, and bit-equal to the skinny kernel
    run over 64-row blocks with one wave per K range (the same k order: groups ascending,
    32-k steps ascending)."""
    from omniserver_amd.linear import F16Linear, GPTQLinear
    say(f"tiled gemm fmt={fmt} M={M} K={K} N={N} bias={bias} silu={silu}")
    b = f16((N,), 91, 0.02) if bias else None
    x = f16((M, K), 92)
    if fmt == "int4":
        qw, sc = _gptq(K, N, 93 + K + N)
        W = ref.gptq_dequant(qw, sc)
        lin = GPTQLinear(qw.to(gpu), sc.to(gpu), None if b is None else b.to(gpu), fuse_silu=silu)
    else:
        wt = f16((N, K), 94, 0.02)
        W = wt.float().t()
        lin = F16Linear(wt.to(gpu), None if b is None else b.to(gpu), fuse_silu=silu)
    if silu:
        e = ref.silu_mul(ref.linear(x.float(), W))
    else:
        e = ref.linear(x.float(), W, None if b is None else b.float(),
                       bias_after_round=fmt == "int4")
    xg = x.to(gpu)
    out = torch.empty(M, lin.out_features, device=gpu, dtype=torch.float16)
    lin.forward_out(xg, out, ksplit=1)
    torch.cuda.synchronize()
    d = (out.cpu().float() - e).abs().max().item()
    assert d <= 2e-3 * max(1.0, e.abs().max().item()), d
    blocks = torch.empty_like(out)
    for s0 in range(0, M, 64):
        s1 = min(M, s0 + 64)
        lin.forward_out(xg[s0:s1], blocks[s0:s1], preset=1)
    assert torch.equal(out.cpu(), blocks.cpu())
    # split along K (the default for few tiles; 2 slices forced): the slices' fp32 sums add in
    # another order, so an fp16 result may sit one step from the unsplit one
    # (and the bias, added after that rounding for int4, can leave a result far smaller
    # than the sum it was rounded at)
    # (and where the sum nearly cancels, the fp32 accumulation error of the summed term
    # magnitudes dominates)
    if not silu and K >= 1024:
        e_nb = ref.linear(x.float(), W).abs()
        absprod = x.float().abs() @ W.abs()
        for ks in (None, 2):
            sp = torch.empty_like(out)
            lin.forward_out(xg, sp, ksplit=ks)
            torch.cuda.synchronize()
            ds = (sp.cpu().float() - out.cpu().float()).abs()
            mag = torch.maximum(torch.maximum(out.cpu().float().abs(), sp.cpu().float().abs()), e_nb)
            assert (ds <= mag * 2.0 ** -9 + absprod * 2.0 ** -20).all(), ds.max().item()
            assert (sp.cpu().float() - e).abs().max().item() <= 2e-3 * max(1.0, e.abs().max().item())


def _packed_plan(M, N, K, fmt, epi, has_bias=0):
    import ctypes
    from omniserver_amd._lib import lib
    r, c, k = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
    assert lib().omni_packed_gemm_pipe_plan(M, N, K, fmt, epi, has_bias, 0, 0, ctypes.byref(r),
                                            ctypes.byref(c), ctypes.byref(k)) == 0
    return r.value, c.value, k.value


@pytest.mark.parametrize("M,K,N", [(256, 1536, 17920), (200, 1536, 17920), (129, 512, 1280)])
def test_packed_gemm_pipe_silu160(gpu, M, K, N):
    """The SiLU-fused gate_up at 129-256 rows on 128 x 160 tiles (five gate|up pairs, one
    tile per workgroup: config 1's 256-token gate_up), equal bit for bit to the forced
    256 x 128 tiles (same K order per output), a ragged last row tile included, and sampled
    rows within tolerance of the oracle."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd.linear import F16Linear
    assert _packed_plan(M, N, K, 1, 1) == (128, 160, 1)
    say(f"packed gemm pipe silu160 M={M} K={K} N={N}")
    wt = f16((N, K), 121, 0.02)
    x = f16((M, K), 122)
    lin = F16Linear(wt.to(gpu), fuse_silu=True)
    xg = x.to(gpu)

    def run(tile_rows):
        out = torch.full((M, N // 2), float("nan"), device=gpu, dtype=torch.float16)
        call("omni_packed_gemm_pipe", ptr(xg), K, ptr(lin.weight_packed), None, 1, None, 0,
             ptr(out), N // 2, M, N, K, 1, tile_rows, 1, None, stream())
        torch.cuda.synchronize()
        return out.cpu()

    narrow, wide = run(0), run(256)
    assert not torch.isnan(narrow).any()
    assert torch.equal(narrow, wide)
    rows = torch.tensor(sorted({0, 31, 32, 77, 127, 128, M - 1}))
    e = ref.silu_mul(ref.linear(x[rows].float(), wt.float().t()))
    tol = 2e-3 * max(1.0, e.abs().max().item())
    assert (narrow[rows].float() - e).abs().max().item() <= tol


@pytest.mark.parametrize("M,K,bias", [(4096, 1536, True), (4000, 8960, False)])
def test_packed_gemm_pipe_wide_tiles(gpu, M, K, bias):
    """The 128 x 192 tiles omni_packed_gemm_pipe picks for config 5's N = 1536 projections
    (fp16 weights, one K slice; a ragged M puts a partial row tile in the round): STORE
    and PARTIAL results equal the 256 x 128 tiles' bit for bit (same k order per output),
    and 64 sampled rows (every row tile) are within tolerance of the oracle."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd.linear import F16Linear
    N = 1536
    rows, cols, ks = _packed_plan(M, N, K, 1, 0, int(bias))
    say(f"packed gemm pipe wide tiles M={M} K={K} N={N} bias={bias}: {rows} x {cols}, {ks} slice")
    assert (rows, cols, ks) == (128, 192, 1)
    assert _packed_plan(M, N, K, 1, 2)[1] == 192
    wt = f16((N, K), 99, 0.02)
    b = f16((N,), 100, 0.02) if bias else None
    x = f16((M, K), 101)
    lin = F16Linear(wt.to(gpu), None if b is None else b.to(gpu))
    xg = x.to(gpu)

    def run(tile_rows, epi):
        out = torch.full((M, N), float("nan"), device=gpu, dtype=torch.float16)
        ws = torch.full((M * N,), float("nan"), device=gpu, dtype=torch.float32)
        call("omni_packed_gemm_pipe", ptr(xg), K, ptr(lin.weight_packed), None, 1,
             ptr(lin.bias) if epi == 0 else None, 0, ptr(out) if epi == 0 else None, N, M, N, K,
             epi, tile_rows, 1, ptr(ws) if epi == 2 else None, stream())
        torch.cuda.synchronize()
        return out.cpu() if epi == 0 else ws.cpu()

    wide, o256 = run(0, 0), run(256, 0)
    assert torch.equal(wide, o256)
    assert torch.equal(run(0, 2), run(256, 2))
    rows_s = torch.tensor(sorted({64 * i + (37 * i) % 64 for i in range(M // 64)} | {M - 1}))
    e = ref.linear(x[rows_s].float(), wt.float().t(), None if b is None else b.float())
    tol = 2e-3 * max(1.0, e.abs().max().item())
    assert (wide[rows_s].float() - e).abs().max().item() <= tol


@pytest.mark.parametrize("M,K,N,silu", [(4096, 1536, 17920, True), (4096, 1536, 17920, False),
                                        (8192, 1536, 2048, False)])
def test_packed_gemm_pipe_big_tiles(gpu, M, K, N, silu):
    """The persistent 256 x 256 tiles omni_packed_gemm_pipe picks for config 5's gate_up (SiLU)
    at M = 4096 (and an unbiased STORE at that shape): 1024 whole tiles over the first 16384
    columns, the last 1536 in 256 x 128 half tiles; and an unbiased STORE at M = 8192 (whole
    tiles only): equal to the 256 x 128 tiles' results bit for bit (same k order per output),
    and 64 sampled rows (every row tile) within tolerance of the oracle."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd.linear import F16Linear
    rows, cols, ks = _packed_plan(M, N, K, 1, 1 if silu else 0)
    say(f"packed gemm pipe big tiles M={M} K={K} N={N} silu={silu}: {rows} x {cols}, {ks} slice")
    assert (rows, cols, ks) == (256, 256, 1)
    assert _packed_plan(M, N, K, 1, 0, 1)[1] != 256          # a bias keeps the pipelined tiles
    wt = f16((N, K), 102, 0.02)
    x = f16((M, K), 103)
    lin = F16Linear(wt.to(gpu), fuse_silu=silu)
    xg = x.to(gpu)
    nout = N // 2 if silu else N

    def run(tile_rows):
        out = torch.full((M, nout), float("nan"), device=gpu, dtype=torch.float16)
        call("omni_packed_gemm_pipe", ptr(xg), K, ptr(lin.weight_packed), None, 1, None, 0,
             ptr(out), nout, M, N, K, 1 if silu else 0, tile_rows, 1, None, stream())
        torch.cuda.synchronize()
        return out.cpu()

    big, o256 = run(0), run(256)
    assert torch.equal(big, o256)
    rows_s = torch.tensor(sorted({64 * i + (37 * i) % 64 for i in range(M // 64)} | {M - 1}))
    rows_s = rows_s[:: max(1, len(rows_s) // 64)]
    W = wt.float().t()
    e = ref.linear(x[rows_s].float(), W)
    if silu:
        e = ref.silu_mul(e)
    tol = 2e-3 * max(1.0, e.abs().max().item())
    assert (big[rows_s].float() - e).abs().max().item() <= tol


@pytest.mark.parametrize("M,K,N,form", [(4096, 8960, 1536, (256, 192, 2)),
                                         (4096, 8960, 2048, (256, 256, 2))])
def test_packed_gemm_pipe_big_partial(gpu, M, K, N, form):
    """fp32 partial output with the K slices left to the plan (ksplit 0): the persistent
    256-row tiles in two slices (config 5's down projection at M = 4096 on 256 x 192 tiles; a
    2048-wide projection on 256 x 256).  Slice s holds the products over its whole 128-groups
    [s G / S, (s + 1) G / S) of G = K / 128: each slice within fp32 tolerance of the oracle's
    sums over that K range on sampled rows (every row tile), and fp16 of the slices' sum
    within one fp16 step of the finished STORE output."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd.linear import F16Linear
    plan = _packed_plan(M, N, K, 1, 2)
    say(f"packed gemm pipe big partial M={M} K={K} N={N}: plan {plan}")
    assert plan == form
    S = plan[2]
    wt = f16((N, K), 112, 0.02)
    x = f16((M, K), 113)
    lin = F16Linear(wt.to(gpu))
    xg = x.to(gpu)
    assert lin.partial_plan(M) == S
    part = torch.full((S * M * N,), float("nan"), device=gpu, dtype=torch.float32)
    assert lin.forward_partial_planned(xg, part) == S
    out = torch.full((M, N), float("nan"), device=gpu, dtype=torch.float16)
    call("omni_packed_gemm_pipe", ptr(xg), K, ptr(lin.weight_packed), None, 1, None, 0,
         ptr(out), N, M, N, K, 0, 0, 0, None, stream())
    torch.cuda.synchronize()
    P = part.view(S, M, N).cpu()
    assert not torch.isnan(P).any()
    rows_s = torch.tensor(sorted({64 * i + (29 * i) % 64 for i in range(M // 64)} | {M - 1}))
    rows_s = rows_s[:: max(1, len(rows_s) // 64)]
    G = K // 128
    for s_ in range(S):
        k0, k1 = 128 * (s_ * G // S), 128 * ((s_ + 1) * G // S)
        e = x[rows_s, k0:k1].float() @ wt[:, k0:k1].float().t()
        d = (P[s_][rows_s] - e).abs().max().item()
        tol = 5e-4 * max(1.0, e.abs().max().item())
        say(f"  slice {s_}: k [{k0}, {k1}) max|d| {d:.2e} (tol {tol:.1e})")
        assert d <= tol
    tot, mag = P[0].clone(), P[0].abs()
    for s_ in range(1, S):
        tot += P[s_]
        mag += P[s_].abs()
    o = out.cpu().float()
    # one fp16 step of the output, plus the fp32 rounding of the slices' sums, which shows
    # where slices of opposite sign nearly cancel (e.g. -0.4315 + 0.4319), and of the running
    # sums over K (the finished output itself is 1.5e-6 from the oracle's at such a point)
    ulp = torch.clamp(o.abs(), min=6.1e-5) * 2.0 ** -10
    assert ((tot.half().float() - o).abs() <= ulp * 1.01 + 1e-5 * mag + 5e-6).all()


@pytest.mark.parametrize("fmt", ["int4", "fp16"])
@pytest.mark.parametrize("M", [65, 300, 1000])
@pytest.mark.parametrize("K,N,bias,silu", [
    (1536, 2048, True, False), (8960, 1536, True, False), (1536, 17920, False, True),
    (384, 256, False, False),
])
def test_packed_gemm_pipe(gpu, fmt, M, K, N, bias, silu):
    """omni_packed_gemm_pipe through the C ABI at both tile heights and several K splits:
    unsplit results equal at 128 and 256 rows (the same k order per output) and equal to
    the skinny kernel over 64-row blocks; every form within tolerance of the oracle; split
    results within a rounding step of the unsplit ones."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd.linear import F16Linear, GPTQLinear
    say(f"packed gemm pipe fmt={fmt} M={M} K={K} N={N} bias={bias} silu={silu}")
    b = f16((N,), 95, 0.02) if bias else None
    x = f16((M, K), 96)
    if fmt == "int4":
        qw, sc = _gptq(K, N, 97 + K + N)
        W = ref.gptq_dequant(qw, sc)
        lin = GPTQLinear(qw.to(gpu), sc.to(gpu), None if b is None else b.to(gpu), fuse_silu=silu)
        wp, sp, code = lin.qweight_packed, lin.scales_packed, 0
    else:
        wt = f16((N, K), 98, 0.02)
        W = wt.float().t()
        lin = F16Linear(wt.to(gpu), None if b is None else b.to(gpu), fuse_silu=silu)
        wp, sp, code = lin.weight_packed, None, 1
    if silu:
        e = ref.silu_mul(ref.linear(x.float(), W))
    else:
        e = ref.linear(x.float(), W, None if b is None else b.float(),
                       bias_after_round=fmt == "int4")
    tol = 2e-3 * max(1.0, e.abs().max().item())
    xg = x.to(gpu)
    bg = lin.bias
    epi = 1 if silu else 0
    nout = lin.out_features

    def run(tile_rows, ksplit):
        out = torch.full((M, nout), float("nan"), device=gpu, dtype=torch.float16)
        ws = torch.empty(max(4, ksplit) * M * N, device=gpu, dtype=torch.float32)  # ksplit 0: <= 4
        call("omni_packed_gemm_pipe", ptr(xg), K, ptr(wp), ptr(sp), code, ptr(bg),
             int(fmt == "int4"), ptr(out), nout, M, N, K, epi, tile_rows, ksplit,
             ptr(ws) if ksplit != 1 else None, stream())
        torch.cuda.synchronize()
        return out.cpu()

    o128, o256 = run(128, 1), run(256, 1)
    assert torch.equal(o128, o256)
    assert (o128.float() - e).abs().max().item() <= tol
    blocks = torch.empty(M, nout, device=gpu, dtype=torch.float16)
    for s0 in range(0, M, 64):
        s1 = min(M, s0 + 64)
        lin.forward_out(xg[s0:s1], blocks[s0:s1], preset=1)
    assert torch.equal(o128, blocks.cpu())
    if silu:
        return
    e_nb = ref.linear(x.float(), W).abs()
    absprod = x.float().abs() @ W.abs()
    KG = K // 128
    for tr, ks in ((128, 0), (128, 2), (256, KG // 3), (256, 0)):
        if ks > 1 and 2 * (KG // ks) < (6 if fmt == "int4" and tr == 128 else 4):
            continue
        sp_out = run(tr, ks)
        ds = (sp_out.float() - o128.float()).abs()
        mag = torch.maximum(torch.maximum(o128.float().abs(), sp_out.float().abs()), e_nb)
        assert (ds <= mag * 2.0 ** -9 + absprod * 2.0 ** -20).all(), (tr, ks, ds.max().item())
        assert (sp_out.float() - e).abs().max().item() <= tol, (tr, ks)


@pytest.mark.parametrize("K,N,bias,silu", [
    (1536, 2048, True, False), (8960, 1536, False, False), (1536, 17920, False, True),
])
def test_gptq_prefill_unpacked(gpu, K, N, bias, silu):
    """From GPTQLinear.UNPACK_ROWS rows the int4 weights are unpacked to packed fp16 and the
    fp16 pipeline runs: omni_w4_unpack_f16 equals omni_f16_pack of the dequantised weight,
    the output equals the int4 pipeline's at the same K split (same fp16 weights, same k
    order), and it is within tolerance of the oracle."""
    from omniserver_amd._lib import call, lib, ptr, stream
    from omniserver_amd.linear import GPTQLinear
    M = GPTQLinear.UNPACK_ROWS + 37
    say(f"gptq prefill unpacked M={M} K={K} N={N} bias={bias} silu={silu}")
    qw, sc = _gptq(K, N, 111 + K + N)
    b = f16((N,), 112, 0.02) if bias else None
    x = f16((M, K), 113)
    lin = GPTQLinear(qw.to(gpu), sc.to(gpu), None if b is None else b.to(gpu), fuse_silu=silu)
    unp = torch.empty(N * K, device=gpu, dtype=torch.float16)
    call("omni_w4_unpack_f16", ptr(lin.qweight_packed), ptr(lin.scales_packed), ptr(unp), K, N,
         stream())
    ref_pack = torch.empty(N * K, device=gpu, dtype=torch.float16)
    call("omni_f16_pack", ptr(lin.dequantized().t().contiguous()), ptr(ref_pack), K, N, 0, stream())
    torch.cuda.synchronize()
    assert torch.equal(unp.cpu(), ref_pack.cpu())
    xg = x.to(gpu)
    out = torch.empty(M, lin.out_features, device=gpu, dtype=torch.float16)
    lin.forward_out(xg, out)
    ks = 1 if silu else lib().omni_f16_gemm_pipe_splits(M, N, K, 0)
    direct = torch.empty_like(out)
    ws = torch.empty(ks * M * N, device=gpu, dtype=torch.float32)
    call("omni_packed_gemm_pipe", ptr(xg), K, ptr(lin.qweight_packed), ptr(lin.scales_packed), 0,
         ptr(lin.bias), 1, ptr(direct), lin.out_features, M, N, K, 1 if silu else 0, 0, ks,
         ptr(ws) if ks > 1 else None, stream())
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), direct.cpu())
    W = ref.gptq_dequant(qw, sc)
    if silu:
        e = ref.silu_mul(ref.linear(x.float(), W))
    else:
        e = ref.linear(x.float(), W, None if b is None else b.float(), bias_after_round=True)
    assert (out.cpu().float() - e).abs().max().item() <= 2e-3 * max(1.0, e.abs().max().item())


@pytest.mark.parametrize("K,N,bias,silu", [(1536, 2048, True, False), (1536, 17920, False, True)])
def test_gptq_prefill_resident_f16(gpu, K, N, bias, silu):
    """From GPTQLinear.F16_ROWS rows a GPTQ linear runs on the fp16 expansion of its int4
    weights, made at the first such call and kept: two calls (the second with fewer rows)
    use one buffer and equal the int4 pipeline's outputs bit for bit (same fp16 values, same
    k order), the partial-sum form equals the int4 partial form, and with keep_f16 off no
    copy is made and the int4 pipeline runs."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd.linear import EPI_PARTIAL, GPTQLinear
    qw, sc = _gptq(K, N, 211 + K + N)
    b = f16((N,), 212, 0.02) if bias else None
    lin = GPTQLinear(qw.to(gpu), sc.to(gpu), None if b is None else b.to(gpu), fuse_silu=silu)

    def int4_direct(xg, ks):
        o = torch.empty(xg.shape[0], lin.out_features, device=gpu, dtype=torch.float16)
        ws = torch.empty(max(1, ks) * xg.shape[0] * N, device=gpu, dtype=torch.float32)
        call("omni_packed_gemm_pipe", ptr(xg), K, ptr(lin.qweight_packed), ptr(lin.scales_packed), 0,
             ptr(lin.bias), 1, ptr(o), lin.out_features, xg.shape[0], N, K, 1 if silu else 0, 0, ks,
             ptr(ws) if ks > 1 else None, stream())
        return o

    from omniserver_amd._lib import lib
    bufs = []
    for M in (GPTQLinear.F16_ROWS + 300, GPTQLinear.F16_ROWS + 7):
        say(f"gptq resident fp16 M={M} K={K} N={N} bias={bias} silu={silu}")
        xg = f16((M, K), 213 + M).to(gpu)
        out = torch.empty(M, lin.out_features, device=gpu, dtype=torch.float16)
        lin.forward_out(xg, out)
        bufs.append(lin._w16.data_ptr())
        ks = 1 if silu else lib().omni_f16_gemm_pipe_splits(M, N, K, 0)
        direct = int4_direct(xg, ks)
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), direct.cpu()), M
    assert bufs[0] == bufs[1]
    if not silu:
        M = GPTQLinear.F16_ROWS + 44
        xg = f16((M, K), 214).to(gpu)
        p16 = torch.empty(8 * M * N, device=gpu, dtype=torch.float32)
        S = lin.forward_partial(xg, p16, ksplit=4)
        p4 = torch.empty_like(p16)
        call("omni_packed_gemm_pipe", ptr(xg), K, ptr(lin.qweight_packed), ptr(lin.scales_packed), 0,
             None, 0, None, 0, M, N, K, EPI_PARTIAL, 0, S, ptr(p4), stream())
        torch.cuda.synchronize()
        assert torch.equal(p16[:S * M * N].cpu(), p4[:S * M * N].cpu())
    lin.release_f16()
    lin.keep_f16 = False
    xg = f16((GPTQLinear.F16_ROWS + 5, K), 215).to(gpu)
    out = torch.empty(xg.shape[0], lin.out_features, device=gpu, dtype=torch.float16)
    lin.forward_out(xg, out)
    assert lin._w16 is None


@pytest.mark.parametrize("M", [1, 16, 32])
@pytest.mark.parametrize("K,N,bias,silu", [
    (1536, 2048, True, False), (8960, 1536, False, False), (1536, 17920, False, True),
])
def test_f16_gemm(gpu, M, K, N, bias, silu):
    from omniserver_amd.linear import F16Linear
    say(f"f16 gemm M={M} K={K} N={N} bias={bias} silu={silu}")
    w = f16((N, K), 81, 0.02)
    b = f16((N,), 82, 0.02) if bias else None
    x = f16((M, K), 83)
    lin = F16Linear(w.to(gpu), None if b is None else b.to(gpu), fuse_silu=silu)
    y = lin(x.to(gpu)).cpu().float()
    if silu:
        e = ref.silu_mul(ref.linear(x.float(), w.float().t()))
    else:
        e = ref.linear(x.float(), w.float().t(), None if b is None else b.float())
    d = (y - e).abs()
    tol = 2e-3 * max(1.0, e.abs().max().item())
    assert d.max().item() <= tol, (d.max().item(), tol)


@pytest.mark.parametrize("S,M,H", [(7, 32, 1536), (20, 5, 1536), (11, 3, 4096), (2, 1000, 1536),
                                   (3, 300, 4096)])
def test_add_rmsnorm_partials(gpu, S, M, H):
    """x = fp16(sum of split-K partials in slice order), then add + RMSNorm (H = 4096 runs
    the 1024-thread form, 20 slices two batches of the 256-thread one; past 256 rows the
    many-row kernel, bit-equal to omni_add_rmsnorm on the slice-ordered fp16 sum)."""
    from omniserver_amd import fused_ops as F
    say(f"add_rmsnorm over split-K partials S={S} M={M} H={H}")
    g = torch.Generator().manual_seed(101)
    parts = torch.randn(S, M, H, generator=g) * 0.3
    r = f16((M, H), 102)
    w = torch.ones(H, dtype=torch.float16)
    pg, rg, wg = parts.to(gpu), r.to(gpu), w.to(gpu)
    y = torch.empty(M, H, device=gpu, dtype=torch.float16)
    nr = torch.empty_like(y)
    F.add_rms_norm_partials_out(pg, S, rg, wg, 1e-6, y, nr)
    torch.cuda.synchronize()
    x16 = ref.r16(parts.sum(0))
    ey, er = ref.add_rms_norm(x16, r.float(), w.float(), 1e-6)
    # the slice-ordered fp32 sum can differ from torch's sum order by an ulp before the
    # fp16 rounding: residuals agree to one fp16 ulp
    assert (nr.cpu().float() - er).abs().max().item() <= 2e-3 * er.abs().max().item()
    assert (y.cpu().float() - ey).abs().max().item() <= 2e-3 * ey.abs().max().item()
    if M > 256:
        xs = pg[0].clone()
        for p in range(1, S):
            xs = xs + pg[p]
        y2, r2 = torch.empty_like(y), torch.empty_like(y)
        F.add_rms_norm_out(xs.half(), rg, wg, 1e-6, y2, r2)
        torch.cuda.synchronize()
        assert torch.equal(y.cpu(), y2.cpu()) and torch.equal(nr.cpu(), r2.cpu())


@pytest.mark.parametrize("H,M", [(1536, 1001), (3584, 300)])
def test_addnorm_rows_equals_generic(gpu, H, M):
    """Past 256 rows at H = 1536 / 3584 the add+RMSNorm runs the load-batched many-row kernel
    (x fp16, or 1-4 / 1-2 partial slices); any other slice count runs the generic many-row
    kernel.  Padding the slices with zero slices up to 5 (x + 0 = x in fp32) sends the same
    sums through the generic kernel: outputs and residuals equal bit for bit, with the
    residual updated in place as the prefill does; a ragged last workgroup (M % 4 != 0)."""
    from omniserver_amd import fused_ops as F
    g = torch.Generator().manual_seed(111 + H)
    gain = (1.0 + 0.1 * f16((H,), 112)).to(gpu)
    res = f16((M, H), 113).to(gpu)
    x = f16((M, H), 114).to(gpu)
    nps = (0, 1, 2, 3, 4) if H == 1536 else (0, 1, 2)
    for S in nps:
        say(f"addnorm rows H={H} M={M} slices={S}")
        if S == 0:
            sl = [x.float()]
        else:
            sl = [(torch.randn(M, H, generator=g) * 0.3).to(gpu) for _ in range(S)]
        y = torch.empty(M, H, device=gpu, dtype=torch.float16)
        r_new = res.clone()
        if S == 0:
            F.add_rms_norm_out(x, r_new, gain, 1e-6, y, r_new)
        else:
            F.add_rms_norm_partials_out(torch.stack(sl), S, r_new, gain, 1e-6, y, r_new)
        pad = torch.stack(sl + [torch.zeros(M, H, device=gpu)] * (5 - len(sl)))
        y5, r5 = torch.empty_like(y), torch.empty_like(y)
        F.add_rms_norm_partials_out(pad, 5, res, gain, 1e-6, y5, r5)
        torch.cuda.synchronize()
        assert torch.equal(r_new.cpu(), r5.cpu()) and torch.equal(y.cpu(), y5.cpu())


@pytest.mark.parametrize("fmt", ["int4", "fp16"])
@pytest.mark.parametrize("M", [1, 2])
def test_gemm_addnorm(gpu, fmt, M):
    """qkv / gate_up with the add+RMSNorm in their input staging (omni_*_gemm_addnorm) equal
    add+RMSNorm over the partials followed by the linear, bit for bit: the new residual, the
    qkv split-K partial sums and the gate_up SiLU output; residual_out must not alias the
    residual, and rows past what the workgroup holds are refused."""
    from omniserver_amd import fused_ops as F
    from omniserver_amd.linear import F16Linear, GPTQLinear
    H = 1536
    g = torch.Generator().manual_seed(301 + M)
    for nparts, (N, silu) in ((14, (2048, False)), (12, (17920, True))):
        say(f"gemm_addnorm fmt={fmt} M={M} nparts={nparts} N={N} silu={silu}")
        parts = (torch.randn(nparts, M, H, generator=g) * 0.3).to(gpu)
        res = f16((M, H), 302 + nparts).to(gpu)
        gain = (1.0 + 0.1 * f16((H,), 303)).to(gpu)
        if fmt == "int4":
            qw, sc = _gptq(H, N, 304 + N)
            lin = GPTQLinear(qw.to(gpu), sc.to(gpu), f16((N,), 305, 0.02).to(gpu) if not silu else None,
                             fuse_silu=silu)
        else:
            lin = F16Linear(f16((N, H), 306, 0.02).to(gpu), f16((N,), 305, 0.02).to(gpu) if not silu else None,
                            fuse_silu=silu)
        # reference: the norm launch, then the linear
        y = torch.empty(M, H, device=gpu, dtype=torch.float16)
        r1 = torch.empty_like(y)
        F.add_rms_norm_partials_out(parts, nparts, res, gain, 1e-6, y, r1)
        r2 = torch.full_like(y, float("nan"))
        if silu:
            o1 = torch.empty(M, N // 2, device=gpu, dtype=torch.float16)
            lin.forward_out(y, o1)
            o2 = torch.full_like(o1, float("nan"))
            lin.forward_addnorm(parts, nparts, res, gain, 1e-6, r2, out=o2)
        else:
            S = lin.partial_slices()
            o1 = torch.empty(S * M * N, device=gpu, dtype=torch.float32)
            S1 = lin.forward_partial(y, o1)
            o2 = torch.full_like(o1, float("nan"))
            S2 = lin.forward_addnorm(parts, nparts, res, gain, 1e-6, r2, partial=o2)
            assert S1 == S2 == S
        torch.cuda.synchronize()
        assert torch.equal(r1.cpu(), r2.cpu())
        assert torch.equal(o1.cpu(), o2.cpu())
        with pytest.raises(ValueError):
            lin.forward_addnorm(parts, nparts, res, gain, 1e-6, res, out=o2, partial=o2)
    if fmt == "int4":
        big = 3 * 512 // (H // 8) + 1          # more rows than the 512-thread form holds
        p3 = torch.zeros(14, big, H, device=gpu)
        r3 = torch.zeros(big, H, device=gpu, dtype=torch.float16)
        qw, sc = _gptq(H, 2048, 307)
        lin = GPTQLinear(qw.to(gpu), sc.to(gpu))
        with pytest.raises(RuntimeError):
            lin.forward_addnorm(p3, 14, r3, torch.ones(H, device=gpu, dtype=torch.float16), 1e-6,
                                torch.empty_like(r3),
                                partial=torch.empty(8 * big * 2048, device=gpu))


@pytest.mark.parametrize("M", [1, 32, 49, 64])
def test_lmhead_argmax(gpu, M):
    from omniserver_amd.linear import LMHeadArgmax
    say(f"lm_head argmax M={M}")
    V, H = 151936, 1536
    E = f16((V, H), 91, 0.02)
    h = f16((M, H), 92)
    lm = LMHeadArgmax(E.to(gpu))
    ids = torch.empty(M, device=gpu, dtype=torch.int64)
    logits = torch.empty(M, V, device=gpu, dtype=torch.float16)
    for rep in range(2):
        lm.argmax_out(h.to(gpu), ids, logits)
        torch.cuda.synchronize()
    e = ref.r16(h.float() @ E.float().t())
    lg = logits.cpu().float()
    d = (lg - e).abs().max().item()
    assert d <= 2e-2, d
    cos = torch.nn.functional.cosine_similarity(lg, e, dim=-1).min().item()
    assert cos >= 0.9999
    # the fused argmax is exactly torch.argmax of the kernel's own fp16 logits
    assert torch.equal(ids.cpu(), logits.cpu().float().argmax(-1))
    # and agrees with the oracle wherever the oracle's top-2 margin exceeds the tolerance
    margin = ref.top2_margin(e)
    ok = margin > 2 * d
    assert torch.equal(ids.cpu()[ok], e.argmax(-1)[ok])


def test_lmhead_argmax_ties(gpu):
    """Equal fp16 logits at several columns: the lowest index wins (torch.argmax)."""
    from omniserver_amd.linear import LMHeadArgmax
    say("lm_head argmax ties")
    V, H = 151936, 1536
    E = torch.zeros(V, H, dtype=torch.float16)
    for n in (70000, 3, 151935, 1000):
        E[n, 0] = 1.0
    h = torch.zeros(2, H, dtype=torch.float16)
    h[:, 0] = 1.0
    lm = LMHeadArgmax(E.to(gpu))
    ids = torch.empty(2, device=gpu, dtype=torch.int64)
    lm.argmax_out(h.to(gpu), ids)
    torch.cuda.synchronize()
    assert ids.cpu().tolist() == [3, 3]


@pytest.mark.parametrize("bias_after_round", [0, 1])
def test_mrope_from_partials(gpu, bias_after_round):
    """qkv rows formed from split-K partials (+ bias) then rotated: bit-equal to forming
    the fp16 rows on the host the same way and running the plain kernel."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd.qwen2_llm import rope_tables
    say(f"mrope from partials bias_after_round={bias_after_round}")
    cfg = ref.Qwen2Config()
    nh, nkv, hd = 12, 2, 128
    T, S, P, ML = 5, 7, 6, 64
    W = (nh + 2 * nkv) * hd
    g = torch.Generator().manual_seed(111)
    parts = torch.randn(S, T, W, generator=g) * 0.2
    bias = f16((W,), 112, 0.02)
    lengths = torch.randint(0, 40, (P,), generator=torch.Generator().manual_seed(113))
    acc = torch.zeros(T, W)
    for s_ in range(S):          # slice order, as the kernel adds them
        acc = acc + parts[s_]
    if bias_after_round:
        rows = (acc.half().float() + bias.float()).half()
    else:
        rows = (acc + bias.float()).half()
    cos, sin = rope_tables(cfg, 128, gpu)
    outs = []
    for mode in ("partials", "plain"):
        kc = torch.zeros(P, ML, nkv, hd, dtype=torch.float16, device=gpu)
        vc = torch.zeros_like(kc)
        lg = lengths.to(gpu)
        if mode == "partials":
            q = torch.zeros(T, W, dtype=torch.float16, device=gpu)
            pg, bg = parts.to(gpu), bias.to(gpu)
            call("omni_mrope_kv_write_partials", ptr(q), W, ptr(pg), S, ptr(bg), bias_after_round,
                 None, ptr(lg), None, ptr(cos), ptr(sin), 128, ptr(kc), ptr(vc), None, None, P,
                 ML, T, nh, nkv, hd, 16, 24, 24, stream())
        else:
            q = rows.to(gpu)
            call("omni_mrope_kv_write", ptr(q), W, None, ptr(lg), None, ptr(cos), ptr(sin), 128,
                 ptr(kc), ptr(vc), None, None, P, ML, T, nh, nkv, hd, 16, 24, 24, stream())
        torch.cuda.synchronize()
        outs.append((q.cpu(), kc.cpu(), vc.cpu()))
    # sums can differ from the host's in the last fp32 ulp -> allow 1 fp16 ulp
    for a, b in zip(outs[0], outs[1]):
        d = (a.float() - b.float()).abs()
        assert d.max().item() <= 2e-3 * max(1.0, b.float().abs().max().item())
        assert (d > 0).float().mean().item() < 0.01


@pytest.mark.parametrize("bias_after_round,splits,lengths", [
    (1, 3, [2047, 31, 0, 500]), (0, 1, [64, 7]), (1, 8, [4000, 1000]),
])
def test_decode_attention_fused_equals_unfused(gpu, bias_after_round, splits, lengths):
    """Fused prologue (qkv partials + bias + M-RoPE + KV write) + attention gives exactly
    what the separate M-RoPE-from-partials and attention launches give."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd.qwen2_llm import rope_tables
    say(f"fused decode attention bar={bias_after_round} splits={splits} lengths={lengths}")
    cfg = ref.Qwen2Config()
    nh, nkv, hd, ML = 12, 2, 128, 4096
    n = len(lengths)
    P = n + 1
    W = (nh + 2 * nkv) * hd
    S = 6
    g = torch.Generator().manual_seed(120)
    parts = (torch.randn(S, n, W, generator=g) * 0.3).to(gpu)
    bias = f16((W,), 121, 0.02).to(gpu)
    delta = torch.tensor([0, 3, -2, 1, 0][:P], dtype=torch.int64).to(gpu)
    kp0 = f16((P, ML, nkv, hd), 122)
    vp0 = f16((P, ML, nkv, hd), 123)
    lens = torch.tensor(lengths + [0], dtype=torch.int64).to(gpu)
    cos, sin = rope_tables(cfg, 8192, gpu)
    rows = torch.empty(n, hd, device=gpu, dtype=torch.float16)
    call("omni_rope_rows", None, ptr(lens), ptr(delta), ptr(cos), ptr(sin), 8192, P, n, ptr(rows),
         stream())
    outs = []
    for mode in ("fused", "fused-rows", "separate"):
        kc, vc = kp0.to(gpu), vp0.to(gpu)
        out = torch.empty(n, nh, hd, device=gpu, dtype=torch.float16)
        ws = torch.empty(n * nkv * splits * 6 * 132, device=gpu, dtype=torch.float32)
        if mode.startswith("fused"):
            call("omni_decode_attention_fused", ptr(parts), S, ptr(bias), bias_after_round,
                 ptr(cos), ptr(sin), 8192, ptr(delta), 16, 24, 24, ptr(kc), ptr(vc), P, ML, None,
                 ptr(lens), ptr(out), n, nh, nkv, hd, hd ** -0.5, 8, splits, ptr(ws), ws.numel(),
                 1, ptr(rows) if mode == "fused-rows" else None, stream())
        else:
            qkv = torch.empty(n, W, device=gpu, dtype=torch.float16)
            call("omni_mrope_kv_write_partials", ptr(qkv), W, ptr(parts), S, ptr(bias),
                 bias_after_round, None, ptr(lens), ptr(delta), ptr(cos), ptr(sin), 8192, ptr(kc),
                 ptr(vc), None, None, P, ML, n, nh, nkv, hd, 16, 24, 24, stream())
            call("omni_decode_attention", ptr(qkv), W, ptr(kc), ptr(vc), P, ML, None, ptr(lens),
                 1, 1, ptr(out), n, nh, nkv, hd, hd ** -0.5, 8, splits, ptr(ws), ws.numel(),
                 stream())
        torch.cuda.synchronize()
        outs.append((out.cpu(), kc.cpu(), vc.cpu()))
    for other in outs[1:]:
        for a, b in zip(outs[0], other):
            assert torch.equal(a, b)


@pytest.mark.parametrize("fmt,splits,n,ksplit", [
    ("int4", 4, 32, None), ("int4", 1, 32, None), ("fp16", 3, 32, None), ("int4", 11, 32, None),
    # 9-16 splits for few rows: the merge's two batches requested by two threads
    ("int4", 16, 1, 6), ("int4", 16, 2, 6), ("int4", 9, 8, None), ("fp16", 16, 8, None),
    ("int4", 13, 3, 12)])
def test_oproj_merges_attention_states(gpu, fmt, splits, n, ksplit):
    """o_proj reading the decode attention's split states (merge in its input staging)
    gives exactly merge launch + o_proj on the merged fp16 output."""
    from omniserver_amd._lib import call, ptr, stream
    from omniserver_amd.linear import F16Linear, GPTQLinear
    from omniserver_amd.qwen2_llm import rope_tables
    from omniserver_amd.synth import gptq_random
    say(f"o_proj from attention states fmt={fmt} splits={splits} rows={n} ksplit={ksplit}")
    cfg = ref.Qwen2Config()
    nh, nkv, hd, ML, H = 12, 2, 128, 4096, 1536
    lengths = ([2047, 31, 0, 500, 1300, 7, 64, 129] * 4)[:n]
    P = n + 1
    W = (nh + 2 * nkv) * hd
    g = torch.Generator().manual_seed(130)
    parts = (torch.randn(6, n, W, generator=g) * 0.3).to(gpu)
    bias = f16((W,), 131, 0.02).to(gpu)
    delta = torch.zeros(P, dtype=torch.int64).to(gpu)
    kc = f16((P, ML, nkv, hd), 132).to(gpu)
    vc = f16((P, ML, nkv, hd), 133).to(gpu)
    lens = torch.tensor(lengths + [0], dtype=torch.int64).to(gpu)
    cos, sin = rope_tables(cfg, 8192, gpu)
    if fmt == "int4":
        qw, sc = gptq_random(H, H, 134, "oproj")
        lin = GPTQLinear(qw.to(gpu), sc.to(gpu))
    else:
        lin = F16Linear(f16((H, H), 135, 0.02).to(gpu))
    ws = torch.empty(n * nkv * splits * 6 * 132, device=gpu, dtype=torch.float32)
    out = torch.empty(n, nh, hd, device=gpu, dtype=torch.float16)
    S_o = lin.partial_slices(ksplit)
    pa = torch.empty(S_o * n * H, device=gpu, dtype=torch.float32)
    pb = torch.empty_like(pa)

    def attn(merge):
        call("omni_decode_attention_fused", ptr(parts), 6, ptr(bias), 1, ptr(cos), ptr(sin), 8192,
             ptr(delta), 16, 24, 24, ptr(kc), ptr(vc), P, ML, None, ptr(lens),
             ptr(out) if merge else None, n, nh, nkv, hd, hd ** -0.5, 8, splits, ptr(ws),
             ws.numel(), merge, None, stream())
    attn(0)
    lin.forward_partial_attn(ws, splits, nkv, nh // nkv, n, pa, ksplit=ksplit)
    attn(1)                       # same K/V row rewritten with the same values
    lin.forward_partial(out, pb, ksplit=ksplit)
    torch.cuda.synchronize()
    assert torch.equal(pa, pb)


@pytest.mark.parametrize("length", [-1, 0, 1, 63, 64, 65, 300, 512])
def test_kv_copy_slot(gpu, length):
    """move_slot / copy_slot_kv (kv_prealloc.py:51-57, 79-84): tokens [0, L) of row src copied
    to row dst in every layer's K and V, bit-exact, nothing else written; lengths[dst] = L
    (length -1: L = lengths[src] read on the device)."""
    from omniserver_amd.kv_cache import PreallocatedKVCache
    say(f"kv slot copy length={length}")
    pool = PreallocatedKVCache(3, 5, 2, 512, 128, gpu, n_heads=12)
    g = torch.Generator().manual_seed(150)
    before = torch.randn(pool.storage.shape, generator=g).half()
    pool.storage.copy_(before)
    pool.lengths.copy_(torch.tensor([10, 300, 7, 0, 512]))
    src, dst = 1, 3
    if length < 0:
        pool.move_slot(src, dst)
        L = 300
    else:
        pool.copy_slot_kv(src, dst, length)
        L = length
    torch.cuda.synchronize()
    exp = before.clone()
    exp[:, :, dst, :L] = before[:, :, src, :L]
    assert torch.equal(pool.storage.cpu(), exp)
    assert pool.lengths.cpu().tolist() == [10, 300, 7, L, 512]
    pool.copy_slot_kv(4, 4, 5)                      # same row: only the length changes
    torch.cuda.synchronize()
    assert torch.equal(pool.storage.cpu(), exp) and int(pool.lengths[4]) == 5


# ----------------------------------------------------------------------------- fp8 W8A8
def test_fp8_quant_rows_bit_exact(gpu):
    """quant_fp8 (fp8_linear.py:45-63): per-row amax/448 scale and e4m3 codes, bit-exact."""
    from omniserver_amd._lib import call, ptr, stream
    say("fp8 row quantisation")
    M, K = 37, 1536
    x = f16((M, K), 140, 1.5)
    x[3] = 0.5                                    # constant row
    xg = x.to(gpu)
    q = torch.empty(M, K, device=gpu, dtype=torch.uint8)
    s = torch.empty(M, device=gpu, dtype=torch.float32)
    call("omni_fp8_quant_rows", ptr(xg), K, ptr(q), ptr(s), M, K, 0.0, stream())
    torch.cuda.synchronize()
    eq, es = ref.quant_fp8(x.float())
    assert torch.equal(s.cpu(), es.view(-1))
    assert torch.equal(q.cpu(), eq.view(torch.uint8))


def test_fp8_quant_weight_rows_bit_exact(gpu):
    """FP8Linear's row-wise weight form (fp8_linear.py:83-86): scale = fp16(amax / 448)
    (an op on the fp16 weight), codes = e4m3(w / scale), bit-exact."""
    from omniserver_amd._lib import call, ptr, stream
    say("fp8 row-wise weight quantisation")
    N, K = 300, 1536
    w = f16((N, K), 148, 0.02)
    w[7] = 0.25                                   # constant row
    wg = w.to(gpu)
    q = torch.empty(N, K, device=gpu, dtype=torch.uint8)
    s = torch.empty(N, device=gpu, dtype=torch.float32)
    call("omni_fp8_quant_weight_rows", ptr(wg), K, ptr(q), ptr(s), N, K, stream())
    torch.cuda.synchronize()
    eq, es = ref.fp8_weight_rowwise(w.float())
    assert torch.equal(s.cpu(), es)
    assert torch.equal(q.cpu(), eq.view(torch.uint8))


@pytest.mark.parametrize("rows,K,bf16", [(1, 384, False), (37, 1536, False), (300, 1536, True),
                                         (1000, 8960, False), (2000, 384, True)])
def test_fp8_quant_tensor_bit_exact(gpu, rows, K, bf16):
    """Per-tensor quantisation (_quant_fp8_pertensor's eager branch, fp8_linear.py:40-41;
    the per-tensor weight form :87-89): one scale R(amax / 448) over the whole tensor (an
    outlier placed in one row), codes e4m3(R(x / s)), R the input's rounding; bit-exact,
    also past the 256 rows one workgroup of the amax pass covers."""
    from omniserver_amd._lib import call, lib, ptr, stream
    say(f"fp8 per-tensor quantisation rows={rows} K={K} bf16={bf16}")
    x = f16((rows, K), 150 + rows % 17, 1.5)
    x[rows // 2, K // 3] = -37.0
    xt = x.to(torch.bfloat16) if bf16 else x
    xg = xt.to(gpu)
    q = torch.empty(rows, K, device=gpu, dtype=torch.uint8)
    s = torch.empty(rows, device=gpu, dtype=torch.float32)
    work = torch.empty(lib().omni_fp8_quant_tensor_work(rows), device=gpu, dtype=torch.float32)
    call("omni_fp8_quant_tensor", ptr(xg), K, ptr(q), ptr(s), ptr(work), rows, K, int(bf16),
         stream())
    torch.cuda.synchronize()
    eq, es = ref.quant_fp8_pertensor(xt.float(), bf16=bf16)
    assert torch.equal(s.cpu(), es.expand(rows))
    assert torch.equal(q.cpu(), eq.view(torch.uint8))


def fp8_abs_product(xq, sa, wq, sw):
    """|xq| . |wq|^T * sa * sw: the scale of the terms each output sums."""
    return (xq.float().abs() @ wq.float().abs().t()) * sa.view(-1, 1) * sw.view(1, -1)


@pytest.mark.parametrize("M,N,K,bias", [(1, 256, 1536, False), (100, 2048, 1536, True),
                                        (256, 1536, 8960, False), (130, 384, 256, True),
                                        (512, 1280, 4096, True)])
def test_fp8_linear_matches_oracle(gpu, M, N, K, bias):
    """FP8Linear.forward: bf16((xq.Wq^T)*sa*sw) -> fp16 (+bias) against the oracle on the
    same quantised operands.  The fp8 MFMA sums groups of products with fewer bits than
    fp32 (an on-device probe loses 1 next to +-448^2 inside one group, as fp8 tensor-core
    GEMMs elsewhere do), so the bound is one bf16 step of the result plus 2^-14 of the
    summed term magnitudes; nearly all outputs are still identical."""
    from omniserver_amd.linear import FP8Linear
    say(f"fp8 linear M={M} N={N} K={K} bias={bias}")
    W = f16((N, K), 141, 0.02)
    b = f16((N,), 142, 0.02) if bias else None
    x = f16((M, K), 143)
    lin = FP8Linear(W.to(gpu), None if b is None else b.to(gpu), rowwise=True)
    y = lin(x.to(gpu))
    torch.cuda.synchronize()
    wq, sw = ref.fp8_weight_rowwise(W.float())
    assert torch.equal(lin.weight_fp8.cpu(), wq.view(torch.uint8))
    assert torch.equal(lin.weight_scale.cpu(), sw)
    xq, sa = ref.quant_fp8(x.float())
    e = ref.fp8_linear_rowwise(xq, sa, wq, sw, None if b is None else b.float())
    e0 = ref.fp8_linear_rowwise(xq, sa, wq, sw, None)          # before the bias
    yc = y.cpu().float()
    d = (yc - e).abs()
    # one bf16 step of the pre-bias value (<= 2^-7 relative), the fp16 bias rounding, and
    # the MFMA's reduced intermediate precision on the summed term magnitudes
    tol = e0.abs() * 2.0 ** -7 + e.abs() * 2.0 ** -10 + fp8_abs_product(xq, sa, wq, sw) * 2.0 ** -14
    assert (d <= tol + 1e-6).all(), (d - tol).max().item()
    assert (d == 0).float().mean().item() > 0.95


@pytest.mark.parametrize("M,N,K,bias,bf16", [(1, 256, 1536, False, False),
                                              (100, 2048, 1536, True, False),
                                              (256, 1536, 8960, False, True),
                                              (512, 1280, 4096, True, False)])
def test_fp8_linear_pertensor_matches_oracle(gpu, M, N, K, bias, bf16):
    """FP8Linear's default per-tensor form (fp8_linear.py:87-90, 119-125): weight and
    activation codes and scales bit-exact, the fp16 product (+ fp16 bias) within one fp16
    step plus the MFMA's reduced intermediate precision (see test_fp8_linear_matches_oracle)."""
    from omniserver_amd.linear import FP8Linear
    say(f"fp8 per-tensor linear M={M} N={N} K={K} bias={bias} bf16 input={bf16}")
    W = f16((N, K), 161, 0.02)
    b = f16((N,), 162, 0.02) if bias else None
    x = f16((M, K), 163)
    xt = x.to(torch.bfloat16) if bf16 else x
    lin = FP8Linear(W.to(gpu), None if b is None else b.to(gpu))
    assert not lin.rowwise
    xq_g, sa_g = lin.quantize_input(xt.to(gpu))
    y = lin(xt.to(gpu))
    torch.cuda.synchronize()
    assert y.dtype == torch.float16
    wq, sw = ref.fp8_weight_pertensor(W.float())
    assert torch.equal(lin.weight_fp8.cpu(), wq.view(torch.uint8))
    assert torch.equal(lin.weight_scale.cpu(), sw.expand(N))
    assert torch.equal(lin.wscale.cpu(), sw)
    xq, sa = ref.quant_fp8_pertensor(xt.float(), bf16=bf16)
    assert torch.equal(xq_g.cpu(), xq.view(torch.uint8))
    assert torch.equal(sa_g.cpu().view(-1), sa.expand(M))
    e = ref.fp8_linear_pertensor(xq, sa, wq, sw, None if b is None else b.float())
    e0 = ref.fp8_linear_pertensor(xq, sa, wq, sw, None)
    d = (y.cpu().float() - e).abs()
    tol = (e0.abs() + e.abs()) * 2.0 ** -10 + fp8_abs_product(xq, sa, wq, sw) * 2.0 ** -14
    assert (d <= tol + 1e-6).all(), (d - tol).max().item()
    # an fp16 result has 3 more bits than the bf16 of the row-wise form, so the MFMA's
    # reduced intermediate precision shows as a last-bit difference more often (93 % of
    # the outputs bit-equal measured at M = 1)
    assert (d == 0).float().mean().item() > 0.85


def test_fp8_linear_matches_reference_fixture(gpu):
    """FP8Linear in both forms against the reference's own FP8Linear outputs
    (tests/golden/ref_fp8_route.npz, written on the CPU by make_ref_vit_fp8.py): weight
    codes and scales bit for bit; forward (fp16 and bf16 input, with and without bias) and
    forward_prequant within the bounds of the oracle tests above."""
    import os
    import sys
    import numpy as np
    from omniserver_amd.linear import FP8Linear
    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    sys.path.insert(0, golden)
    import fp8_case as P
    g = np.load(os.path.join(golden, "ref_fp8_route.npz"))
    say("fp8 linear vs the reference's FP8Linear outputs")
    w, b, x = P.linear_case()
    W, B, X = w.half().to(gpu), b.half().to(gpu), x.half().to(gpu)
    for tag, rowwise in (("pt", False), ("rw", True)):
        lin = FP8Linear(W, B, rowwise=rowwise)
        nb = FP8Linear(W, None, rowwise=rowwise)
        assert np.array_equal(lin.weight_fp8.cpu().numpy(), g[f"{tag}_wq"])
        assert np.array_equal(lin.wscale.cpu().reshape(-1).numpy(), g[f"{tag}_wscale"])
        # one step of the stored product's rounding (fp16 per-tensor, bf16 row-wise), the
        # bias rounding, and the MFMA's reduced intermediate precision (2^-10 of the
        # largest output bounds 2^-14 of any output's summed term magnitudes here)
        step = 2.0 ** -10 if tag == "pt" else 2.0 ** -7
        for key, got in ((f"{tag}_out", lin(X)), (f"{tag}_out_nobias", nb(X)),
                         (f"{tag}_out_bf16in", lin(X.bfloat16()))):
            want = torch.tensor(g[key])
            d = (got.cpu().float() - want).abs()
            tol = want.abs() * (step + 2.0 ** -10) + 2.0 ** -10 * want.abs().max() + 1e-6
            assert (d <= tol).all(), (key, (d - tol).max().item())
            assert (d == 0).float().mean().item() > 0.9, key
    rw = FP8Linear(W, B, rowwise=True)
    xq = torch.tensor(g["rw_xq"]).to(gpu)
    s = torch.tensor(g["rw_xscale"]).to(gpu)
    got = rw.forward_prequant(xq, s).cpu().float()
    want = torch.tensor(g["rw_prequant"])
    assert (got - want).abs().max().item() <= 2.0 ** -6 * want.abs().max().item()


def test_fp8_prequant_chain(gpu):
    """add_rms_norm_fp8 -> FP8Linear.forward_prequant (the reference MLP's fp8 route,
    qwen2_llm.py:130-134) returns the bf16 product of the norm-quantised rows."""
    from omniserver_amd import fused_ops as F
    from omniserver_amd.linear import FP8Linear
    say("fp8 prequant chain")
    M, H, N = 64, 1536, 1024
    x, r = f16((M, H), 144), f16((M, H), 145)
    w = (1 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(146))).half()
    W = f16((N, H), 147, 0.02)
    lin = FP8Linear(W.to(gpu), rowwise=True)
    q, s, nr = F.add_rms_norm_fp8(x.to(gpu), r.to(gpu), w.to(gpu), 1e-6)
    y = lin.forward_prequant(q, s)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16
    wq, sw = ref.fp8_weight_rowwise(W.float())
    qc = q.cpu().view(torch.float8_e4m3fn)
    e = ref.fp8_linear_rowwise(qc, s.cpu(), wq, sw, out_f16=False)
    d = (y.cpu().float() - e).abs()
    tol = e.abs() * 2.0 ** -7 + fp8_abs_product(qc, s.cpu(), wq, sw) * 2.0 ** -14
    assert (d <= tol + 1e-6).all(), (d - tol).max().item()
