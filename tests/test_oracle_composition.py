"""Pins the composition of the oracle's decoder (oracle/qwen2_ref.py ``Qwen2Ref.prefill`` /
``decode_step``): op order, slices, head map, residual threading and fp16 rounding points.

1. Against the reference's own forward.  tests/golden/ref_composition.npz holds what
   omniserve's ``Qwen2LLM.forward`` (model/qwen2_llm.py:179-190 with DecoderLayer :145-157,
   Attention :86-113 through its cache.update + SDPA branch, MLP :123-134), built as
   models/qwen2_vl.py:50 builds it (``.half()``) and run on the CPU in fp16 by
   tests/golden/make_ref_composition.py, produced on the seeded case of composition_case.py:
   two prompts (one with an image run and 3-D M-RoPE positions) prefilled into pool rows 0
   and 1, then four decode steps.  The oracle in its fp16 mode reproduces
     * every K/V row layer 0 writes, prefill and decode, bit for bit (input RMSNorm, qkv
       linear + bias with one rounding, q|k|v split, M-RoPE from the fp16 inverse-frequency
       buffer with its three fp16 roundings, write at the token's position);
     * layer 0's MLP input bit for bit from the reference's o_proj output, and o_proj /
       SiLU-mul / down within one fp16 ulp (fp32 summation order of the CPU GEMM);
     * the logits within 1e-2 (measured 5e-3): the one difference is inside the attention
       (torch's fp16 CPU SDPA rounds internally; the oracle's softmax is exact), and with
       torch's SDPA called the way the reference calls it in place of the oracle's attention
       the layer-0 attention output agrees to one fp16 ulp;
     * the M-RoPE position ids and rope deltas of five prompts (positions.py:17-58), also
       for the product's positions function.
2. Closed forms (float64, the oracle's fp32 mode) with special weights, each reducing the
   decoder to a formula that names the structure it pins:
     silenced   o_proj = 0, down = 0: logits = E . rmsnorm(E[id]) w_final (embedding row,
                first-layer residual, final norm, tied lm_head)
     one key    empty context, o_proj = I, down = 0: attention over the single new key
                returns its v, so the residual is x + [v_{h // G}]_h (v slice of q|k|v, GQA
                head map, o_proj placement); the K row written is k rotated by
                (0 + rope_delta) * inv_freq as a complex multiplication
     two keys   one cached key: softmax of q.k / sqrt(128) over the cached and the new key,
                q and k rotated at position 1 + rope_delta (scale, inclusive keys, rotation)
     mlp        o_proj = 0, down = I: residual x + silu(h Wg) * (h Wu) with h = rmsnorm(x)
                w_post (gate|up order, post-attention norm)
     threading  two layers as above: layer 2's MLP sees rmsnorm(x + m1) w_post2 and the final
                norm sees x + m1 + m2 (the MLP output joins the residual at the next norm)
3. Planted mistakes in the oracle (k/v slices swapped, head map h % n_kv, a residual add
   dropped, gate/up swapped, the fp32 inverse-frequency buffer) each fail at least one of
   the checks above.
"""

import os
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import qwen2_ref as ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import composition_case as C  # noqa: E402


# ----------------------------------------------------------------------------- fixture
def _case_oracle(f16=True):
    cfg = ref.Qwen2Config(hidden_size=C.HIDDEN, num_layers=C.LAYERS, num_heads=C.HEADS,
                          num_kv_heads=C.KV_HEADS, head_dim=C.HEAD_DIM,
                          intermediate_size=C.INTER, vocab_size=C.VOCAB, rms_norm_eps=C.EPS,
                          rope_theta=C.THETA, mrope_section=list(C.SECTIONS))
    w = C.weights()
    layers = [ref.LayerWeights(
        in_norm=l["in_norm"], post_norm=l["post_norm"], qkv_t=l["qkv_w"].t().contiguous(),
        qkv_b=l["qkv_b"], o_t=l["o_w"].t().contiguous(),
        gate_up_t=l["gate_up_w"].t().contiguous(), down_t=l["down_w"].t().contiguous())
        for l in w["layers"]]
    return ref.Qwen2Ref(cfg, w["embed"], w["norm"], layers, False, f16)


def _run_case(orc):
    kp = [torch.zeros(3, C.MAX_LEN, C.KV_HEADS, C.HEAD_DIM) for _ in range(C.LAYERS)]
    vp = [torch.zeros_like(k) for k in kp]
    lens = torch.zeros(3, dtype=torch.int64)
    pre, deltas = [], []
    for slot, (ids, img, grids) in enumerate(C.prompts()):
        emb = orc.embed[torch.tensor(ids)].clone()
        if img is not None:
            emb[torch.tensor(ids) == C.CASE_IMAGE_ID] = img
        if grids:
            pos, d = ref.mrope_position_ids(ids, grids, C.CASE_IMAGE_ID, C.CASE_VSTART_ID)
        else:
            pos, d = torch.arange(len(ids)).view(1, -1).expand(3, -1), 0
        pre.append(orc.prefill(emb, pos, [len(ids)], [slot], kp, vp, lens)[0])
        deltas.append(d)
    rd = torch.tensor(deltas + [0])
    dec = []
    for ids in C.decode_ids():
        dec.append(orc.decode_step(ids, kp, vp, lens, rd))
        lens[:2] += 1
    return torch.stack(pre), torch.stack(dec), kp, vp, lens, deltas


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(GOLDEN, "ref_composition.npz"))


@pytest.fixture(scope="module")
def case_f16():
    return _run_case(_case_oracle(True))


def test_fixture_inv_freq_is_the_fp16_buffer(golden):
    cfg = ref.Qwen2Config(head_dim=C.HEAD_DIM, rope_theta=C.THETA)
    assert np.array_equal(golden["inv_freq"], ref.inv_freq(cfg).numpy())
    assert not np.array_equal(golden["inv_freq"], ref.inv_freq(cfg, f16_buffer=False).numpy())


def test_layer0_kv_rows_bit_exact(golden, case_f16):
    _, _, kp, vp, lens, deltas = case_f16
    assert lens[:2].tolist() == golden["lengths"].tolist()
    assert deltas == golden["rope_delta"].tolist()
    for name, pool in (("k", kp), ("v", vp)):
        got = pool[0][:2].numpy()
        want = golden[f"{name}_pool"][0].astype(np.float32)
        assert np.array_equal(got, want), f"layer-0 {name} rows differ"
        for l in range(1, C.LAYERS):      # deeper layers carry the attention's rounding
            d = np.abs(pool[l][:2].numpy() - golden[f"{name}_pool"][l].astype(np.float32))
            assert d.max() <= 8e-3, (name, l, d.max())


def test_logits_match_reference_forward(golden, case_f16):
    pre, dec, *_ = case_f16
    for got, want in ((pre, golden["prefill_logits"]), (dec, golden["decode_logits"])):
        want = torch.tensor(want)
        assert (got - want).abs().max().item() <= 1e-2
        cos = F.cosine_similarity(got.reshape(-1, C.VOCAB), want.reshape(-1, C.VOCAB), dim=-1)
        assert cos.min().item() >= 0.99999
        margin = ref.top2_margin(want)
        decisive = margin > 2e-2
        assert torch.equal(got.argmax(-1)[decisive], want.argmax(-1)[decisive])


def _layer0_inputs():
    w = C.weights()
    l0 = w["layers"][0]
    orc = _case_oracle(True)
    ids = C.prompts()[0][0]
    x = w["embed"][torch.tensor(ids)]
    return orc, l0, x, len(ids)


def test_layer0_intermediates(golden):
    """Layer 0 of the first prompt's prefill, op by op from the reference's own inputs."""
    orc, l0, x, T = _layer0_inputs()
    lw = orc.layers[0]
    tap = lambda k: torch.tensor(golden[f"l0_prefill_{k}"])
    h, _ = ref.rms_norm(x, lw.in_norm, C.EPS), None
    q, k, v = orc._attn_in(h, lw, torch.arange(T).view(1, -1).expand(3, -1))
    # attention: torch's fp16 SDPA called as Attention.forward calls it (qwen2_llm.py:108-113)
    rep = C.HEADS // C.KV_HEADS
    q4 = q.transpose(0, 1)[None].half()
    k4 = k.transpose(0, 1)[None].repeat_interleave(rep, 1).half()
    v4 = v.transpose(0, 1)[None].repeat_interleave(rep, 1).half()
    mask = torch.ones(T, T, dtype=torch.bool).tril()
    sdpa = F.scaled_dot_product_attention(q4, k4, v4, attn_mask=mask)[0].transpose(0, 1)
    ulp = 2.0 ** -10
    assert (sdpa.float().reshape(T, -1) - tap("attn")).abs().max().item() <= ulp
    # the oracle's exact-softmax attention: within a few fp16 ulps of it
    exact = ref.prefill_attention(q, k, v, [T], C.HEAD_DIM ** -0.5)
    assert (exact.reshape(T, -1) - tap("attn")).abs().max().item() <= 4 * ulp
    o = ref.linear(tap("attn"), lw.o_t, None)
    assert (o - tap("o")).abs().max().item() <= ulp
    mlp_in, _ = ref.add_rms_norm(tap("o"), x, lw.post_norm, C.EPS)
    assert torch.equal(mlp_in, tap("mlp_in"))
    act = ref.silu_mul(ref.linear(tap("mlp_in"), lw.gate_up_t, None))
    assert (act - tap("act")).abs().max().item() <= ulp
    out = ref.linear(tap("act"), lw.down_t, None)
    assert (out - tap("mlp_out")).abs().max().item() <= ulp


def test_positions_match_reference(golden):
    from omniserver_amd.positions import mrope_positions
    for i, (ids, grids) in enumerate(C.position_cases()):
        want = golden[f"pos{i}"]
        want_d = int(golden[f"pos{i}_delta"])
        pos, d = ref.mrope_position_ids(ids, grids)
        assert np.array_equal(pos.numpy(), want) and d == want_d, i
        p2, d2 = mrope_positions(ids, grids)
        assert np.array_equal(p2.numpy(), want) and d2 == want_d, i


# ----------------------------------------------------------------------------- closed forms
H, NH, NKV, HD, V = 512, 4, 2, 128, 300
G = NH // NKV
SEC = [16, 24, 24]


def _rnd(shape, tag, std=1.0):
    g = torch.Generator().manual_seed(sum(ord(c) * (i + 3) for i, c in enumerate(tag)))
    return (torch.randn(*shape, generator=g) * std).half().float()


def _cf_oracle(n_layers, o_mode, down_mode, f16=False):
    cfg = ref.Qwen2Config(hidden_size=H, num_layers=n_layers, num_heads=NH, num_kv_heads=NKV,
                          head_dim=HD, intermediate_size=H, vocab_size=V)
    layers = []
    for i in range(n_layers):
        qkv_out = (NH + 2 * NKV) * HD
        o_t = torch.zeros(NH * HD, H) if o_mode == "zero" else torch.eye(H)
        down_t = torch.zeros(H, H) if down_mode == "zero" else torch.eye(H)
        layers.append(ref.LayerWeights(
            in_norm=1 + _rnd((H,), f"in{i}", 0.2), post_norm=1 + _rnd((H,), f"post{i}", 0.2),
            qkv_t=_rnd((H, qkv_out), f"qkv{i}", 0.05), qkv_b=_rnd((qkv_out,), f"b{i}", 0.2),
            o_t=o_t, gate_up_t=_rnd((H, 2 * H), f"gu{i}", 0.08), down_t=down_t))
    return ref.Qwen2Ref(cfg, _rnd((V, H), "E", 0.05), 1 + _rnd((H,), "fin", 0.2), layers,
                        False, f16)


def _np(t):
    return t.double().numpy()


def _rms(x, w):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * w


def _silu(g):
    return g / (1 + np.exp(-g))


def _rotate(x, p, inv):
    """x [..., 128] rotated by angle p * inv_d on the pairs (d, d + 64)."""
    z = x[..., :64] + 1j * x[..., 64:]
    r = z * np.exp(1j * p * inv)
    return np.concatenate([r.real, r.imag], -1)


def _split_qkv(qkv):
    return (qkv[..., :NH * HD].reshape(-1, NH, HD),
            qkv[..., NH * HD:(NH + NKV) * HD].reshape(-1, NKV, HD),
            qkv[..., (NH + NKV) * HD:].reshape(-1, NKV, HD))


def _pool(n, L, tag):
    kp = [torch.zeros(n + 1, 8, NKV, HD) for _ in range(2)]
    vp = [torch.zeros_like(k) for k in kp]
    for l in range(2):
        kp[l][:n, :L] = _rnd((n, L, NKV, HD), f"k{tag}{l}")
        vp[l][:n, :L] = _rnd((n, L, NKV, HD), f"v{tag}{l}")
    return kp, vp


IDS = [17, 250]
DELTA = torch.tensor([7, -3, 0])


def cf_silenced(f16=False):
    orc = _cf_oracle(1, "zero", "zero", f16)
    kp, vp = _pool(2, 5, "s")
    lg = orc.decode_step(IDS, kp, vp, torch.tensor([5, 5, 0]), DELTA)
    x = _np(orc.embed[IDS])
    want = _rms(x, _np(orc.final_norm)) @ _np(orc.embed).T
    return np.abs(_np(lg) - want).max()


def cf_one_key(f16=False):
    orc = _cf_oracle(1, "eye", "zero", f16)
    kp, vp = _pool(2, 0, "o")
    lg = orc.decode_step(IDS, kp, vp, torch.tensor([0, 0, 0]), DELTA)
    lw = orc.layers[0]
    x = _np(orc.embed[IDS])
    qkv = _rms(x, _np(lw.in_norm)) @ _np(lw.qkv_t) + _np(lw.qkv_b)
    _, k, v = _split_qkv(qkv)
    resid = x + np.concatenate([v[:, h // G] for h in range(NH)], -1)
    want = _rms(resid, _np(orc.final_norm)) @ _np(orc.embed).T
    err = np.abs(_np(lg) - want).max()
    inv = _np(ref.inv_freq(orc.cfg))
    for b in range(2):
        krow = _rotate(k[b], 0 + int(DELTA[b]), inv)
        err = max(err, np.abs(_np(kp[0][b, 0]) - krow).max(), np.abs(_np(vp[0][b, 0]) - v[b]).max())
    return err


def cf_two_keys(f16=False):
    orc = _cf_oracle(1, "eye", "zero", f16)
    kp, vp = _pool(2, 1, "t")
    k0, v0 = _np(kp[0][:2, 0]), _np(vp[0][:2, 0])
    lg = orc.decode_step(IDS, kp, vp, torch.tensor([1, 1, 0]), DELTA)
    lw = orc.layers[0]
    x = _np(orc.embed[IDS])
    q, k, v = _split_qkv(_rms(x, _np(lw.in_norm)) @ _np(lw.qkv_t) + _np(lw.qkv_b))
    inv = _np(ref.inv_freq(orc.cfg))
    outs = []
    for b in range(2):
        p = 1 + int(DELTA[b])
        qr, kr = _rotate(q[b], p, inv), _rotate(k[b], p, inv)
        heads = []
        for h in range(NH):
            g = h // G
            s = np.array([qr[h] @ k0[b, g], qr[h] @ kr[g]]) / np.sqrt(HD)
            e = np.exp(s - s.max())
            heads.append((e[0] * v0[b, g] + e[1] * v[b, g]) / e.sum())
        outs.append(np.concatenate(heads))
    resid = x + np.stack(outs)
    want = _rms(resid, _np(orc.final_norm)) @ _np(orc.embed).T
    return np.abs(_np(lg) - want).max()


def _mlp(h, lw):
    gu = h @ _np(lw.gate_up_t)
    return _silu(gu[:, :H]) * gu[:, H:]


def cf_mlp(f16=False):
    orc = _cf_oracle(1, "zero", "eye", f16)
    kp, vp = _pool(2, 3, "m")
    lg = orc.decode_step(IDS, kp, vp, torch.tensor([3, 3, 0]), DELTA)
    lw = orc.layers[0]
    x = _np(orc.embed[IDS])
    resid = x + _mlp(_rms(x, _np(lw.post_norm)), lw)
    want = _rms(resid, _np(orc.final_norm)) @ _np(orc.embed).T
    return np.abs(_np(lg) - want).max()


def cf_threading(f16=False):
    orc = _cf_oracle(2, "zero", "eye", f16)
    kp, vp = _pool(2, 3, "r")
    lg = orc.decode_step(IDS, kp, vp, torch.tensor([3, 3, 0]), DELTA)
    l1, l2 = orc.layers
    x = _np(orc.embed[IDS])
    m1 = _mlp(_rms(x, _np(l1.post_norm)), l1)
    r1 = x + m1
    m2 = _mlp(_rms(r1, _np(l2.post_norm)), l2)
    want = _rms(r1 + m2, _np(orc.final_norm)) @ _np(orc.embed).T
    return np.abs(_np(lg) - want).max()


CLOSED_FORMS = {"silenced": cf_silenced, "one_key": cf_one_key, "two_keys": cf_two_keys,
                "mlp": cf_mlp, "threading": cf_threading}
TOL32 = 2e-4        # fp32 evaluation of the same sums (float64 closed form)
TOL16 = 2e-2        # fp16 storage points in between


@pytest.mark.parametrize("name", list(CLOSED_FORMS))
def test_closed_form_fp32(name):
    err = CLOSED_FORMS[name](f16=False)
    assert err <= TOL32, (name, err)


@pytest.mark.parametrize("name", list(CLOSED_FORMS))
def test_closed_form_fp16_mode(name):
    err = CLOSED_FORMS[name](f16=True)
    assert err <= TOL16, (name, err)


# ----------------------------------------------------------------------------- planted mistakes
def _swap_kv(monkeypatch):
    orig = ref.Qwen2Ref._attn_in

    def bad(self, x, lw, pos3):
        q, k, v = orig(self, x, lw, pos3)
        return q, v, k
    monkeypatch.setattr(ref.Qwen2Ref, "_attn_in", bad)


def _remap_heads_attention():
    orig = ref.decode_attention

    def bad(q, k_pool, v_pool, rows, kv_len, scale, f16=True, p16=False):
        n, nh, hd = q.shape
        nkv = k_pool.shape[2]
        out = torch.empty(n, nh, hd)
        for h in range(nh):                       # head h reads kv head h % nkv
            g = h % nkv
            out[:, h:h + 1] = orig(q[:, h:h + 1], k_pool[:, :, g:g + 1], v_pool[:, :, g:g + 1],
                                   rows, kv_len, scale, f16, p16)
        return out
    return bad


def _drop_residual(monkeypatch):
    monkeypatch.setattr(ref, "add_rms_norm",
                        lambda x, residual, w, eps, f16=True: (ref.rms_norm(x, w, eps, f16), residual))


def _swap_gate_up(monkeypatch):
    orig = ref.silu_mul

    def bad(gate_up, f16=True):
        n = gate_up.shape[-1] // 2
        return orig(torch.cat([gate_up[..., n:], gate_up[..., :n]], -1), f16)
    monkeypatch.setattr(ref, "silu_mul", bad)


def _fp32_inv_freq(monkeypatch):
    orig = ref.inv_freq
    monkeypatch.setattr(ref, "inv_freq", lambda cfg, f16_buffer=True: orig(cfg, False))


MISTAKES = {"swap_kv": _swap_kv,
            "head_map_mod": lambda mp: mp.setattr(ref, "decode_attention", _remap_heads_attention()),
            "drop_residual": _drop_residual, "swap_gate_up": _swap_gate_up,
            "fp32_inv_freq": _fp32_inv_freq}


@pytest.mark.parametrize("mistake", list(MISTAKES))
def test_planted_mistake_is_caught(mistake, monkeypatch, golden):
    MISTAKES[mistake](monkeypatch)
    caught = [n for n, f in CLOSED_FORMS.items() if f(f16=False) > 100 * TOL32]
    if mistake == "fp32_inv_freq":
        # the closed forms take inv_freq from the oracle; the reference's own K rows do not
        _, _, kp, _, _, _ = _run_case(_case_oracle(True))
        if not np.array_equal(kp[0][:2].numpy(), golden["k_pool"][0].astype(np.float32)):
            caught.append("fixture k rows")
    assert caught, f"planted mistake {mistake} passed every check"
