"""Pins of the vision-tower oracle (oracle/qwen2_vit_ref.py) and the host tables of
omniserver_amd/vit.py, CPU only.

Each check reaches the oracle's answer by a different route than the oracle's own
formula: torch's float64 library routines (F.layer_norm, F.gelu,
scaled_dot_product_attention with a block-diagonal mask), complex multiplication for
the rotary, a per-patch loop of the merge-window order for the positions, and
invariants (norm preservation, identity at position 0, segment independence).  The
reference ships no vision golden vectors; model/qwen2_vit.py:8 states bit-equality with
Hugging Face's model.visual, which needs weights that are not on this machine.

The tower's composition (block order, norm placement, residuals, rotary on q and k, the
merger's LayerNorm -> view -> fc1 -> GELU -> fc2) is pinned against the reference's own
Qwen2VIT.forward, run on the CPU by tests/golden/make_ref_vit_fp8.py into
tests/golden/ref_vit.npz: every stage of block 0 and of the merger from the reference's
own stage inputs within one fp16 ulp, the rotary tables bit for bit, the whole tower
within a few ulps; planted mistakes in the oracle (norms swapped, a residual dropped,
rotary on q only, (h, w) swapped, the merger's GELU or LayerNorm changed, the blocks'
QuickGELU as exact GELU, an fp16 rotary table) each fail one of these checks.
"""

import math

import pytest
import torch
import torch.nn.functional as Fn

from oracle import qwen2_vit_ref as vref


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_rot_pos_ids_window_order():
    grids = [(1, 4, 6), (2, 2, 2), (1, 6, 4)]
    got = vref.rot_pos_ids(grids)
    want = []
    for t, h, w in grids:
        frame = [(bh * 2 + i, bw * 2 + j) for bh in range(h // 2) for bw in range(w // 2)
                 for i in range(2) for j in range(2)]
        want += frame * t
    assert got.tolist() == [list(p) for p in want]


def test_host_tables_match_oracle():
    from omniserver_amd import vit
    grids = [(1, 4, 6), (2, 2, 2), (1, 16, 10)]
    assert torch.equal(vit.rot_pos_ids(grids, 2).long(), vref.rot_pos_ids(grids))
    assert vit.cu_seqlens(grids).tolist() == vref.cu_seqlens(grids)
    inv = vit.vision_inv_freq(80, 10000.0)
    assert inv.dtype == torch.float32 and inv.shape == (20,)
    assert torch.allclose(inv.double(), 10000.0 ** (-torch.arange(0, 40, 2, dtype=torch.float64) / 40),
                          rtol=1e-6)
    tiles = vit.query_tiles(vit.cu_seqlens(grids)).tolist()
    cu = vref.cu_seqlens(grids)
    covered = []
    for q0, s in tiles:
        assert cu[s] <= q0 < cu[s + 1]
        covered += list(range(q0, min(q0 + 64, cu[s + 1])))
    assert covered == list(range(cu[-1]))
    with pytest.raises(ValueError):
        vit.rot_pos_ids([(1, 3, 4)], 2)


def test_rot_cos_sin_angles():
    grids = [(1, 6, 8)]
    cos, sin = vref.rot_cos_sin(grids, 80)
    pos = vref.rot_pos_ids(grids).double()
    inv = 10000.0 ** (-torch.arange(0, 40, 2, dtype=torch.float64) / 40)
    ang = torch.cat([pos[:, :1] * inv, pos[:, 1:] * inv], 1)          # [S, 40]: h, then w
    assert torch.allclose(cos[:, :40].double(), torch.cos(ang), atol=2e-6)
    assert torch.allclose(sin[:, :40].double(), torch.sin(ang), atol=2e-6)
    assert torch.equal(cos[:, :40], cos[:, 40:]) and torch.equal(sin[:, :40], sin[:, 40:])


def test_vision_rope_is_complex_rotation():
    S, nh, hd = 12, 3, 80
    q = torch.randn(S, nh, hd, generator=_g(1))
    k = torch.randn(S, nh, hd, generator=_g(2))
    cos, sin = vref.rot_cos_sin([(1, 2, 6)], hd)
    rq, rk = vref.vision_rope(q, k, cos, sin, f16=False)
    z = torch.complex(q[..., :40].double(), q[..., 40:].double())
    e = torch.complex(cos[:, None, :40].double(), sin[:, None, :40].double())
    w = z * e
    assert torch.allclose(rq[..., :40].double(), w.real, atol=1e-5)
    assert torch.allclose(rq[..., 40:].double(), w.imag, atol=1e-5)
    # rotation keeps each pair's norm; position (0, 0) is the identity
    n0 = q[..., :40] ** 2 + q[..., 40:] ** 2
    n1 = rq[..., :40] ** 2 + rq[..., 40:] ** 2
    assert torch.allclose(n0, n1, rtol=1e-5, atol=1e-5)
    assert torch.equal(rk[0], k[0])


def test_layer_norm_matches_library():
    x = torch.randn(7, 1280, generator=_g(3)) * 3 + 0.5
    w = 1 + 0.1 * torch.randn(1280, generator=_g(4))
    b = 0.1 * torch.randn(1280, generator=_g(5))
    got = vref.layer_norm(x, w, b, 1e-6, f16=False)
    want = Fn.layer_norm(x.double(), (1280,), w.double(), b.double(), 1e-6)
    assert torch.allclose(got.double(), want, atol=1e-5)


def test_gelu_forms():
    x = torch.linspace(-6, 6, 2001)
    assert torch.allclose(vref.gelu(x, f16=False).double(), Fn.gelu(x.double()), atol=1e-6)
    qg = vref.quick_gelu(x, f16=False).double()
    assert torch.allclose(qg, x.double() * torch.sigmoid(1.702 * x.double()), atol=1e-6)
    # with the fp16 roundings every value is within a few fp16 ulps of the exact one
    xh = x.half().float()
    d = (vref.quick_gelu(xh, f16=True).double() - xh.double() * torch.sigmoid(1.702 * xh.double())).abs()
    assert (d <= 3 * 2.0 ** -10 * xh.double().abs().clamp(min=2.0 ** -14) + 1e-4).all()


def test_seg_attention_block_diagonal():
    cu = [0, 5, 5 + 64, 5 + 64 + 37]
    S, nh, hd = cu[-1], 4, 80
    q, k, v = (torch.randn(S, nh, hd, generator=_g(10 + i)) for i in range(3))
    got = vref.seg_attention(q, k, v, cu, hd ** -0.5, f16=False)
    mask = torch.zeros(S, S, dtype=torch.bool)
    for a, b in zip(cu[:-1], cu[1:]):
        mask[a:b, a:b] = True
    want = Fn.scaled_dot_product_attention(q.double().transpose(0, 1), k.double().transpose(0, 1),
                                           v.double().transpose(0, 1), attn_mask=mask,
                                           scale=hd ** -0.5).transpose(0, 1)
    assert torch.allclose(got.double(), want, atol=1e-5)


def test_tower_segments_independent():
    """Two images in one call give the rows of two separate calls (cu_seqlens isolate the
    images; the merger groups 4 consecutive patches of one image)."""
    from omniserver_amd import synth
    from omniserver_amd.vit import VisionConfig
    cfg = VisionConfig(depth=1)
    sd = synth.vision_tower(cfg, seed=3, depth=1)
    g1, g2 = (1, 4, 4), (1, 2, 6)
    p1 = synth.pixel_patches([g1], cfg.patch_dim, 1).float()
    p2 = synth.pixel_patches([g2], cfg.patch_dim, 2).float()
    both = vref.vit_forward(torch.cat([p1, p2]), [g1, g2], sd, f16=False)
    a = vref.vit_forward(p1, [g1], sd, f16=False)
    b = vref.vit_forward(p2, [g2], sd, f16=False)
    assert both.shape == (4 + 3, 1536)
    # fp32: equal up to the summation order of the row-count-dependent matmuls; a segment
    # leak would move every row by far more
    assert torch.allclose(both, torch.cat([a, b]), atol=1e-4, rtol=1e-4)


# ----------------------------------------------------------------------------- reference forward
# tests/golden/ref_vit.npz: the reference's own Qwen2VIT.forward (model/qwen2_vit.py:
# 36-129, built as models/qwen2_vl.py:46-48 builds it: ``.half()``) on the seeded tower of
# tests/golden/vit_case.py (2 blocks, head_dim 80, two images over three segments), run
# on the CPU by tests/golden/make_ref_vit_fp8.py with vLLM's varlen flash attention as
# exact per-segment softmax attention and the Triton vision_rope as the module's own
# apply_rotary_vision.  Kept: every stage of block 0, block 1's input and output, the
# merger's stages, the output and the rotary tables.
import os  # noqa: E402
import sys  # noqa: E402

import numpy as np  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import vit_case as VC  # noqa: E402

TOWER_TOL = 4e-3          # whole tower: ~4 fp16 ulps at the output's magnitude (~1.2)


@pytest.fixture(scope="module")
def vit_golden():
    return np.load(os.path.join(GOLDEN, "ref_vit.npz"))


def _ulp(want: torch.Tensor) -> torch.Tensor:
    """One fp16 ulp at each value's magnitude (subnormal spacing below 2^-14)."""
    e = torch.floor(torch.log2(want.abs().clamp(min=2.0 ** -14)))
    return torch.pow(2.0, e - 10)


def _within(got, want, ulps=1, slack=2.0 ** -13, scale=None):
    """|got - want| within ``ulps`` fp16 ulps of want (or of ``scale``, elementwise, for a
    sum whose addends are larger than the result) plus ``slack`` (outputs of a GEMM that
    cancel to near zero carry the fp32 summation order's error, not one ulp of themselves)."""
    ref_mag = want if scale is None else torch.maximum(want.abs(), scale.abs())
    return bool(((got - want).abs() <= ulps * _ulp(ref_mag) + slack).all())


def test_rotary_tables_bit_equal_to_reference(vit_golden):
    assert rotary_tables_equal(vit_golden)


def block0_stage_failures(vit_golden):
    """Every op of block 0 from the reference's own stage inputs: within one fp16 ulp
    (LayerNorm's fp32 statistics and the GEMMs' summation order differ from the CPU
    library's), the attention within two.  Returns the names of the stages that differ."""
    g = lambda k: torch.tensor(vit_golden[k])
    sd = VC.state_dict()
    w = lambda k: sd["visual.blocks.0." + k].float()
    S, D, nh = g("b0_in").shape[0], VC.EMBED, VC.HEADS
    bad = []
    check = lambda name, ok: None if ok else bad.append(name)
    pe = vref.linear(VC.pixels(), sd["visual.patch_embed.proj.weight"].reshape(D, -1), None)
    check("patch_embed", _within(pe, g("b0_in")))
    check("norm1", _within(vref.layer_norm(g("b0_in"), w("norm1.weight"), w("norm1.bias")),
                           g("b0_norm1")))
    check("qkv", _within(vref.linear(g("b0_norm1"), w("attn.qkv.weight"), w("attn.qkv.bias")),
                         g("b0_qkv")))
    cos, sin = vref.rot_cos_sin(VC.GRIDS, D // nh, VC.THETA, VC.MERGE)
    qkv = g("b0_qkv").view(S, 3, nh, D // nh)
    q, k = vref.vision_rope(qkv[:, 0], qkv[:, 1], cos, sin)
    o = vref.seg_attention(q, k, qkv[:, 2], vref.cu_seqlens(VC.GRIDS), (D // nh) ** -0.5)
    check("attention", _within(o.reshape(S, D), g("b0_attn"), 2))
    # residual adds: one ulp of the larger addend (the projection's own rounding)
    a = vref.linear(g("b0_attn"), w("attn.proj.weight"), w("attn.proj.bias"))
    check("proj+residual", _within(vref.r16(g("b0_in") + a), g("b0_mid"), scale=a))
    check("norm2", _within(vref.layer_norm(g("b0_mid"), w("norm2.weight"), w("norm2.bias")),
                           g("b0_norm2")))
    check("fc1", _within(vref.linear(g("b0_norm2"), w("mlp.fc1.weight"), w("mlp.fc1.bias")),
                         g("b0_fc1")))
    check("quick_gelu", _within(vref.quick_gelu(g("b0_fc1")), g("b0_act")))
    m = vref.linear(g("b0_act"), w("mlp.fc2.weight"), w("mlp.fc2.bias"))
    check("fc2+residual", _within(vref.r16(g("b0_mid") + m), g("b0_out"), scale=m))
    return bad


def test_block0_stages_match_reference(vit_golden):
    assert block0_stage_failures(vit_golden) == []


def merger_stage_failures(vit_golden):
    g = lambda k: torch.tensor(vit_golden[k])
    sd = VC.state_dict()
    w = lambda k: sd["visual.merger." + k].float()
    bad = []
    check = lambda name, ok: None if ok else bad.append(name)
    check("ln_q", _within(vref.layer_norm(g("b1_out"), w("ln_q.weight"), w("ln_q.bias")),
                          g("merger_ln")))
    m = VC.EMBED * VC.MERGE * VC.MERGE
    f1 = vref.linear(g("merger_ln").reshape(-1, m), w("mlp.0.weight"), w("mlp.0.bias"))
    check("fc1", _within(f1, g("merger_fc1")))
    check("gelu", _within(vref.gelu(g("merger_fc1")), g("merger_act")))
    check("fc2", _within(vref.linear(g("merger_act"), w("mlp.2.weight"), w("mlp.2.bias")),
                         g("out")))
    return bad


def test_merger_stages_match_reference(vit_golden):
    """merger_ln_q -> view(-1, 4 D) -> merger_fc1 -> GELU -> merger_fc2
    (model/qwen2_vit.py:128) from the reference's own stage inputs."""
    assert merger_stage_failures(vit_golden) == []


def rotary_tables_equal(vit_golden):
    cos, sin = vref.rot_cos_sin(VC.GRIDS, VC.EMBED // VC.HEADS, VC.THETA, VC.MERGE)
    return np.array_equal(cos.numpy(), vit_golden["cos"]) and \
        np.array_equal(sin.numpy(), vit_golden["sin"])


def tower_error(vit_golden):
    """Max-abs difference of the oracle's whole tower (fp16 mode) from the reference's
    output, and of its block-1 input (block 0's output)."""
    sd = VC.state_dict()
    y = vref.vit_forward(VC.pixels(), VC.GRIDS, sd, n_heads=VC.HEADS, m=VC.MERGE, theta=VC.THETA)
    return float(np.abs(y.numpy() - vit_golden["out"]).max())


def test_tower_matches_reference_forward(vit_golden):
    """The oracle's tower end to end: the stages above compose in the reference's order
    (measured 1.1e-3, the rounding differences of the stages carried through)."""
    assert tower_error(vit_golden) <= TOWER_TOL


# planted mistakes in the oracle's tower composition, each built from the oracle's own
# leaves; every one must move the tower's output far past TOWER_TOL
def _block_with(mistake):
    def block(x, sd, p, cos, sin, cu, n_heads=16, f16=True):
        g = lambda key: sd[p + key].float()
        S, D = x.shape
        hd = D // n_heads
        n1, n2 = ("norm2", "norm1") if mistake == "swap_norms" else ("norm1", "norm2")
        h = vref.layer_norm(x, g(n1 + ".weight"), g(n1 + ".bias"), f16=f16)
        qkv = vref.linear(h, g("attn.qkv.weight"), g("attn.qkv.bias"), f16).view(S, 3, n_heads, hd)
        q, k = vref.vision_rope(qkv[:, 0], qkv[:, 1], cos, sin, f16)
        if mistake == "rotary_q_only":
            k = qkv[:, 1]
        o = vref.seg_attention(q, k, qkv[:, 2], cu, hd ** -0.5, f16)
        a = vref.linear(o.reshape(S, D), g("attn.proj.weight"), g("attn.proj.bias"), f16)
        x = a if mistake == "drop_attn_residual" else vref.r16(x + a, f16)
        h = vref.layer_norm(x, g(n2 + ".weight"), g(n2 + ".bias"), f16=f16)
        f = vref.linear(h, g("mlp.fc1.weight"), g("mlp.fc1.bias"), f16)
        f = vref.gelu(f, f16) if mistake == "exact_gelu_in_blocks" else vref.quick_gelu(f, f16)
        m = vref.linear(f, g("mlp.fc2.weight"), g("mlp.fc2.bias"), f16)
        return m if mistake == "drop_mlp_residual" else vref.r16(x + m, f16)
    return block


BLOCK_MISTAKES = ["swap_norms", "rotary_q_only", "drop_attn_residual", "drop_mlp_residual"]


@pytest.mark.parametrize("mistake", BLOCK_MISTAKES)
def test_planted_block_mistake_is_caught(mistake, monkeypatch, vit_golden):
    monkeypatch.setattr(vref, "vit_block", _block_with(mistake))
    assert tower_error(vit_golden) > 10 * TOWER_TOL


def test_planted_gelu_form_is_caught(monkeypatch, vit_golden):
    """The blocks' QuickGELU (three fp16 roundings) replaced by the exact GELU: too small
    a change to show at the tower's output through these weights, caught at its stage."""
    monkeypatch.setattr(vref, "quick_gelu", lambda x, f16=True: vref.gelu(x, f16))
    assert "quick_gelu" in block0_stage_failures(vit_golden)


def test_planted_block_rewrite_is_faithful(monkeypatch, vit_golden):
    """The rewritten block without a mistake is the oracle's block: the planted variants
    differ from it in the named step only."""
    monkeypatch.setattr(vref, "vit_block", _block_with(None))
    assert tower_error(vit_golden) <= TOWER_TOL


def all_failures(vit_golden):
    """The names of every reference-forward check above that fails."""
    bad = block0_stage_failures(vit_golden) + ["merger:" + n for n in merger_stage_failures(vit_golden)]
    if not rotary_tables_equal(vit_golden):
        bad.append("rotary tables")
    if tower_error(vit_golden) > TOWER_TOL:
        bad.append("tower output")
    return bad


def _skip_merger_ln(orig):
    lnw = VC.state_dict()["visual.merger.ln_q.weight"].float()

    def ln(x, w, b, eps=1e-6, f16=True):
        return x if torch.equal(w, lnw) else orig(x, w, b, eps, f16)
    return ln


def test_planted_tower_mistakes_are_caught(monkeypatch, vit_golden):
    """Patch positions (h, w) swapped; the merger's GELU as QuickGELU; the merger's
    LayerNorm skipped; the rotary's fp32 table rounded to fp16 (the reference keeps it
    fp32, qwen2_vit.py:107-109, 122): each fails at least one check above."""
    orig_pos, orig_ln, orig_cs = vref.rot_pos_ids, vref.layer_norm, vref.rot_cos_sin
    cases = {
        "swap_hw": ("rot_pos_ids", lambda grid, m=2: orig_pos(grid, m).flip(-1)),
        "merger_quick_gelu": ("gelu", lambda x, f16=True: vref.quick_gelu(x, f16)),
        "merger_ln_skipped": ("layer_norm", _skip_merger_ln(orig_ln)),
        "fp16_rotary_table": ("rot_cos_sin", lambda *a, **k: tuple(
            vref.r16(t) for t in orig_cs(*a, **k))),
    }
    for name, (attr, fn) in cases.items():
        with monkeypatch.context() as mp:
            mp.setattr(vref, attr, fn)
            assert all_failures(vit_golden), name
