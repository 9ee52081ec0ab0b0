"""Pins of the vision-tower oracle (oracle/qwen2_vit_ref.py) and the host tables of
omniserver_amd/vit.py, CPU only.

Each check reaches the oracle's answer by a different route than the oracle's own
formula: torch's float64 library routines (F.layer_norm, F.gelu,
scaled_dot_product_attention with a block-diagonal mask), complex multiplication for
the rotary, a per-patch loop of the merge-window order for the positions, and
invariants (norm preservation, identity at position 0, segment independence).  The
reference ships no vision golden vectors; model/qwen2_vit.py:8 states bit-equality with
Hugging Face's model.visual, which needs weights that are not on this machine.
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
