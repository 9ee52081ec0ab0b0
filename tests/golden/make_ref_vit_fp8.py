"""Writes tests/golden/ref_vit.npz and tests/golden/ref_fp8_route.npz: outputs of the
reference's own vision tower and FP8 W8A8 modules on the seeded cases of vit_case.py,
fp8_case.py and composition_case.py, in this container's CPU PyTorch.

What runs is omniserve's code from /root/reference, imported here (never shipped, never
run on a GPU box):
  * model/qwen2_vit.py  Qwen2VIT.forward (patch-embed matmul, _rot_pos_emb, cu_seqlens,
    the blocks, merger_ln_q -> view -> merger_fc1 -> GELU -> merger_fc2), VisionBlock
    forward / attn, load_vit_from_state_dict, built as models/qwen2_vl.py:46-48 builds it
    (``.half()``);
  * kernels/fp8_linear.py  FP8Linear (both weight forms, forward, forward_prequant,
    _quant_fp8_pertensor's eager branch);
  * kernels/mixed_precision.py  apply_mixed, fuse_norm_fp8; model/qwen2_llm.py
    RMSNorm.forward (fp8_out), MLP.forward, the decoder of make_ref_composition.py.
Stand-ins, for what cannot run on a CPU in this image:
  * vLLM's flash_attn_varlen_func (VisionBlock.attn) -> exact softmax attention per
    segment (torch's scaled_dot_product_attention on the fp32 values, fp16 result);
  * kernels/vision_rope.py's Triton kernel -> the module's own apply_rotary_vision
    (qwen2_vit.py:27-33, the formula the kernel fuses);
  * kernels/fused_ops.py's Triton kernels (rms_norm, add_rms_norm, add_rms_norm_fp8,
    silu_mul) and fp8_linear.py's quant_fp8 -> torch evaluations of the same per-row
    formulas (fp32 math, stored in the kernel's output dtype);
  * torch._scaled_mm with row-wise scales (the CPU build takes per-tensor scales only) ->
    fp32 accumulation times the row and column scales, rounded once to the output dtype.
    Per-tensor _scaled_mm is torch's own CPU routine.
vLLM is not installed, so _quant_fp8_pertensor takes its eager branch (fp8_linear.py:40-41).

Run: python tests/golden/make_ref_vit_fp8.py   (needs /root/reference)
"""

import os
import sys
import types

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import composition_case as C  # noqa: E402
import fp8_case as P  # noqa: E402
import make_ref_composition as MRC  # noqa: E402
import vit_case as V  # noqa: E402

REF = "/root/reference"
OUT_VIT = os.path.join(HERE, "ref_vit.npz")
OUT_FP8 = os.path.join(HERE, "ref_fp8_route.npz")
E4M3 = torch.float8_e4m3fn


# ----------------------------------------------------------------------------- stand-ins
def _flash_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                  softmax_scale, causal=False):
    assert not causal and torch.equal(cu_seqlens_q, cu_seqlens_k)
    cu = cu_seqlens_q.tolist()
    out = torch.empty_like(q)
    for s0, s1 in zip(cu[:-1], cu[1:]):
        qs, ks, vs = (t[s0:s1].transpose(0, 1).float()[None] for t in (q, k, v))
        o = F.scaled_dot_product_attention(qs, ks, vs, scale=softmax_scale)[0]
        out[s0:s1] = o.transpose(0, 1).to(q.dtype)
    return out


def _install_vllm_flash():
    mods = {n: types.ModuleType(n) for n in
            ("vllm", "vllm.vllm_flash_attn", "vllm.vllm_flash_attn.flash_attn_interface")}
    mods["vllm.vllm_flash_attn.flash_attn_interface"].flash_attn_varlen_func = _flash_varlen
    sys.modules.update(mods)


def _torch_fp8_ops(FO, FL):
    def add_rms_norm_fp8(x, residual, weight, eps):
        n = x.shape[-1]
        x2, r2 = x.reshape(-1, n), residual.reshape(-1, n)
        r16 = (r2.float() + x2.float()).to(residual.dtype)
        rf = r16.float()
        rstd = 1.0 / torch.sqrt((rf * rf).sum(-1, keepdim=True) / n + eps)
        y = rf * rstd * weight.float()
        scale = torch.clamp(y.abs().amax(-1, keepdim=True) / 448.0, min=1e-12)
        return (y / scale).to(E4M3), scale, r16.reshape(residual.shape)

    def quant_fp8(x):
        x2 = x.reshape(-1, x.shape[-1]).float()
        s = x2.abs().amax(-1, keepdim=True) / 448.0
        return (x2 / s).to(E4M3), s

    FO.add_rms_norm_fp8 = add_rms_norm_fp8
    FL.quant_fp8 = quant_fp8


_SCALED_MM = torch._scaled_mm


def _scaled_mm(a, b, scale_a, scale_b, out_dtype, **kw):
    if scale_a.numel() == 1 and scale_b.numel() == 1:
        return _SCALED_MM(a, b, scale_a=scale_a, scale_b=scale_b, out_dtype=out_dtype, **kw)
    y = (a.float() @ b.float()) * scale_a.float().reshape(-1, 1) * scale_b.float().reshape(1, -1)
    return y.to(out_dtype)


# ----------------------------------------------------------------------------- vision tower
def vit_fixture():
    import omniserve.kernels.vision_rope as VR
    import omniserve.model.qwen2_vit as QV
    _install_vllm_flash()
    VR.vision_rope = lambda q, k, cos, sin: QV.apply_rotary_vision(q, k, cos, sin)
    vit = QV.Qwen2VIT(embed_dim=V.EMBED, depth=V.DEPTH, n_heads=V.HEADS, in_chans=V.IN_CH,
                      patch_size=V.PATCH, temporal_patch_size=V.TPATCH,
                      spatial_merge_size=V.MERGE, mlp_ratio=V.MLP // V.EMBED,
                      out_hidden=V.OUT, rope_theta=V.THETA)
    QV.load_vit_from_state_dict(vit, V.state_dict())
    vit = vit.half().eval()                     # models/qwen2_vl.py:48
    out = {}

    def tap(name, which):
        def hook(mod, inp, res):
            t = inp[0] if which == "in" else res
            out[name] = t.float().numpy().copy()
        return hook

    for i, blk in enumerate(vit.blocks):
        blk.register_forward_hook(tap(f"b{i}_in", "in"))
        blk.register_forward_hook(tap(f"b{i}_out", "out"))
        if i > 0:                               # every stage of block 0, the others' ends
            continue
        blk.norm1.register_forward_hook(tap(f"b{i}_norm1", "out"))
        blk.attn_qkv.register_forward_hook(tap(f"b{i}_qkv", "out"))
        blk.attn_proj.register_forward_hook(tap(f"b{i}_attn", "in"))
        blk.norm2.register_forward_hook(tap(f"b{i}_mid", "in"))
        blk.norm2.register_forward_hook(tap(f"b{i}_norm2", "out"))
        blk.fc1.register_forward_hook(tap(f"b{i}_fc1", "out"))
        blk.fc2.register_forward_hook(tap(f"b{i}_act", "in"))
    vit.merger_ln_q.register_forward_hook(tap("merger_ln", "out"))
    vit.merger_fc1.register_forward_hook(tap("merger_fc1", "out"))
    vit.merger_fc2.register_forward_hook(tap("merger_act", "in"))
    grids = torch.tensor(V.GRIDS)
    y = vit(V.pixels().half(), grids)
    out["out"] = y.float().numpy()
    cos, sin = vit._rot_pos_emb(grids, torch.device("cpu"))
    out["cos"], out["sin"] = cos.numpy(), sin.numpy()
    return out


# ----------------------------------------------------------------------------- FP8
def fp8_linear_fixture(FL):
    w, b, x = P.linear_case()
    W, B, X = w.half(), b.half(), x.half()
    out = {}
    for tag, rowwise in (("pt", False), ("rw", True)):
        lin = FL.FP8Linear(W, B, rowwise=rowwise)
        out[f"{tag}_wq"] = lin.wq.view(torch.uint8).numpy().copy()
        out[f"{tag}_wscale"] = lin.wscale.float().reshape(-1).numpy().copy()
        out[f"{tag}_out"] = lin(X).float().numpy()
        out[f"{tag}_out_bf16in"] = lin(X.bfloat16()).float().numpy()
        nb = FL.FP8Linear(W, None, rowwise=rowwise)
        out[f"{tag}_out_nobias"] = nb(X).float().numpy()
    rw = FL.FP8Linear(W, B, rowwise=True)
    xq, s = FL.quant_fp8(X)
    out["rw_xq"] = xq.view(torch.uint8).numpy().copy()
    out["rw_xscale"] = s.numpy().copy()
    out["rw_prequant"] = rw.forward_prequant(xq, s).float().numpy()
    xq_pt, sa_pt = FL._quant_fp8_pertensor(X.reshape(-1, P.K))
    out["pt_xq"] = xq_pt.view(torch.uint8).numpy().copy()
    out["pt_xscale"] = sa_pt.reshape(-1).numpy().copy()
    xq_b, sa_b = FL._quant_fp8_pertensor(X.bfloat16())
    out["pt_xq_bf16"] = xq_b.view(torch.uint8).numpy().copy()
    out["pt_xscale_bf16"] = sa_b.float().reshape(-1).numpy().copy()
    return out


def fp8_route_taps(model, tap):
    """Layer 0's MLP under an FP8 plan: the post-attention norm's output ((e4m3 rows,
    scale) when fused), gate_up's output (forward or forward_prequant), the SiLU-mul
    output (down's input) and down's output."""
    mlp = model.layers[0].mlp
    mlp.register_forward_hook(tap("mlp_in", "in"))
    mlp.down_proj.register_forward_hook(tap("act", "in"))
    mlp.down_proj.register_forward_hook(tap("mlp_out", "out"))
    gu = mlp.gate_up_proj
    if hasattr(gu, "forward_prequant"):
        inner = gu.forward_prequant

        def recorded(xq, scale):
            y = inner(xq, scale)
            tap.record("gate_up", y)
            return y
        gu.forward_prequant = recorded
    gu.register_forward_hook(tap("gate_up", "out"))


def fp8_route_fixture(M, KV, positions_fn, decode_positions, MP):
    out = {}
    for name, plan in P.PLANS.items():
        def prepare(model, plan=plan, name=name):
            MP.apply_mixed(model, dict(plan))
            if name == "fused":
                MP.fuse_norm_fp8(model)
            l0 = model.layers[0].mlp
            for op in ("gate_up_proj", "down_proj"):
                lin = getattr(l0, op)
                out[f"{name}_{op}_wscale"] = lin.wscale.float().reshape(-1).numpy().copy()
                out[f"{name}_{op}_rowwise"] = np.array(int(lin.rowwise))
        res = MRC.run(torch.float16, M, KV, positions_fn, decode_positions, prepare=prepare,
                      register_taps=fp8_route_taps)
        for k in ("prefill_logits", "decode_logits", "lengths", "rope_delta"):
            out[f"{name}_{k}"] = res[k]
        for k, v in res.items():
            if k.startswith("l0_"):
                out[f"{name}_{k}"] = v
    return out


def main():
    sys.dont_write_bytecode = True       # nothing is written under the reference tree
    sys.path.insert(0, REF)
    import omniserve.kernels.fp8_linear as FL
    import omniserve.kernels.fused_ops as FO
    import omniserve.kernels.mixed_precision as MP
    import omniserve.model.qwen2_llm as M
    from omniserve.cache.kv_prealloc import PreallocatedKVCache
    from omniserve.model.positions import mrope_position_ids
    from omniserve.models.qwen2_vl import Qwen2VLAdapter
    MRC._torch_fused_ops(FO)
    _torch_fp8_ops(FO, FL)
    torch._scaled_mm = _scaled_mm
    with torch.no_grad():
        vit = vit_fixture()
        fp8 = fp8_linear_fixture(FL)
    fp8.update(fp8_route_fixture(M, PreallocatedKVCache, mrope_position_ids,
                                 Qwen2VLAdapter.decode_positions, MP))
    np.savez_compressed(OUT_VIT, **vit)
    np.savez_compressed(OUT_FP8, **fp8)
    for path, data in ((OUT_VIT, vit), (OUT_FP8, fp8)):
        print(f"wrote {path}: " + ", ".join(f"{k}{list(v.shape)}" for k, v in data.items()))


if __name__ == "__main__":
    main()
