"""Writes tests/golden/ref_composition.npz: outputs of the reference's own decoder forward
on the seeded case of composition_case.py, in this container's CPU PyTorch.

What runs is omniserve's code from /root/reference, imported here (never shipped, never
run on a GPU box):
  * model/qwen2_llm.py  Qwen2LLM.forward, DecoderLayer.forward, Attention.forward (the
    cache.update + SDPA branch, :105-113), MLP.forward, apply_mrope, rope, load_from_hf;
  * cache/kv_prealloc.py  PreallocatedKVCache.prefill_cache (_PrefillWriter.update) for
    each prompt and view() (_CacheView.update) for the decode steps;
  * model/positions.py  mrope_position_ids; models/qwen2_vl.py decode_positions.
The model is built the way models/qwen2_vl.py:50 builds it (``Qwen2LLM(cfg).half()``,
then the checkpoint copied in); the reference runs only in fp16 (MLP.forward casts the
SiLU output to fp16 before down_proj, qwen2_llm.py:132-133).
Only kernels/fused_ops.py's Triton kernels, which cannot run on CPU tensors, are replaced,
by torch evaluations of the same per-row formulas (fp32 math, result stored in the input
dtype, the new residual rounded to its dtype before the norm).  The decode view is wrapped
so that only ``update`` is visible: the vLLM flash branch needs vLLM and a GPU.

Run: python tests/golden/make_ref_composition.py   (needs /root/reference)
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import composition_case as C  # noqa: E402

REF = "/root/reference"
OUT = os.path.join(HERE, "ref_composition.npz")


def _torch_fused_ops(FO):
    def rms_norm(x, weight, eps):
        xf = x.float()
        rstd = 1.0 / torch.sqrt((xf * xf).sum(-1, keepdim=True) / x.shape[-1] + eps)
        return (xf * rstd * weight.float()).to(x.dtype)

    def add_rms_norm(x, residual, weight, eps):
        r = (residual.float() + x.float()).to(residual.dtype)
        return rms_norm(r, weight, eps).to(x.dtype), r

    def silu_mul(gate_up):
        n = gate_up.shape[-1] // 2
        g, u = gate_up[..., :n].float(), gate_up[..., n:].float()
        return ((g * torch.sigmoid(g)) * u).to(gate_up.dtype)

    FO.rms_norm, FO.add_rms_norm, FO.silu_mul = rms_norm, add_rms_norm, silu_mul


def _tap_value(t):
    """A tapped tensor as a 2-D numpy array: float32 values (e4m3 codes as their float
    values); an (e4m3 rows, scale) tuple as the codes' values followed by the scale column."""
    if isinstance(t, tuple):
        q, s = t
        return np.concatenate([_tap_value(q), _tap_value(s)], axis=1)
    return t.reshape(-1, t.shape[-1]).float().numpy().copy()


class _UpdateOnly:
    """The decode view with only the transformers-cache ``update`` visible."""

    def __init__(self, view):
        self._v = view

    def update(self, k, v, layer_idx, cache_kwargs=None):
        return self._v.update(k, v, layer_idx)


def _hf_state_dict(w):
    """The case's fused weights split back into Hugging Face key names (load_from_hf
    concatenates them again in its own order)."""
    q, kv = C.HEADS * C.HEAD_DIM, C.KV_HEADS * C.HEAD_DIM
    sd = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["norm"]}
    for i, l in enumerate(w["layers"]):
        p = f"model.layers.{i}."
        qw, kw, vw = l["qkv_w"].split([q, kv, kv], 0)
        qb, kb, vb = l["qkv_b"].split([q, kv, kv], 0)
        gw, uw = l["gate_up_w"].split([C.INTER, C.INTER], 0)
        sd.update({p + "self_attn.q_proj.weight": qw, p + "self_attn.k_proj.weight": kw,
                   p + "self_attn.v_proj.weight": vw, p + "self_attn.q_proj.bias": qb,
                   p + "self_attn.k_proj.bias": kb, p + "self_attn.v_proj.bias": vb,
                   p + "self_attn.o_proj.weight": l["o_w"], p + "mlp.gate_proj.weight": gw,
                   p + "mlp.up_proj.weight": uw, p + "mlp.down_proj.weight": l["down_w"],
                   p + "input_layernorm.weight": l["in_norm"],
                   p + "post_attention_layernorm.weight": l["post_norm"]})
    return sd


def default_taps(model, tap):
    """Layer 0's o_proj input (attention output) and output, MLP input / output and
    down_proj input (SiLU-mul output)."""
    lay0 = model.layers[0]
    lay0.self_attn.o_proj.register_forward_hook(tap("attn", "in"))
    lay0.self_attn.o_proj.register_forward_hook(tap("o", "out"))
    lay0.mlp.register_forward_hook(tap("mlp_in", "in"))
    lay0.mlp.register_forward_hook(tap("mlp_out", "out"))
    lay0.mlp.down_proj.register_forward_hook(tap("act", "in"))


def run(dtype, M, KV, positions_fn, decode_positions, prepare=None, register_taps=default_taps):
    """The case's prompts and decode steps through the reference's forward.  ``prepare``
    (if given) rewrites the loaded fp16 model before it runs (e.g. an FP8 plan);
    ``register_taps(model, tap)`` installs the forward hooks whose values are kept for the
    first prompt's prefill and the first decode step."""
    cfg = M.Qwen2Config(hidden_size=C.HIDDEN, num_layers=C.LAYERS, num_heads=C.HEADS,
                        num_kv_heads=C.KV_HEADS, head_dim=C.HEAD_DIM,
                        intermediate_size=C.INTER, vocab_size=C.VOCAB, rms_norm_eps=C.EPS,
                        rope_theta=C.THETA, mrope_section=list(C.SECTIONS))
    model = M.Qwen2LLM(cfg).half()               # models/qwen2_vl.py:50
    M.load_from_hf(model, _hf_state_dict(C.weights()))
    if prepare is not None:
        prepare(model)
    model.eval()
    pool = KV(C.LAYERS, 3, C.KV_HEADS, C.MAX_LEN, C.HEAD_DIM, "cpu", dtype)
    out = {}
    # layer 0's intermediate values (first prompt's prefill, first decode step): the input
    # of o_proj (attention output), its output, the MLP's input and output
    taps, tap_on = {}, {"tag": None}

    def tap(name, which):
        def hook(mod, inp, res):
            if tap_on["tag"] is not None:
                t = inp[0] if which == "in" else res
                taps[f"{tap_on['tag']}_{name}"] = _tap_value(t)
        return hook

    tap.record = lambda name, t: (taps.__setitem__(f"{tap_on['tag']}_{name}", _tap_value(t))
                                  if tap_on["tag"] is not None else None)
    register_taps(model, tap)
    prefill, deltas = [], []
    with torch.no_grad():
        for slot, (ids, img, grids) in enumerate(C.prompts()):
            L = len(ids)
            ids_t = torch.tensor([ids])
            emb = model.embed_tokens(ids_t)
            if img is not None:
                emb[0, ids_t[0] == C.CASE_IMAGE_ID] = img.to(dtype)
            if grids:
                pos, d = positions_fn(ids_t, torch.tensor(grids), image_token_id=C.CASE_IMAGE_ID,
                                      vision_start_token_id=C.CASE_VSTART_ID)
                d = int(d.flatten()[0])
            else:
                pos, d = torch.arange(L).view(1, 1, -1).expand(3, 1, -1), 0
            mask = torch.ones(L, L, dtype=torch.bool).tril()
            tap_on["tag"] = "l0_prefill" if slot == 0 else None
            lg = model(emb, pos, mask, pool.prefill_cache(slot), logits_indices=[L - 1])
            prefill.append(lg[0, -1].float().numpy())
            deltas.append(d)
        out["prefill_logits"] = np.stack(prefill)
        rope = torch.tensor(deltas)
        dec = []
        for step, step_ids in enumerate(C.decode_ids()):
            tap_on["tag"] = "l0_decode" if step == 0 else None
            view = pool.view(2)
            ids = torch.tensor(step_ids).view(2, 1)
            pos = decode_positions(None, view.write_pos, rope)
            kv_len = view.ret_len
            mask = (torch.arange(kv_len).view(1, -1) <= view.write_pos.view(-1, 1))
            lg = model(model.embed_tokens(ids), pos, mask.view(2, 1, 1, kv_len),
                       _UpdateOnly(view))[:, -1, :]
            dec.append(lg.float().numpy())
        out["decode_logits"] = np.stack(dec)
    out["lengths"] = pool.lengths[:2].numpy().copy()
    out["rope_delta"] = np.array(deltas, dtype=np.int64)
    out["k_pool"] = np.stack([pool.k[l][:2].float().numpy() for l in range(C.LAYERS)])
    out["v_pool"] = np.stack([pool.v[l][:2].float().numpy() for l in range(C.LAYERS)])
    out["inv_freq"] = model.inv_freq.float().numpy()
    out.update(taps)
    return out


def main():
    sys.dont_write_bytecode = True       # nothing is written under the reference tree
    sys.path.insert(0, REF)
    import omniserve.kernels.fused_ops as FO
    import omniserve.model.qwen2_llm as M
    from omniserve.cache.kv_prealloc import PreallocatedKVCache
    from omniserve.model.positions import mrope_position_ids
    from omniserve.models.qwen2_vl import Qwen2VLAdapter
    _torch_fused_ops(FO)
    data = {}
    for k, v in run(torch.float16, M, PreallocatedKVCache, mrope_position_ids,
                    Qwen2VLAdapter.decode_positions).items():
        data[k] = v.astype(np.float16) if k.endswith("pool") else v
    for i, (ids, grids) in enumerate(C.position_cases()):
        pos, d = mrope_position_ids(torch.tensor([ids]), torch.tensor(grids))
        data[f"pos{i}"] = pos[:, 0].numpy()
        data[f"pos{i}_delta"] = np.array(int(d.flatten()[0]))
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT}: " + ", ".join(f"{k}{list(v.shape)}" for k, v in data.items()))


if __name__ == "__main__":
    main()
