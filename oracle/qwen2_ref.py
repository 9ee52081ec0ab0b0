"""CPU oracle: an fp32 restatement of omniserve's Qwen2-VL text-decoder token loop.

TEST INFRASTRUCTURE ONLY.  Nothing under ``omniserver_amd/`` imports this
module; only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg use it, as the checker (and as the reported CPU baseline),
never as the path that is measured or shipped.

Every function cites the reference file:line it restates (paths relative to the
omniserve repository).  Tensors are CPU ``float32``.  ``f16=True`` rounds to
fp16 at exactly the points where the reference's GPU path stores fp16 (weights
are already fp16 values), so the GPU kernels can be compared tightly;
``f16=False`` is the plain fp32 restatement used as the CPU baseline.

How each part is pinned (checked in tests/test_oracle.py) is listed in the
module docstring of that test file; no part is "parity unpinned" except where
stated there.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np
import torch

E4M3 = torch.float8_e4m3fn


def r16(x: torch.Tensor, on: bool = True) -> torch.Tensor:
    """Round fp32 values to fp16 and back (the reference's fp16 storage)."""
    return x.to(torch.float16).to(torch.float32) if on else x


# --------------------------------------------------------------------------- config
@dataclass
class Qwen2Config:
    """omniserve/model/qwen2_llm.py:25-36."""
    hidden_size: int = 1536
    num_layers: int = 28
    num_heads: int = 12
    num_kv_heads: int = 2
    head_dim: int = 128
    intermediate_size: int = 8960
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    mrope_section: List[int] = field(default_factory=lambda: [16, 24, 24])


# --------------------------------------------------------------------------- norms
def rms_norm(x, w, eps, f16=True):
    """kernels/fused_ops.py:21-29: y = x * (1/sqrt(sum(x^2)/N + eps)) * w, fp32 math."""
    rstd = 1.0 / torch.sqrt((x * x).sum(-1, keepdim=True) / x.shape[-1] + eps)
    return r16(x * rstd * w, f16)


def add_rms_norm(x, residual, w, eps, f16=True):
    """kernels/fused_ops.py:43-57: r = round(res + x) is the new residual, y = norm(r)."""
    r = r16(residual + x, f16)
    return rms_norm(r, w, eps, f16), r


def add_rms_norm_fp8(x, residual, w, eps):
    """kernels/fused_ops.py:74-91: y32 = norm(r); s = max(amax/448, 1e-12); q = e4m3(y32/s).

    Returns (q as e4m3fn tensor, s [M,1], new residual).  fp16 residual rounding."""
    r = r16(residual + x)
    rstd = 1.0 / torch.sqrt((r * r).sum(-1, keepdim=True) / r.shape[-1] + eps)
    y = r * rstd * w
    s = torch.clamp(y.abs().amax(-1, keepdim=True) / 448.0, min=1e-12)
    return (y / s).to(E4M3), s, r


def silu_mul(gate_up, f16=True):
    """kernels/fused_ops.py:111-119: out = silu(g) * u in fp32 (g = first half)."""
    n = gate_up.shape[-1] // 2
    g, u = gate_up[..., :n], gate_up[..., n:]
    return r16(g * torch.sigmoid(g) * u, f16)


# --------------------------------------------------------------------------- rope
def inv_freq(cfg: Qwen2Config, f16_buffer: bool = True) -> torch.Tensor:
    """model/qwen2_llm.py:169: 1 / theta^(arange(0, hd, 2)/hd) computed in fp32 and
    registered as a buffer (:170).  The deployed model is ``Qwen2LLM(cfg).half()``
    (models/qwen2_vl.py:50), which casts that buffer to fp16 like every floating tensor of
    the module, so the frequencies the reference uses are the fp16 roundings
    (``f16_buffer``; False = the buffer of a module left in fp32)."""
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2).float() / cfg.head_dim))
    return r16(inv, f16_buffer)


def rope_cos_sin(position_ids: torch.Tensor, cfg: Qwen2Config, f16=True, f16_buffer=True):
    """model/qwen2_llm.py:172-177 (+ the fp16 cast at :181): freqs = pos.float() * inv in
    fp32 (the fp16 buffer promotes to fp32), cos / sin in fp32, cast to fp16.

    position_ids [3, B, L] int -> cos, sin [3, B, L, head_dim]."""
    freqs = position_ids[..., None].float() * inv_freq(cfg, f16_buffer)
    emb = torch.cat([freqs, freqs], dim=-1)
    return r16(emb.cos(), f16), r16(emb.sin(), f16)


def rope_table(max_pos: int, cfg: Qwen2Config, f16_buffer: bool = True):
    """cos/sin of p * inv_freq for p in [0, max_pos), fp16-rounded, [max_pos, hd/2]:
    the same values rope_cos_sin produces for any position id (first half of emb)."""
    freqs = torch.arange(max_pos)[:, None].float() * inv_freq(cfg, f16_buffer)
    return r16(freqs.cos()), r16(freqs.sin())


def rotate_half(x):
    """model/qwen2_llm.py:59-61."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_mrope(q, k, cos, sin, mrope_section, f16=True):
    """model/qwen2_llm.py:64-72: per doubled section i, axis i % 3; q*cos + rot(q)*sin.

    q [B, nh, L, hd], k [B, nkv, L, hd], cos/sin [3, B, L, hd].  With f16 each of the
    product, product and sum is rounded to fp16 (the reference runs it in fp16)."""
    sec = list(mrope_section) * 2
    cos = torch.cat([m[i % 3] for i, m in enumerate(cos.split(sec, dim=-1))], dim=-1).unsqueeze(1)
    sin = torch.cat([m[i % 3] for i, m in enumerate(sin.split(sec, dim=-1))], dim=-1).unsqueeze(1)

    def rot(x):
        return r16(r16(x * cos, f16) + r16(rotate_half(x) * sin, f16), f16)

    return rot(q), rot(k)


def mrope_position_ids(input_ids: Sequence[int], grids: Sequence[Sequence[int]],
                       image_token_id: int = 151655, vision_start_id: int = 151652,
                       merge: int = 2):
    """model/positions.py:17-58 for one sequence.  The number of images is the number of
    vision-start tokens directly followed by an image token (:27-30); image i is the run
    that starts at the first image token at or after the current token index (:35), whether
    or not a vision-start precedes it, and takes grids[i].  Text tokens get sequential
    positions on all three axes, starting at the previous piece's max + 1 (:39, :51); an
    image run of t*(h/merge)*(w/merge) tokens gets its grid (t, h, w) coordinates offset
    by the text before it and that start (:42-49).

    Returns (pos [3, L] int64, delta = max + 1 - L)."""
    ids = list(input_ids)
    L = len(ids)
    n_images = sum(1 for i in range(L - 1)
                   if ids[i] == vision_start_id and ids[i + 1] == image_token_id)
    pieces: List[np.ndarray] = []
    st = 0
    for img in range(n_images):
        t, h, w = grids[img]
        ed = ids.index(image_token_id, st)
        gh, gw = h // merge, w // merge
        text_len = ed - st
        start = int(pieces[-1].max()) + 1 if pieces else 0
        pieces.append(np.tile(np.arange(text_len) + start, (3, 1)))
        ti = np.repeat(np.arange(t), gh * gw)
        hi = np.tile(np.repeat(np.arange(gh), gw), t)
        wi = np.tile(np.arange(gw), t * gh)
        pieces.append(np.stack([ti, hi, wi]) + text_len + start)
        st = ed + t * gh * gw
    if st < L:
        start = int(pieces[-1].max()) + 1 if pieces else 0
        pieces.append(np.tile(np.arange(L - st) + start, (3, 1)))
    pos = np.concatenate(pieces, axis=1).astype(np.int64)
    return torch.from_numpy(pos), int(pos.max()) + 1 - L


# --------------------------------------------------------------------------- int4
def gptq_pack(codes: torch.Tensor) -> torch.Tensor:
    """AutoGPTQ qweight packing (the format marlin_linear.py:83-96 ingests):
    codes [K, N] in 0..15 -> int32 [K/8, N], k % 8 at bits 4*(k % 8)."""
    K, N = codes.shape
    c = codes.to(torch.int64).reshape(K // 8, 8, N)
    word = torch.zeros(K // 8, N, dtype=torch.int64)
    for e in range(8):
        word |= c[:, e, :] << (4 * e)
    word = torch.where(word >= 2**31, word - 2**32, word)
    return word.to(torch.int32)


def gptq_unpack(qweight: torch.Tensor) -> torch.Tensor:
    """Inverse of gptq_pack: int32 [K/8, N] -> codes [K, N] int64."""
    w = qweight.to(torch.int64) & 0xFFFFFFFF
    parts = [(w >> (4 * e)) & 0xF for e in range(8)]
    return torch.stack(parts, dim=1).reshape(-1, qweight.shape[1])


def gptq_dequant(qweight: torch.Tensor, scales: torch.Tensor, group: int = 128) -> torch.Tensor:
    """uint4b8 symmetric dequant used by the Marlin path (marlin_linear.py:34, 47-50, 93):
    W[k, n] = fp16((q[k, n] - 8) * s[k // group, n]).  Returns fp32 holding fp16 values, [K, N]."""
    q = gptq_unpack(qweight).float()
    s = scales.float().repeat_interleave(group, dim=0)
    return r16((q - 8.0) * s)


def rtn_int4(weight: torch.Tensor, group: int = 128):
    """Round-to-nearest int4 of an fp16 weight [N, K] as the reference's MarlinInt4Linear
    gets it (kernels/marlin_linear.py:65-80 -> vLLM 0.12 marlin_quantize -> quantize_weights
    for scalar type uint4b8, symmetric, group ``group`` along K; vLLM is not in this image,
    so this restates its published algorithm): on fp16 values, per group and column,
    s = max(|max w / 7|, |min w / -8|) (the type's largest / smallest unbiased code),
    q = clamp(round(w / s), -8, 7) + 8 (round half to even), dequantised fp16((q - 8) s).
    Returns (qweight [K/8, N] int32 AutoGPTQ packing, scales [K/group, N] fp16 values as
    fp32).  An all-zero group (s = 0) gets code 8."""
    N, K = weight.shape
    w = weight.t().to(torch.float16).reshape(K // group, group, N)
    mx = w.amax(1, keepdim=True)
    mn = w.amin(1, keepdim=True)
    s = torch.maximum((mx / 7.0).abs(), (mn / -8.0).abs())
    safe = torch.where(s == 0, torch.ones_like(s), s)
    codes = torch.clamp(torch.round(w / safe).to(torch.int32), -8, 7) + 8
    qweight = gptq_pack(codes.reshape(K, N))
    return qweight, s.reshape(K // group, N).float()


# --------------------------------------------------------------------------- fp8
def fp8_weight_rowwise(weight: torch.Tensor):
    """kernels/fp8_linear.py:83-86 on the fp16 weight of the reference's ``.half()``
    model: ``weight.abs().amax(1) / 448.0`` is an fp16 tensor op, so sw[n] =
    fp16(amax_k |W[n, :]| / 448) (stored as fp32); ``weight / wscale`` with the [N, 1]
    fp32 scale promotes to fp32, so Wq = e4m3(W / sw) rounds once.
    weight [N, K] (fp16 values) -> (wq e4m3 [N, K], sw [N] fp32)."""
    sw = r16(weight.abs().amax(1, keepdim=True) / 448.0)
    return (weight / sw).to(E4M3), sw.view(-1)


def fp8_weight_pertensor(weight: torch.Tensor):
    """kernels/fp8_linear.py:87-90 (FP8Linear's default form) on the fp16 weight:
    sw = fp16(amax |W| / 448); ``weight / wscale`` with the 0-dim scale stays fp16, so
    Wq = e4m3(fp16(W / sw)) (two roundings).  -> (wq e4m3 [N, K], sw 0-dim fp32)."""
    sw = r16(weight.abs().max() / 448.0)
    return r16(weight / sw).to(E4M3), sw


def quant_fp8(x: torch.Tensor):
    """kernels/fp8_linear.py:45-63: per-token s = amax/448 (no clamp), q = e4m3(x / s)."""
    s = x.abs().amax(-1, keepdim=True) / 448.0
    return (x / s).to(E4M3), s


def rbf16(x: torch.Tensor) -> torch.Tensor:
    """Round fp32 values to bf16 and back."""
    return x.to(torch.bfloat16).to(torch.float32)


def quant_fp8_pertensor(x: torch.Tensor, bf16: bool = False):
    """_quant_fp8_pertensor's eager branch (kernels/fp8_linear.py:40-41, the one that runs
    without vLLM) on an fp16 tensor (bf16=True: the bf16 silu_mul output): sa =
    dtype(amax / 448) and q = e4m3(dtype(x / sa)), every op in the input's dtype.
    -> (q e4m3 [M, K], sa 0-dim fp32)."""
    rd = rbf16 if bf16 else r16
    sa = rd(x.abs().max() / 448.0)
    return rd(x / sa).to(E4M3), sa


def fp8_linear_pertensor(xq, sa, wq, sw, bias=None):
    """FP8Linear.forward, per-tensor (kernels/fp8_linear.py:119-125): _scaled_mm with
    scalar scales and out_dtype fp16 = fp16((sum_k xq wq) * sa * sw) (fp32 accumulation,
    scaled in that order as torch's _scaled_mm does), then ``out + bias`` in fp16."""
    y = r16((xq.float() @ wq.float().t()) * sa * sw)
    return y if bias is None else r16(y + bias)


def fp8_linear(x, w, bf16_in: bool = False):
    """An FP8Linear's forward on fp16 (or bf16) activations x, for w = (wq, sw) of either
    form: per-tensor (0-dim sw, fp16 out) or row-wise (quant_fp8 per token, bf16 product
    cast to fp16).  Returns fp32 holding fp16 values."""
    wq, sw = w
    if sw.dim() == 0:
        xq, sa = quant_fp8_pertensor(x, bf16_in)
        return fp8_linear_pertensor(xq, sa, wq, sw)
    xq, sa = quant_fp8(x)
    return fp8_linear_rowwise(xq, sa, wq, sw)


def fp8_linear_prequant(xq, sa, wq, sw, bias=None):
    """FP8Linear.forward_prequant (kernels/fp8_linear.py:99-108): the bf16 product of
    _scaled_mm, plus bias.to(bf16) added in bf16.  Returns fp32 holding bf16 values."""
    y = rbf16((xq.float() @ wq.float().t()) * sa.view(-1, 1) * sw.view(1, -1))
    return y if bias is None else rbf16(y + rbf16(bias.float()))


def fp8_linear_rowwise(xq, sa, wq, sw, bias=None, out_f16=True):
    """kernels/fp8_linear.py:115-118: y = (xq . Wq^T) * sa * sw accumulated in fp32,
    emitted as bf16 by _scaled_mm and then cast to fp16 (two roundings)."""
    y = (xq.float() @ wq.float().t()) * sa.view(-1, 1) * sw.view(1, -1)
    y = y.to(torch.bfloat16).float()
    if out_f16:
        y = r16(y)
    if bias is not None:
        y = r16(y + bias)
    return y


# --------------------------------------------------------------------------- linears
def linear(x, w_t, bias=None, f16=True, bias_after_round=False):
    """y = x . W (W given as W^T [K, N] fp32 holding fp16 values), fp32 accumulate.

    fp16 nn.Linear (qwen2_llm.py:82-83) rounds once after the bias; the GPTQ path adds
    the bias after the fp16 GEMM output (marlin_linear.py:59-62)."""
    y = x @ w_t
    if bias is None:
        return r16(y, f16)
    if bias_after_round:
        return r16(r16(y, f16) + bias, f16)
    return r16(y + bias, f16)


# --------------------------------------------------------------------------- attention
def decode_attention(q, k_pool, v_pool, rows, kv_len, scale, f16=True, p16=False):
    """cache/kv_prealloc.py:272-290 semantics in the SDPA + repeat_interleave form of
    model/qwen2_llm.py:105-113: per token b and head h,
    softmax(scale * q[b,h] . K[rows[b], 0:kv_len[b], h // G]^T) . V[...] (fp32 softmax).

    ``p16`` places one more rounding where a flash kernel has it (the published
    FlashAttention-2 algorithm, which vLLM's flash_attn_varlen_func follows: the
    unnormalised probabilities exp(s - max) are cast to fp16 for the P.V product, their
    sum stays fp32); the block-wise running maximum of a real kernel is not modelled (the
    row's maximum is used), so this is one member of the family of roundings the
    reference's flash path can produce, not its bits.

    q [n, nh, hd]; k_pool/v_pool [P, max_len, nkv, hd]; returns [n, nh, hd]."""
    n, nh, hd = q.shape
    nkv = k_pool.shape[2]
    rep = nh // nkv
    out = torch.empty(n, nh, hd)
    for b in range(n):
        L = int(kv_len[b])
        k = k_pool[int(rows[b]), :L].transpose(0, 1).repeat_interleave(rep, 0)  # [nh, L, hd]
        v = v_pool[int(rows[b]), :L].transpose(0, 1).repeat_interleave(rep, 0)
        s = torch.einsum("hd,hld->hl", q[b], k) * scale
        if p16:
            e = torch.exp(s - s.max(-1, keepdim=True).values)
            out[b] = torch.einsum("hl,hld->hd", r16(e), v) / e.sum(-1, keepdim=True)
        else:
            p = torch.softmax(s, dim=-1)
            out[b] = torch.einsum("hl,hld->hd", p, v)
    return r16(out, f16)


def prefill_attention(q, k, v, seg_lens, scale, f16=True, p16=False):
    """cache/kv_prealloc.py:181-203: causal attention inside each packed segment.
    q [T, nh, hd], k/v [T, nkv, hd] -> [T, nh, hd].  ``p16``: the probabilities rounded to
    fp16 for the P.V product as a flash kernel rounds them (see decode_attention)."""
    T, nh, hd = q.shape
    rep = nh // k.shape[1]
    out = torch.empty(T, nh, hd)
    off = 0
    for L in seg_lens:
        qs = q[off:off + L].transpose(0, 1)                       # [nh, L, hd]
        ks = k[off:off + L].transpose(0, 1).repeat_interleave(rep, 0)
        vs = v[off:off + L].transpose(0, 1).repeat_interleave(rep, 0)
        s = torch.einsum("hid,hjd->hij", qs, ks) * scale
        mask = torch.ones(L, L, dtype=torch.bool).tril()
        s = s.masked_fill(~mask, float("-inf"))
        if p16:
            e = torch.exp(s - s.max(-1, keepdim=True).values)
            o = torch.einsum("hij,hjd->hid", r16(e), vs) / e.sum(-1, keepdim=True)
        else:
            o = torch.einsum("hij,hjd->hid", torch.softmax(s, dim=-1), vs)
        out[off:off + L] = o.transpose(0, 1)
        off += L
    return r16(out, f16)


# --------------------------------------------------------------------------- model
@dataclass
class LayerWeights:
    """One decoder layer in the reference's fused layout (qwen2_llm.py:193-219):
    qkv = q|k|v along the output dim (+ bias), gate_up = gate|up.  Linear weights are
    held transposed ([K, N]) as fp32 holding fp16 (or dequantised int4) values."""
    in_norm: torch.Tensor
    post_norm: torch.Tensor
    qkv_t: torch.Tensor
    qkv_b: torch.Tensor
    o_t: torch.Tensor
    gate_up_t: torch.Tensor
    down_t: torch.Tensor
    # the FP8 MLP route (kernels/mixed_precision.py apply_mixed / fuse_norm_fp8):
    # (Wq e4m3 [N, K], sw) of an FP8 gate_up / down - sw [N] row-wise, 0-dim per-tensor
    # (FP8Linear's default, what apply_mixed builds) - or None for fp16
    fp8_gate_up: Optional[tuple] = None
    fp8_down: Optional[tuple] = None
    # fuse_norm_fp8 (mixed_precision.py:53-75): the post-attention norm emits e4m3 rows
    # for the FP8 gate_up's forward_prequant; False = FP8Linear.forward quantises itself
    norm_fp8: bool = False


class Qwen2Ref:
    """The decode step and packed prefill of model/qwen2_llm.py:179-190 + DecoderLayer
    (:145-157) + Attention (:86-113) + MLP (:123-134), with the KV-pool semantics of
    cache/kv_prealloc.py (write rotated K / raw V first, then attend over [0, pos]) and the
    greedy emit of runners/multimodal.py:306-310."""

    def __init__(self, cfg: Qwen2Config, embed: torch.Tensor, final_norm: torch.Tensor,
                 layers: List[LayerWeights], gptq_bias_after_round: bool = False,
                 f16: bool = True, attn_p16: bool = False):
        self.cfg = cfg
        self.embed = embed          # [V, H] (tied lm_head, qwen2_llm.py:167-168)
        self.final_norm = final_norm
        self.layers = layers
        self.bias_after_round = gptq_bias_after_round
        self.f16 = f16
        # attention with the flash kernel's fp16 probabilities (decode_attention p16)
        self.attn_p16 = attn_p16

    # -- pieces
    def _attn_in(self, x, lw: LayerWeights, pos3):
        """qkv projection + split + M-RoPE (qwen2_llm.py:86-93).  x [T, H], pos3 [3, T]."""
        c = self.cfg
        qkv = linear(x, lw.qkv_t, lw.qkv_b, self.f16, self.bias_after_round)
        T = x.shape[0]
        q = qkv[:, :c.num_heads * c.head_dim].reshape(T, c.num_heads, c.head_dim)
        k = qkv[:, c.num_heads * c.head_dim:(c.num_heads + c.num_kv_heads) * c.head_dim]
        k = k.reshape(T, c.num_kv_heads, c.head_dim)
        v = qkv[:, (c.num_heads + c.num_kv_heads) * c.head_dim:].reshape(T, c.num_kv_heads,
                                                                            c.head_dim)
        cos, sin = rope_cos_sin(pos3.view(3, 1, T), c, self.f16)
        qr, kr = apply_mrope(q.transpose(0, 1).unsqueeze(0), k.transpose(0, 1).unsqueeze(0),
                             cos, sin, c.mrope_section, self.f16)
        return qr[0].transpose(0, 1), kr[0].transpose(0, 1), v

    def _mlp(self, x, lw: LayerWeights):
        gu = linear(x, lw.gate_up_t, None, self.f16)
        return linear(silu_mul(gu, self.f16), lw.down_t, None, self.f16)

    def _post_norm_mlp(self, o, residual, lw: LayerWeights):
        """post_attention_layernorm + MLP (qwen2_llm.py:153-154, 123-134) with either linear
        of the MLP optionally FP8 (FP8Linear, fp8_linear.py:66-126, per-tensor or row-wise):
        * fused norm (norm_fp8, fuse_norm_fp8, which makes gate_up row-wise):
          add_rms_norm_fp8 quantises the normed rows (fused_ops.py:74-91),
          gate_up.forward_prequant returns the bf16 product (:99-108), silu_mul keeps bf16
          (fused_ops.py:122-130 stores in its input dtype);
        * otherwise the fp16 norm output goes to gate_up's forward (fp8_linear);
        the down projection takes the activation as it comes: an FP8 one quantises it (bf16
        or fp16, qwen2_llm.py:132-134), an fp16 one gets it cast to fp16 (:132-133)."""
        c = self.cfg
        bf16_act = False
        if lw.fp8_gate_up is not None and lw.norm_fp8:
            if lw.fp8_gate_up[1].dim() == 0:
                raise ValueError("the fused norm feeds a row-wise FP8 gate_up only "
                                 "(mixed_precision.py:69-70)")
            xq, sa, residual = add_rms_norm_fp8(o, residual, lw.post_norm, c.rms_norm_eps)
            gu = fp8_linear_prequant(xq, sa, *lw.fp8_gate_up)
            n = gu.shape[-1] // 2
            g, u = gu[..., :n], gu[..., n:]
            act = rbf16(g * torch.sigmoid(g) * u)
            bf16_act = True
        else:
            h, residual = add_rms_norm(o, residual, lw.post_norm, c.rms_norm_eps, self.f16)
            if lw.fp8_gate_up is None:
                if lw.fp8_down is None:
                    return self._mlp(h, lw), residual
                gu = linear(h, lw.gate_up_t, None, self.f16)
            else:
                gu = fp8_linear(h, lw.fp8_gate_up)
            act = silu_mul(gu, self.f16)
        if lw.fp8_down is None:
            return linear(r16(act), lw.down_t, None, self.f16), residual
        return fp8_linear(act, lw.fp8_down, bf16_act), residual

    def lm_head(self, h):
        return r16(h @ self.embed.t(), self.f16)

    # -- decode step
    def decode_step(self, ids, k_pool: List[torch.Tensor], v_pool: List[torch.Tensor],
                    lengths: torch.Tensor, rope_delta: Optional[torch.Tensor] = None,
                    return_hidden: bool = False):
        """One decode step for sequences in pool rows 0..n-1 (runners/multimodal.py:296-313).

        Writes the new K/V at position lengths[b] of each row, attends over
        [0, lengths[b]] and returns fp16-valued logits [n, V].  Does not advance lengths."""
        c = self.cfg
        n = len(ids)
        x = self.embed[torch.as_tensor(ids, dtype=torch.long)]
        wpos = lengths[:n].clone()
        d = rope_delta[:n] if rope_delta is not None else torch.zeros(n, dtype=torch.long)
        pos3 = (wpos + d).view(1, n).expand(3, n)
        residual = None
        scale = c.head_dim ** -0.5
        for i, lw in enumerate(self.layers):
            if residual is None:
                residual = x
                h = rms_norm(x, lw.in_norm, c.rms_norm_eps, self.f16)
            else:
                h, residual = add_rms_norm(x, residual, lw.in_norm, c.rms_norm_eps, self.f16)
            q, k, v = self._attn_in(h, lw, pos3)
            for b in range(n):
                k_pool[i][b, int(wpos[b])] = k[b]
                v_pool[i][b, int(wpos[b])] = v[b]
            a = decode_attention(q, k_pool[i], v_pool[i], torch.arange(n), wpos + 1, scale,
                                 self.f16, self.attn_p16)
            o = linear(a.reshape(n, -1), lw.o_t, None, self.f16)
            x, residual = self._post_norm_mlp(o, residual, lw)
        h, _ = add_rms_norm(x, residual, self.final_norm, c.rms_norm_eps, self.f16)
        logits = self.lm_head(h)
        return (logits, h) if return_hidden else logits

    # -- packed prefill
    def prefill(self, embeds: torch.Tensor, pos3: torch.Tensor, seg_lens: Sequence[int],
                slots: Sequence[int], k_pool, v_pool, lengths: torch.Tensor):
        """Packed prefill (runners/multimodal.py:116-144, cache/kv_prealloc.py:181-203):
        embeds [T, H] fp16 values, pos3 [3, T].  Writes each segment's K/V into
        pool[slot, :L], sets lengths[slot] = L and returns logits at segment ends."""
        c = self.cfg
        scale = c.head_dim ** -0.5
        x = embeds
        residual = None
        for i, lw in enumerate(self.layers):
            if residual is None:
                residual = x
                h = rms_norm(x, lw.in_norm, c.rms_norm_eps, self.f16)
            else:
                h, residual = add_rms_norm(x, residual, lw.in_norm, c.rms_norm_eps, self.f16)
            q, k, v = self._attn_in(h, lw, pos3)
            off = 0
            for slot, L in zip(slots, seg_lens):
                k_pool[i][slot, :L] = k[off:off + L]
                v_pool[i][slot, :L] = v[off:off + L]
                off += L
            a = prefill_attention(q, k, v, seg_lens, scale, self.f16, self.attn_p16)
            o = linear(a.reshape(a.shape[0], -1), lw.o_t, None, self.f16)
            x, residual = self._post_norm_mlp(o, residual, lw)
        last = torch.tensor(np.cumsum(seg_lens) - 1)
        h, _ = add_rms_norm(x[last], residual[last], self.final_norm, c.rms_norm_eps, self.f16)
        for slot, L in zip(slots, seg_lens):
            lengths[slot] = L
        return self.lm_head(h)


def greedy(logits: torch.Tensor) -> List[int]:
    """runners/multimodal.py:307-308: argmax over the (fp16-valued) logits, first index of
    the maximum (torch.argmax semantics)."""
    return logits.argmax(dim=-1).tolist()


def top2_margin(logits: torch.Tensor) -> torch.Tensor:
    """Gap between the largest and second-largest logit per row (near-tie diagnostics)."""
    t = logits.topk(2, dim=-1).values
    return t[..., 0] - t[..., 1]
