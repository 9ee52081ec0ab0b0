"""Qwen2 text decoder (Qwen2-VL-2B shape) driven by the gfx950 HIP kernels.

Host mirror of omniserve/model/qwen2_llm.py: same config, same fused weight
layouts (q|k|v with bias, gate|up), same residual threading (the add folded into
the next RMSNorm, :145-157, final norm = add + norm, :186), M-RoPE with sections
[16, 24, 24] (:59-72), tied lm_head (:167-168).

Two entry points:
* ``forward(inputs_embeds, position_ids, attn_mask, cache, logits_indices)`` - the
  reference signature (:179-190), used for packed prefill (cache =
  ``PackedPrefillWriter``) and eager decode (cache = ``CacheView``); returns logits.
* ``decode_greedy(...)`` - the decode step on static buffers, ending in the fused
  lm_head + argmax; allocation-free and host-sync-free, so the runner captures it
  whole in a HIP graph.
"""

from __future__ import annotations

from typing import Dict, List, Optional

import torch
from torch import nn

from . import fused_ops as F
from .hostio import to_device
from .linear import F16Linear, GPTQLinear, LMHeadArgmax, _Skinny
from .synth import DecoderShape

Qwen2Config = DecoderShape


def _indices_on(indices, device) -> torch.Tensor:
    """logits_indices as an int64 tensor on device: a tensor already there is used as is (no
    host transfer, so a forward given one can be captured in a graph)."""
    if isinstance(indices, torch.Tensor) and indices.device == torch.device(device) \
            and indices.dtype == torch.long:
        return indices
    return to_device(indices, torch.long, device)


def rope_tables(cfg: Qwen2Config, max_pos: int, device):
    """fp16 cos/sin [max_pos, head_dim/2] of p * inv_freq (qwen2_llm.py:169-177, 181):
    inv_freq = 1/theta^(arange(0,hd,2)/hd) in fp32, held in fp16 as the deployed module
    holds its buffer (``Qwen2LLM(cfg).half()``, models/qwen2_vl.py:50, casts it), then
    p*inv_freq in fp32, cos/sin in fp32, cast to fp16.  Built on the CPU once; the kernel
    reads the pair (d, d+64) from column d."""
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2).float() / cfg.head_dim))
    inv = inv.to(torch.float16).float()
    freqs = torch.arange(max_pos)[:, None].float() * inv
    return (freqs.cos().to(torch.float16).to(device).contiguous(),
            freqs.sin().to(torch.float16).to(device).contiguous())


class RMSNorm(nn.Module):
    """model/qwen2_llm.py:40-56: rms_norm without a residual, add_rms_norm with one, and -
    with ``fp8_out`` set (kernels/mixed_precision.py fuse_norm_fp8) - add_rms_norm_fp8,
    returning ((e4m3 rows, per-row scale), new residual) for an FP8 gate_up."""

    def __init__(self, weight: torch.Tensor, eps: float):
        super().__init__()
        self.register_buffer("weight", weight)
        self.eps = eps
        self.fp8_out = False

    def forward(self, x, residual=None):
        if self.fp8_out and residual is not None:
            fq, scale, nres = F.add_rms_norm_fp8(x, residual, self.weight, self.eps)
            return (fq, scale), nres
        if residual is None:
            return F.rms_norm(x, self.weight, self.eps)
        return F.add_rms_norm(x, residual, self.weight, self.eps)


class Attention(nn.Module):
    """The projections of model/qwen2_llm.py:75-84 (attention itself runs in the cache
    adapters): ``qkv_proj`` q|k|v with bias, ``o_proj``; any module with forward(x fp16)
    may be installed on them (kernels/mixed_precision.py:21-50)."""

    def __init__(self, qkv_proj: nn.Module, o_proj: nn.Module):
        super().__init__()
        self.qkv_proj = qkv_proj
        self.o_proj = o_proj


class MLP(nn.Module):
    """model/qwen2_llm.py:115-134.  gate_up -> silu_mul -> down, where
    * a gate_up module built with the SiLU epilogue (``fuse_silu``) already emits
      silu(gate) * up;
    * an (e4m3 rows, scale) input from an fp8_out norm goes to gate_up.forward_prequant,
      whose bf16 product silu_mul keeps in bf16;
    * a non-fp16 activation reaches down_proj as is when down_proj can quantise it itself
      (it has forward_prequant), else cast to fp16."""

    def __init__(self, gate_up_proj: nn.Module, down_proj: nn.Module):
        super().__init__()
        self.gate_up_proj = gate_up_proj
        self.down_proj = down_proj

    def forward(self, x):
        if isinstance(x, tuple):
            xq, scale = x
            gu = self.gate_up_proj.forward_prequant(xq, scale)
        else:
            gu = self.gate_up_proj(x)
        out = gu if getattr(self.gate_up_proj, "fuse_silu", False) else F.silu_mul(gu)
        if out.dtype != torch.float16 and not hasattr(self.down_proj, "forward_prequant"):
            out = out.to(torch.float16)
        return self.down_proj(out)


class DecoderLayer(nn.Module):
    """model/qwen2_llm.py:137-157: input_layernorm, self_attn, post_attention_layernorm,
    mlp (the reference's module names, so linears can be replaced by setattr).  The fused
    decode step reads the same modules through the short aliases below."""

    def __init__(self, in_norm, post_norm, qkv_proj, o_proj, gate_up_proj, down_proj,
                 eps: float = 1e-6):
        super().__init__()
        self.input_layernorm = RMSNorm(in_norm, eps)
        self.self_attn = Attention(qkv_proj, o_proj)
        self.post_attention_layernorm = RMSNorm(post_norm, eps)
        self.mlp = MLP(gate_up_proj, down_proj)

    in_norm = property(lambda self: self.input_layernorm.weight)
    post_norm = property(lambda self: self.post_attention_layernorm.weight)
    qkv_proj = property(lambda self: self.self_attn.qkv_proj)
    o_proj = property(lambda self: self.self_attn.o_proj)
    gate_up_proj = property(lambda self: self.mlp.gate_up_proj)
    down_proj = property(lambda self: self.mlp.down_proj)

    def fused_decode_ready(self) -> bool:
        """The fused decode step needs this library's packed linears (split-K partial
        outputs, the attention-merging o_proj, the SiLU-fused gate_up) and plain norms."""
        lin = (self.qkv_proj, self.o_proj, self.down_proj)
        return (all(isinstance(m, _Skinny) and not m.fuse_silu for m in lin)
                and isinstance(self.gate_up_proj, _Skinny) and self.gate_up_proj.fuse_silu
                and not self.post_attention_layernorm.fp8_out)


class Qwen2LLM(nn.Module):
    def __init__(self, cfg: Qwen2Config, embed: torch.Tensor, final_norm: torch.Tensor,
                 layers: List[DecoderLayer], max_pos: int = 8192):
        super().__init__()
        self.cfg = cfg
        self.lm_head = LMHeadArgmax(embed)         # packed tied table (also the embedding)
        self.register_buffer("norm", final_norm)
        self.layers = nn.ModuleList(layers)
        cos, sin = rope_tables(cfg, max_pos, embed.device)
        self.register_buffer("rope_cos", cos)
        self.register_buffer("rope_sin", sin)
        self.scale = cfg.head_dim ** -0.5
        self._bufs: Dict[int, dict] = {}
        # prefill hands split-K partial sums to the next kernel where prefill_partials_ok
        self.prefill_partials = True

    # ------------------------------------------------------------------ builders
    @classmethod
    def from_fp16(cls, w: Dict, cfg: Qwen2Config, device, max_pos: int = 8192) -> "Qwen2LLM":
        """fp16 weights in nn.Linear layout (see synth.fp16_decoder)."""
        d = torch.device(device)
        layers = []
        for lw in w["layers"]:
            layers.append(DecoderLayer(
                lw["in_norm"].to(d), lw["post_norm"].to(d),
                F16Linear(lw["qkv_w"].to(d), lw["qkv_b"].to(d)),
                F16Linear(lw["o_w"].to(d)),
                F16Linear(lw["gate_up_w"].to(d), fuse_silu=True),
                F16Linear(lw["down_w"].to(d)), cfg.rms_norm_eps))
        return cls(cfg, w["embed"].to(d), w["norm"].to(d), layers, max_pos)

    @classmethod
    def from_gptq(cls, w: Dict, cfg: Qwen2Config, device, max_pos: int = 8192) -> "Qwen2LLM":
        """GPTQ int4 decoder linears (AutoGPTQ layout, see synth.gptq_decoder), fp16
        embedding / lm_head and norms (marlin_linear.py:114-143)."""
        d = torch.device(device)
        layers = []
        for lw in w["layers"]:
            layers.append(DecoderLayer(
                lw["in_norm"].to(d), lw["post_norm"].to(d),
                GPTQLinear(lw["qkv_q"].to(d), lw["qkv_s"].to(d), lw["qkv_b"].to(d)),
                GPTQLinear(lw["o_q"].to(d), lw["o_s"].to(d)),
                GPTQLinear(lw["gate_up_q"].to(d), lw["gate_up_s"].to(d), fuse_silu=True),
                GPTQLinear(lw["down_q"].to(d), lw["down_s"].to(d)), cfg.rms_norm_eps))
        return cls(cfg, w["embed"].to(d), w["norm"].to(d), layers, max_pos)

    def fused_decode_ready(self) -> bool:
        """Whether decode_greedy can run this model (every layer on the packed linears);
        otherwise decoding goes through forward()."""
        return all(layer.fused_decode_ready() for layer in self.layers)

    # ------------------------------------------------------------------ embedding
    def embed_tokens(self, ids: torch.Tensor) -> torch.Tensor:
        """ids [...] int64 -> [..., H] fp16 (models/qwen2_vl.py:93-94), gathered from the
        packed tied table."""
        ids_c = ids.reshape(-1).contiguous()
        out = torch.empty(ids_c.numel(), self.cfg.hidden_size, device=ids.device,
                          dtype=torch.float16)
        F.embedding_out(ids_c, self.lm_head.table_packed, True, out)
        return out.reshape(*ids.shape, self.cfg.hidden_size)

    # ------------------------------------------------------------------ reference forward
    def forward(self, inputs_embeds, position_ids, attn_mask=None, cache=None,
                logits_indices=None):
        """inputs_embeds [B, L, H] fp16 with B*L packed tokens; position_ids [3, B, L].

        ``cache`` must be a pool adapter (PackedPrefillWriter for packed / chunked / mixed
        prefill, CacheView for decode); attn_mask is unused (causality / lengths come from
        the adapter)."""
        cfg = self.cfg
        B, L, H = inputs_embeds.shape
        T = B * L
        x = inputs_embeds.reshape(T, H).contiguous()
        if hasattr(cache, "bind"):              # prefill / append adapters: T tokens
            cache.bind(T)
        decode = not hasattr(cache, "token_slot")
        pos = None if decode else position_ids.reshape(3, T).to(torch.int64).contiguous()
        if not decode and self.prefill_partials_ok(T):
            return self._forward_partials(x, pos, cache, logits_indices, B)
        if not decode and self.prefill_down_partials_ok(T):
            return self._forward_partials(x, pos, cache, logits_indices, B, down_only=True)
        residual = None
        for i, layer in enumerate(self.layers):
            if residual is None:
                residual = x
                h = layer.input_layernorm(x)
            else:
                h, residual = layer.input_layernorm(x, residual)
            qkv = layer.self_attn.qkv_proj(h)
            if decode:
                cache.rope_and_write(qkv, i, self.rope_cos, self.rope_sin, cfg.mrope_section)
            else:
                cache.rope_and_write(qkv, i, pos, self.rope_cos, self.rope_sin,
                                     cfg.mrope_section)
            attn = torch.empty(T, cfg.num_heads, cfg.head_dim, device=x.device,
                               dtype=torch.float16)
            cache.attend_qkv(qkv, i, self.scale, attn)
            o = layer.self_attn.o_proj(attn.reshape(T, -1))
            h, residual = layer.post_attention_layernorm(o, residual)
            x = layer.mlp(h)
        cache.finish()
        if logits_indices is not None:
            idx = _indices_on(logits_indices, x.device)
            x, residual = x[idx].contiguous(), residual[idx].contiguous()
        h, _ = F.add_rms_norm(x, residual, self.norm, cfg.rms_norm_eps)
        logits = self.lm_head.logits(h)
        return logits.reshape(1 if logits_indices is not None else B, -1, cfg.vocab_size)

    def prefill_partials_ok(self, T: int) -> bool:
        """Whether forward runs a T-token prefill with qkv / o / down writing split-K
        partial sums that the next kernel adds (the M-RoPE + KV write, the add+RMSNorms)
        instead of finishing each projection in a launch of its own: the packed linears with
        the SiLU-fused gate_up, more than 64 rows, and every such projection split at T."""
        if not self.prefill_partials or T <= 64 or not self.fused_decode_ready():
            return False
        return all(lin.N % 128 == 0 and lin.tile_ksplit(T) >= 2
                   for layer in self.layers
                   for lin in (layer.qkv_proj, layer.o_proj, layer.down_proj))

    def prefill_down_partials_ok(self, T: int) -> bool:
        """Whether forward runs a T-token prefill with only the down projection writing
        split-K partial sums for the next add+RMSNorm (qkv and o finished in their launches):
        where the tiled GEMM's own plan for partial output splits every layer's down
        projection over K (partial_plan >= 2; e.g. 4096 rows: 256 x 192 tiles in two slices
        fill the CUs once, where the finished form's 128 x 192 tiles run below the persistent
        tiles' rate), so the fp16 store and, for smaller T, a split's finish launch go."""
        if not self.prefill_partials or T <= 64 or not self.fused_decode_ready():
            return False
        return all(layer.down_proj.N % 128 == 0 and layer.down_proj.partial_plan(T) >= 2
                   for layer in self.layers)

    def _forward_partials(self, x, pos, cache, logits_indices, B, down_only: bool = False):
        """forward's prefill with the projections' split-K partial sums handed to the next
        kernel (prefill_partials_ok): the same roundings in the same order as the finished
        projections, so the outputs are identical, with three launches per layer fewer.
        down_only (prefill_down_partials_ok): qkv and o finished as in forward, the down
        projection's partials in the tiled GEMM's planned slices summed by the next
        add+RMSNorm (in slice order, then rounded to fp16 as the finished projection rounds
        its fp32 sum: the same values up to the order of the fp32 additions)."""
        cfg = self.cfg
        T, H = x.shape
        eps = cfg.rms_norm_eps
        dev = x.device
        f32 = lambda n: torch.empty(n, device=dev, dtype=torch.float32)
        l0 = self.layers[0]
        if down_only:
            dparts = max(layer.down_proj.partial_plan(T) for layer in self.layers)
            qpart = opart = None
        else:
            slices = lambda name: max(getattr(layer, name).tile_ksplit(T) for layer in self.layers)
            dparts = slices("down_proj")
            qpart = f32(slices("qkv_proj") * T * l0.qkv_proj.N)
            opart = f32(slices("o_proj") * T * l0.o_proj.N)
        dpart = f32(dparts * T * l0.down_proj.N)
        residual = x.clone()
        h = torch.empty(T, H, device=dev, dtype=torch.float16)
        qkv = torch.empty(T, cfg.qkv_out, device=dev, dtype=torch.float16)
        attn = torch.empty(T, cfg.num_heads, cfg.head_dim, device=dev, dtype=torch.float16)
        act = torch.empty(T, cfg.intermediate_size, device=dev, dtype=torch.float16)
        Sd = 0
        for i, layer in enumerate(self.layers):
            if i == 0:
                h = layer.input_layernorm(x)
            else:
                F.add_rms_norm_partials_out(dpart, Sd, residual, layer.in_norm, eps, h, residual)
            qp = layer.qkv_proj
            if down_only:
                qp.forward_out(h, qkv)
                cache.rope_and_write(qkv, i, pos, self.rope_cos, self.rope_sin, cfg.mrope_section)
            else:
                Sq = qp.forward_partial(h, qpart)
                cache.rope_and_write(qkv, i, pos, self.rope_cos, self.rope_sin, cfg.mrope_section,
                                     parts=(qpart, Sq, qp.bias, qp.fmt == "int4"))
            cache.attend_qkv(qkv, i, self.scale, attn)
            if down_only:
                o = layer.o_proj(attn.reshape(T, -1))
                F.add_rms_norm_out(o, residual, layer.post_norm, eps, h, residual)
            else:
                So = layer.o_proj.forward_partial(attn.reshape(T, -1), opart)
                F.add_rms_norm_partials_out(opart, So, residual, layer.post_norm, eps, h, residual)
            layer.gate_up_proj.forward_out(h, act)
            if down_only:
                Sd = layer.down_proj.forward_partial_planned(act, dpart)
            else:
                Sd = layer.down_proj.forward_partial(act, dpart)
        cache.finish()
        F.add_rms_norm_partials_out(dpart, Sd, residual, self.norm, eps, h, residual)
        if logits_indices is not None:
            idx = _indices_on(logits_indices, dev)
            h = h[idx].contiguous()
        logits = self.lm_head.logits(h)
        return logits.reshape(1 if logits_indices is not None else B, -1, cfg.vocab_size)

    # ------------------------------------------------------------------ decode fast path
    def decode_buffers(self, n: int, device) -> dict:
        """Static activation buffers for an n-row decode step (kept alive for graphs)."""
        if n not in self._bufs:
            cfg = self.cfg
            H, I = cfg.hidden_size, cfg.intermediate_size
            mk = lambda *s: torch.empty(*s, device=device, dtype=torch.float16)
            f32 = lambda *s: torch.empty(*s, device=device, dtype=torch.float32)
            Sd = max(l.down_proj.partial_slices() for l in self.layers)
            So = max(l.o_proj.partial_slices() for l in self.layers)
            Sq = max(l.qkv_proj.partial_slices() for l in self.layers)
            self._bufs[n] = {
                "h": mk(n, H), "res": mk(n, H), "res2": mk(n, H),
                "qkv": mk(n, cfg.qkv_out), "attn": mk(n, cfg.num_heads * cfg.head_dim),
                "act": mk(n, I),
                "dpart": f32(Sd, n, H), "opart": f32(So, n, H), "qpart": f32(Sq, n, cfg.qkv_out),
                "rope": mk(n, cfg.head_dim),
            }
        return self._bufs[n]

    def decode_greedy(self, ids: torch.Tensor, view, ids_out: torch.Tensor,
                      logits_out: Optional[torch.Tensor] = None,
                      next_ids: Optional[torch.Tensor] = None,
                      lengths: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One decode step for pool rows [0, n): ids [n] int64 (device) -> ids_out [n]
        (greedy).  Reads write positions from the view (pool.lengths, or a view_graph
        view's write_pos buffer) plus the rope delta, and writes K/V there.
        With ``lengths`` the final launch also advances lengths[:n] by one and with
        ``next_ids`` copies the new ids there.  No allocation, no host sync.

        Per layer (7 launches): add+RMSNorm over the previous down projection's fp32
        split-K partials -> qkv (partials) -> attention with the qkv bias + M-RoPE +
        KV-pool write in its prologue, split softmax states out -> o_proj merging those
        states while it stages its input (partials) -> add+RMSNorm over them -> gate_up +
        SiLU -> down (partials).  Partial results cross a kernel boundary, never a
        device-scope fence.  Up to ``decode_addnorm_rows`` rows (5 launches per layer): qkv
        and gate_up form the add+RMSNorm over the partials in their own input staging (each
        workgroup reads the rows' partials, a few tens of KB), with the residual alternating
        between two buffers; the outputs are the same."""
        cfg = self.cfg
        if not self.fused_decode_ready():
            raise RuntimeError("decode_greedy runs the packed int4 / fp16 linears only; decode "
                               "a model with other linears (FP8, fp8_out norms) through forward()")
        n = ids.shape[0]
        b = self.decode_buffers(n, ids.device)
        eps = cfg.rms_norm_eps
        h, res = b["h"], b["res"]
        if self._addnorm_ok(n):
            return self._decode_greedy_addnorm(ids, view, ids_out, logits_out, next_ids, lengths, b)
        # the step's rotary rows (one position per row, the same for every layer) come out
        # of the first launch, so that no attention prologue looks them up
        F.embed_rms_norm_rope_out(ids, self.lm_head.table_packed, True, self.layers[0].in_norm,
                                  eps, h, res, view.kv_pos, view.rope_delta, self.rope_cos,
                                  self.rope_sin, b["rope"])
        S = 0
        for i, layer in enumerate(self.layers):
            if i > 0:
                F.add_rms_norm_partials_out(b["dpart"], S, res, layer.in_norm, eps, h, res)
            qp = layer.qkv_proj
            Sq = qp.forward_partial(h, b["qpart"])
            states, Sa = view.attend_fused(b["qpart"], Sq, qp.bias, qp.fmt == "int4", i,
                                           self.scale, self.rope_cos, self.rope_sin,
                                           cfg.mrope_section, rope_rows=b["rope"])
            So = layer.o_proj.forward_partial_attn(states, Sa, cfg.num_kv_heads,
                                                   cfg.num_heads // cfg.num_kv_heads, n, b["opart"])
            F.add_rms_norm_partials_out(b["opart"], So, res, layer.post_norm, eps, h, res)
            layer.gate_up_proj.forward_out(h, b["act"])
            S = layer.down_proj.forward_partial(b["act"], b["dpart"])
        F.add_rms_norm_partials_out(b["dpart"], S, res, self.norm, eps, h, res)
        self.lm_head.argmax_out(h, ids_out, logits_out, next_ids, lengths)
        return ids_out

    # rows up to which decode_greedy forms the add+RMSNorms inside qkv / gate_up (each of
    # their workgroups then reads the rows' fp32 partials: ~86 KB a row for down's 14 slices,
    # which only pays off for a row or two; 0 disables).  The saving is far below the two
    # launches' ~3.7 us each: the consumers' critical path takes the partials' round trip
    # and the rows' reduction instead.
    decode_addnorm_rows = 2
    # o_proj's K slices in that chain (two heads each): few enough that gate_up requests all
    # of them ahead of its weights (8 per thread in flight).  Graph-timed int4 steps, ctx
    # 2048: B = 1 1.118 ms against 1.149 with the norm launches (12 slices: 1.160, 4: 1.125);
    # B = 2 1.159 against 1.181.  Fewer down slices (what qkv reads) made down slower than the
    # smaller read saved (7: 1.176, 5: 1.224 ms).
    decode_addnorm_oslices = 6

    def _addnorm_ok(self, n: int) -> bool:
        """Whether an n-row decode step takes the 5-launch chain: n <= decode_addnorm_rows,
        and the norms' rows fit the fused forms (a chunk of 8 per thread, whole waves per row:
        hidden % 512 == 0, n hidden / 8 <= 512 threads)."""
        H = self.cfg.hidden_size
        return 0 < n <= self.decode_addnorm_rows and H % 512 == 0 and n * (H // 8) <= 512

    def _decode_greedy_addnorm(self, ids, view, ids_out, logits_out, next_ids, lengths, b):
        """decode_greedy's 5-launch layers (n <= decode_addnorm_rows): qkv (layers > 0) and
        gate_up take the previous projection's partials, the residual and the norm gain,
        and write the new residual to the other of res / res2."""
        cfg = self.cfg
        eps = cfg.rms_norm_eps
        n = ids.shape[0]
        h = b["h"]
        cur, other = b["res"], b["res2"]
        F.embed_rms_norm_rope_out(ids, self.lm_head.table_packed, True, self.layers[0].in_norm,
                                  eps, h, cur, view.kv_pos, view.rope_delta, self.rope_cos,
                                  self.rope_sin, b["rope"])
        S = 0
        for i, layer in enumerate(self.layers):
            qp = layer.qkv_proj
            if i > 0:
                Sq = qp.forward_addnorm(b["dpart"], S, cur, layer.in_norm, eps, other,
                                        partial=b["qpart"])
                cur, other = other, cur
            else:
                Sq = qp.forward_partial(h, b["qpart"])
            states, Sa = view.attend_fused(b["qpart"], Sq, qp.bias, qp.fmt == "int4", i,
                                           self.scale, self.rope_cos, self.rope_sin,
                                           cfg.mrope_section, rope_rows=b["rope"])
            So = layer.o_proj.forward_partial_attn(states, Sa, cfg.num_kv_heads,
                                                   cfg.num_heads // cfg.num_kv_heads, n, b["opart"],
                                                   ksplit=self.decode_addnorm_oslices)
            layer.gate_up_proj.forward_addnorm(b["opart"], So, cur, layer.post_norm, eps, other,
                                               out=b["act"])
            cur, other = other, cur
            S = layer.down_proj.forward_partial(b["act"], b["dpart"])
        F.add_rms_norm_partials_out(b["dpart"], S, cur, self.norm, eps, h, cur)
        self.lm_head.argmax_out(h, ids_out, logits_out, next_ids, lengths)
        return ids_out
