"""Deterministic synthetic weights and inputs for the benchmark configurations.

There are no Qwen2-VL checkpoints offline, so every run uses seeded random
weights of the real architecture (Qwen2-VL-2B text decoder): N(0, 0.02) fp16
linears and embeddings, RMSNorm gains 1.0, qkv bias N(0, 0.02).  The int4 (GPTQ)
configuration draws codes uniform in [0, 15] (zero point 8) and per-group fp16
scales |N(0, 0.02)| / 7, in the AutoGPTQ layout the reference ingests
(omniserve/kernels/marlin_linear.py:83-96, 114-143).

Everything is generated on the CPU from ``torch.Generator`` seeds derived from
the tensor name, so the GPU box and the CPU oracle see bit-identical values.
Tensors are returned in the reference's fused layouts (qwen2_llm.py:193-219):
qkv = q|k|v and gate_up = gate|up along the output dimension.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass, field
from typing import Dict, List

import torch


@dataclass
class DecoderShape:
    """Qwen2-VL-2B text decoder (omniserve/model/qwen2_llm.py:25-36)."""
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

    @property
    def qkv_out(self) -> int:
        return (self.num_heads + 2 * self.num_kv_heads) * self.head_dim


def _gen(seed: int, name: str) -> torch.Generator:
    h = hashlib.sha256(f"{seed}:{name}".encode()).digest()
    g = torch.Generator()
    g.manual_seed(int.from_bytes(h[:8], "little") & ((1 << 63) - 1))
    return g


def randn16(shape, std: float, seed: int, name: str) -> torch.Tensor:
    """N(0, std) values rounded to fp16 (CPU)."""
    return (torch.randn(*shape, generator=_gen(seed, name)) * std).to(torch.float16)


def gptq_random(K: int, N: int, seed: int, name: str, group: int = 128):
    """AutoGPTQ-format int4 linear: qweight int32 [K/8, N], scales fp16 [K/group, N]."""
    g = _gen(seed, name)
    codes = torch.randint(0, 16, (K // 8, 8, N), generator=g, dtype=torch.int32)
    word = torch.zeros(K // 8, N, dtype=torch.int64)
    for e in range(8):
        word |= codes[:, e, :].to(torch.int64) << (4 * e)
    word = torch.where(word >= 2**31, word - 2**32, word).to(torch.int32)
    scales = (torch.randn(K // group, N, generator=g).abs() * 0.02 / 7.0).to(torch.float16)
    return word, scales


def fp16_decoder(shape: DecoderShape, seed: int = 0, num_layers: int | None = None) -> Dict:
    """fp16 weights: dict(embed [V,H], norm [H], layers=[dict(...)]), nn.Linear layout [N, K]."""
    L = shape.num_layers if num_layers is None else num_layers
    H, I = shape.hidden_size, shape.intermediate_size
    out = {
        "embed": randn16((shape.vocab_size, H), 0.02, seed, "embed"),
        "norm": torch.ones(H, dtype=torch.float16),
        "layers": [],
    }
    for i in range(L):
        out["layers"].append({
            "in_norm": torch.ones(H, dtype=torch.float16),
            "post_norm": torch.ones(H, dtype=torch.float16),
            "qkv_w": randn16((shape.qkv_out, H), 0.02, seed, f"l{i}.qkv"),
            "qkv_b": randn16((shape.qkv_out,), 0.02, seed, f"l{i}.qkv_b"),
            "o_w": randn16((H, shape.num_heads * shape.head_dim), 0.02, seed, f"l{i}.o"),
            "gate_up_w": randn16((2 * I, H), 0.02, seed, f"l{i}.gate_up"),
            "down_w": randn16((H, I), 0.02, seed, f"l{i}.down"),
        })
    return out


def gptq_decoder(shape: DecoderShape, seed: int = 0, num_layers: int | None = None) -> Dict:
    """int4 GPTQ weights (AutoGPTQ layout, fused q|k|v and gate|up along N); fp16 embed."""
    L = shape.num_layers if num_layers is None else num_layers
    H, I = shape.hidden_size, shape.intermediate_size
    out = {
        "embed": randn16((shape.vocab_size, H), 0.02, seed, "embed"),
        "norm": torch.ones(H, dtype=torch.float16),
        "layers": [],
    }
    for i in range(L):
        qkv_q, qkv_s = gptq_random(H, shape.qkv_out, seed, f"l{i}.qkv")
        o_q, o_s = gptq_random(shape.num_heads * shape.head_dim, H, seed, f"l{i}.o")
        gu_q, gu_s = gptq_random(H, 2 * I, seed, f"l{i}.gate_up")
        d_q, d_s = gptq_random(I, H, seed, f"l{i}.down")
        out["layers"].append({
            "in_norm": torch.ones(H, dtype=torch.float16),
            "post_norm": torch.ones(H, dtype=torch.float16),
            "qkv_q": qkv_q, "qkv_s": qkv_s,
            "qkv_b": randn16((shape.qkv_out,), 0.02, seed, f"l{i}.qkv_b"),
            "o_q": o_q, "o_s": o_s,
            "gate_up_q": gu_q, "gate_up_s": gu_s,
            "down_q": d_q, "down_s": d_s,
        })
    return out


def random_ids(n: int, vocab: int, seed: int, name: str) -> torch.Tensor:
    return torch.randint(0, vocab, (n,), generator=_gen(seed, name), dtype=torch.int64)


def context_lengths(n: int, lo: int, hi: int, seed: int, name: str = "ctx") -> torch.Tensor:
    """Per-sequence context lengths uniform in [lo, hi] (config 2)."""
    return torch.randint(lo, hi + 1, (n,), generator=_gen(seed, name), dtype=torch.int64)


def kv_prefix(n_layers: int, rows: int, max_len: int, nkv: int, hd: int, lengths, seed: int,
              layer: int, which: str) -> torch.Tensor:
    """N(0,1) fp16 pool contents for one layer's K or V, valid up to lengths[b] (zeros after)."""
    g = _gen(seed, f"kv.{which}.{layer}")
    t = torch.zeros(rows, max_len, nkv, hd, dtype=torch.float16)
    for b in range(len(lengths)):
        L = int(lengths[b])
        t[b, :L] = torch.randn(L, nkv, hd, generator=g).to(torch.float16)
    return t


def vision_tower(cfg=None, seed: int = 0, depth: int | None = None) -> Dict[str, torch.Tensor]:
    """Seeded fp16 vision-tower weights under the Hugging Face ``visual.*`` key names
    (the layout load_vit_from_state_dict reads): linear weights and biases N(0, 0.02),
    LayerNorm gains 1 + N(0, 0.02) and biases N(0, 0.02)."""
    from .vit import VisionConfig
    cfg = cfg or VisionConfig()
    D, I, M = cfg.embed_dim, cfg.mlp_dim, cfg.merged_dim
    nb = cfg.depth if depth is None else depth
    one = lambda n, name: (1.0 + randn16((n,), 0.02, seed, name).float()).to(torch.float16)
    sd = {"visual.patch_embed.proj.weight": randn16(
        (D, cfg.in_chans, cfg.temporal_patch_size, cfg.patch_size, cfg.patch_size), 0.02, seed, "pe")}
    for i in range(nb):
        p = f"visual.blocks.{i}."
        for nm in ("norm1", "norm2"):
            sd[p + nm + ".weight"] = one(D, f"{p}{nm}.w")
            sd[p + nm + ".bias"] = randn16((D,), 0.02, seed, f"{p}{nm}.b")
        for nm, (n, k) in {"attn.qkv": (3 * D, D), "attn.proj": (D, D), "mlp.fc1": (I, D),
                           "mlp.fc2": (D, I)}.items():
            sd[p + nm + ".weight"] = randn16((n, k), 0.02, seed, f"{p}{nm}.w")
            sd[p + nm + ".bias"] = randn16((n,), 0.02, seed, f"{p}{nm}.b")
    sd["visual.merger.ln_q.weight"] = one(D, "lnq.w")
    sd["visual.merger.ln_q.bias"] = randn16((D,), 0.02, seed, "lnq.b")
    sd["visual.merger.mlp.0.weight"] = randn16((M, M), 0.02, seed, "m0.w")
    sd["visual.merger.mlp.0.bias"] = randn16((M,), 0.02, seed, "m0.b")
    sd["visual.merger.mlp.2.weight"] = randn16((cfg.out_hidden, M), 0.02, seed, "m2.w")
    sd["visual.merger.mlp.2.bias"] = randn16((cfg.out_hidden,), 0.02, seed, "m2.b")
    return sd


def pixel_patches(grids, patch_dim: int, seed: int, name: str = "px") -> torch.Tensor:
    """N(0, 1) fp16 flattened patches [sum t*h*w, patch_dim] (normalised pixels) for the
    given (t, h, w) grids."""
    n = sum(t * h * w for t, h, w in grids)
    return randn16((n, patch_dim), 1.0, seed, name)
