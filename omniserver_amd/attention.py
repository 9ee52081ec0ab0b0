"""Host side of the pool attention kernels (decode split-K and packed causal prefill).

``prefill_attention_pool`` is the varlen causal attention of the packed prefill
(omniserve/cache/kv_prealloc.py:181-203) over K/V already written to the pool: the host
cuts every segment into query blocks of consecutive tokens and picks one of four kernels:

* <= 32-token blocks, one workgroup per (block, KV head) sharing every K/V tile among the
  group's query heads: omni_prefill_attention_gqa_halves (the block's key tiles split
  between two groups of four waves, merged in LDS; <= 6 query heads per KV head) when the
  longest segment has >= 256 tokens and the workgroups fill half the GPU, else
  omni_prefill_attention_gqa (four waves) when they fill all of it (one wave per SIMD
  leaves its softmax's latency unhidden, so with fewer workgroups the per-head kernels are
  faster);
* otherwise <= 16-token blocks, one (block, query head) item each:
  omni_prefill_attention_split (the item's key tiles split over the four waves of a
  workgroup, states merged in LDS) for up to 4 items per CU, omni_prefill_attention (one
  wave per item) beyond that.

MI355X, 12 heads / 2 KV heads, us per launch (per-wave / split / shared-tile / two-group
shared-tile): one 256-token prompt 13.1 / 6.4 / 24.3 / 23.7; 1 x 1024 39.7 / 32.7 / 79.7 /
57.4; 1 x 2048 101.3 / 109.5 / 152.8 / 103.0; 1 x 4096 285.1 / 404.0 / 302.2 / 195.2;
2 x 2048 160.9 / 197.5 / 154.8 / 105.3; 4 x 1024 99.7 / 93.8 / 81.9 / 59.9; 8 x 512 63.7 /
48.8 / 45.2 / 37.5; 16 x 512 96.8 / 88.6 / 86.7 / 73.9; 8 x 384 33.6 / 31.1 / 34.8 / 31.2;
16 x 256 33.5 / 33.8 / 26.7 / 26.2; 64 x 128 38.1 / 54.6 / 35.0 / 40.3; 128 x 64 28.5 /
46.8 / 25.4 / 34.8; a 256-token chunk appended to 1792 keys 72.0 / 22.6 / 152.3 / 101.9;
32 single tokens at 2048 keys 75.1 / 42.5 / 148.8 / 99.7.  The per-wave and shared-tile
kernels give identical outputs; the split ones agree with them to the fp16 rounding of the
probabilities (and, for the two-group kernel, of the second group's output).
"""

from __future__ import annotations

import torch

from ._lib import call, ptr, stream
from .hostio import to_device

QBLOCK = 16
QBLOCK_GQA = 32
# (block, head) items per CU up to which the key-split kernel runs (0: never)
SPLIT_ITEMS_PER_CU = 4
# the two-group shared-tile kernel: query heads per KV head it is built for, and the
# longest segment from which it runs
HALVES_MAX_GROUP = 6
HALVES_MIN_SEG = 256


_CUS = {}


def _num_cus(device) -> int:
    if device not in _CUS:
        _CUS[device] = torch.cuda.get_device_properties(device).multi_processor_count
    return _CUS[device]


def query_blocks(seg_lengths, device, block: int = QBLOCK) -> torch.Tensor:
    """int32 [nqb, 2] (first token, count) covering every segment in blocks of <= block."""
    blocks = []
    off = 0
    for L in seg_lengths:
        for s in range(0, L, block):
            blocks.append((off + s, min(block, L - s)))
        off += L
    return to_device(blocks, torch.int32, device).reshape(-1, 2)


def prefill_attention_pool(writer, q: torch.Tensor, layer_idx: int, scale: float,
                           out: torch.Tensor, q_stride: int | None = None) -> torch.Tensor:
    """Causal attention of the writer's packed tokens over their pool rows."""
    pool = writer.pool
    nh = pool.n_heads
    plan = getattr(writer, "_attn_plan", None)
    if plan is None:
        cus = _num_cus(q.device)
        nqb32 = sum(-(-L // QBLOCK_GQA) for L in writer.seg)
        items32 = nqb32 * pool.n_kv_heads
        group = nh // pool.n_kv_heads
        if (group <= HALVES_MAX_GROUP and max(writer.seg) >= HALVES_MIN_SEG
                and 2 * items32 >= cus):
            plan = ("omni_prefill_attention_gqa_halves",
                    query_blocks(writer.seg, q.device, QBLOCK_GQA))
        elif items32 >= cus and group <= 8:
            plan = ("omni_prefill_attention_gqa", query_blocks(writer.seg, q.device, QBLOCK_GQA))
        else:
            qb = query_blocks(writer.seg, q.device, QBLOCK)
            split = qb.shape[0] * nh <= SPLIT_ITEMS_PER_CU * cus
            plan = ("omni_prefill_attention_split" if split else "omni_prefill_attention", qb)
        writer._attn_plan = plan
    fn, qb = plan
    call(fn, ptr(q), q_stride or q.stride(0), ptr(pool.k[layer_idx]),
         ptr(pool.v[layer_idx]), pool.max_batch, pool.max_len, ptr(writer.token_slot),
         ptr(writer.kv_len), ptr(qb), qb.shape[0], ptr(out), nh * pool.head_dim, nh,
         pool.n_kv_heads, pool.head_dim, float(scale), stream())
    return out
