"""Host side of the pool attention kernels (decode split-K and packed causal prefill).

``prefill_attention_pool`` is the varlen causal attention of the packed prefill
(omniserve/cache/kv_prealloc.py:181-203) over K/V already written to the pool: the host
cuts every segment into query blocks of consecutive tokens and picks one of three kernels:

* <= 32-token blocks, omni_prefill_attention_gqa: one workgroup per (block, KV head)
  sharing every K/V tile among the group's query heads, when those workgroups fill the GPU
  (one wave per SIMD leaves its softmax's latency unhidden, so with fewer workgroups the
  per-head kernels are faster);
* otherwise <= 16-token blocks, one (block, query head) item each:
  omni_prefill_attention_split (the item's key tiles split over the four waves of a
  workgroup, states merged in LDS) for up to 4 items per CU, omni_prefill_attention (one
  wave per item) beyond that.

MI355X, 12 heads / 2 KV heads, us per launch (per-wave / split / shared-tile): one
256-token prompt 13.0 / 6.3 / 24.0; 4 x 256 13.3 / 12.3 / 24.2; 1 x 1024 40.2 / 33.3 /
78.7; 1 x 2048 101.9 / 110.3 / 152.7; 8 x 512 63.8 / 48.7 / 44.9; a 256-token chunk
appended to 1792 keys 72.3 / 23.1 / 150.9; 32 single tokens at 2048 keys 75.5 / 42.8 /
146.5.  The per-wave and shared-tile kernels give identical outputs; the split one agrees
with them to the fp16 rounding of the probabilities.
"""

from __future__ import annotations

import torch

from ._lib import call, ptr, stream
from .hostio import to_device

QBLOCK = 16
QBLOCK_GQA = 32
# (block, head) items per CU up to which the key-split kernel runs (0: never)
SPLIT_ITEMS_PER_CU = 4


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
        if nqb32 * pool.n_kv_heads >= cus and nh // pool.n_kv_heads <= 8:
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
