"""Host side of the pool attention kernels (decode split-K and packed causal prefill).

``prefill_attention_pool`` is the varlen causal attention of the packed prefill
(omniserve/cache/kv_prealloc.py:181-203) over K/V already written to the pool: the host
cuts every segment into query blocks of consecutive tokens - <= 16 for
omni_prefill_attention, one wavefront per (block, query head), used for short segments
(decode tokens in a mixed batch, small chunks); <= 32 for omni_prefill_attention_gqa, one
workgroup per (block, KV head) sharing every K/V tile among the group's query heads, used
when those workgroups fill the GPU (one wave per SIMD leaves its softmax's latency
unhidden, so with fewer workgroups the per-head kernel is faster: MI355X, 12 heads / 2 KV
heads, 8 x 512 tokens 46 against 64 us, 1 x 256 tokens 24 against 13 us).  The two give
identical outputs.
"""

from __future__ import annotations

import torch

from ._lib import call, ptr, stream

QBLOCK = 16
QBLOCK_GQA = 32


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
    return torch.tensor(blocks, dtype=torch.int32, device=device).reshape(-1, 2)


def prefill_attention_pool(writer, q: torch.Tensor, layer_idx: int, scale: float,
                           out: torch.Tensor, q_stride: int | None = None) -> torch.Tensor:
    """Causal attention of the writer's packed tokens over their pool rows."""
    pool = writer.pool
    nqb32 = sum(-(-L // QBLOCK_GQA) for L in writer.seg)
    gqa = (nqb32 * pool.n_kv_heads >= _num_cus(q.device)
           and pool.n_heads // pool.n_kv_heads <= 8)
    qb = getattr(writer, "_qblocks", None)
    if qb is None:
        qb = query_blocks(writer.seg, q.device, QBLOCK_GQA if gqa else QBLOCK)
        writer._qblocks = qb
    nh = pool.n_heads
    call("omni_prefill_attention_gqa" if gqa else "omni_prefill_attention", ptr(q),
         q_stride or q.stride(0), ptr(pool.k[layer_idx]),
         ptr(pool.v[layer_idx]), pool.max_batch, pool.max_len, ptr(writer.token_slot),
         ptr(writer.kv_len), ptr(qb), qb.shape[0], ptr(out), nh * pool.head_dim, nh,
         pool.n_kv_heads, pool.head_dim, float(scale), stream())
    return out
