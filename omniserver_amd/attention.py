"""Host side of the pool attention kernels (decode split-K and packed causal prefill).

``prefill_attention_pool`` is the varlen causal attention of the packed prefill
(omniserve/cache/kv_prealloc.py:181-203) over K/V already written to the pool:
the host cuts every segment into query blocks of <= 16 consecutive tokens, the
kernel gives each (block, query head) one wavefront.
"""

from __future__ import annotations

import torch

from ._lib import call, ptr, stream

QBLOCK = 16


def query_blocks(seg_lengths, device) -> torch.Tensor:
    """int32 [nqb, 2] (first token, count) covering every segment in blocks of <= 16."""
    blocks = []
    off = 0
    for L in seg_lengths:
        for s in range(0, L, QBLOCK):
            blocks.append((off + s, min(QBLOCK, L - s)))
        off += L
    return torch.tensor(blocks, dtype=torch.int32, device=device).reshape(-1, 2)


def prefill_attention_pool(writer, q: torch.Tensor, layer_idx: int, scale: float,
                           out: torch.Tensor, q_stride: int | None = None) -> torch.Tensor:
    """Causal attention of the writer's packed tokens over their pool rows."""
    pool = writer.pool
    qb = getattr(writer, "_qblocks", None)
    if qb is None:
        qb = query_blocks(writer.seg, q.device)
        writer._qblocks = qb
    nh = pool.n_heads
    call("omni_prefill_attention", ptr(q), q_stride or q.stride(0), ptr(pool.k[layer_idx]),
         ptr(pool.v[layer_idx]), pool.max_batch, pool.max_len, ptr(writer.token_slot),
         ptr(writer.kv_len), ptr(qb), qb.shape[0], ptr(out), nh * pool.head_dim, nh,
         pool.n_kv_heads, pool.head_dim, float(scale), stream())
    return out
