"""Preallocated batched KV pool with the reference's layout and cache-view protocol.

Mirrors omniserve/cache/kv_prealloc.py:
* ``PreallocatedKVCache`` (:20-115): per-layer ``k[l]``, ``v[l]`` of shape
  ``[max_batch, max_len, n_kv, head_dim]`` fp16 (here views into one allocation
  ``[n_layers, 2, max_batch, max_len, n_kv, head_dim]``), ``lengths`` int64 = valid
  length = next write position per slot, slot ops (move/snapshot/restore/copy).
* ``_CacheView.flash_decode`` (:272-290): write the new K/V at row*max_len + pos, then
  attend over keys [0, pos] (inclusive); ``lengths`` advance after the last layer.
* ``_PackedPrefillWriter.flash_prefill`` (:181-203): each packed segment's K/V goes to
  ``pool[slot, :L]``; causal attention inside each segment; ``lengths[slot] = L``.
* ``_ChunkedPrefillWriter`` / ``_MixedWriter`` (:118-174): the append form of the same
  thing - segment s writes its ``new_len`` tokens at ``pool[slot, start:start+new_len]``
  and its query i attends to keys ``[0, start+i]`` (cached prefix + the segment, causal);
  ``lengths[slot] = start + new_len``.  A decode token is a segment of one.

Attention, the K/V writes and the slot copies run on the HIP kernels
(omni_decode_attention, omni_mrope_kv_write, omni_prefill_attention, omni_kv_copy_slot);
snapshots for prefix reuse are torch clones.
"""

from __future__ import annotations

from typing import List, Sequence

import torch

from ._lib import call, ptr, require_cuda, stream
from .hostio import to_device

MAX_ATTN_SPLITS = 16


def decode_plan(n_tokens: int, n_kv: int, ctx: int) -> tuple:
    """(waves per workgroup, workgroups per (token, kv head)) for omni_decode_attention,
    from the pool capacity ``ctx``: one workgroup per CU (256) when contexts can be long,
    so that every wave's first two K/V blocks are in flight at once; a single workgroup
    (no partial-state merge launch) when the context is short."""
    groups = max(1, n_tokens * n_kv)
    if ctx <= 128:
        return 4, 1
    waves = 8 if groups >= 16 else 4     # B = 8 (16 groups): (8, 16) 1.3 % faster than (4, 16)
    splits = max(1, min(MAX_ATTN_SPLITS, 256 // groups, ctx // 128))
    return waves, splits


class PreallocatedKVCache:
    def __init__(self, n_layers: int, max_batch: int, n_kv_heads: int, max_len: int,
                 head_dim: int, device, dtype=torch.float16, n_heads: int | None = None):
        if dtype != torch.float16:
            raise ValueError("the KV pool is fp16")
        self.n_layers = n_layers
        self.max_batch = max_batch
        self.max_len = max_len
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.n_heads = n_heads or 6 * n_kv_heads
        self.device = torch.device(device)
        self.storage = torch.zeros(n_layers, 2, max_batch, max_len, n_kv_heads, head_dim,
                                   device=device, dtype=dtype)
        self.k: List[torch.Tensor] = [self.storage[l, 0] for l in range(n_layers)]
        self.v: List[torch.Tensor] = [self.storage[l, 1] for l in range(n_layers)]
        self.lengths = torch.zeros(max_batch, dtype=torch.long, device=device)
        self._active = 0
        # partial softmax states of split decode attention (shared by all layers: launches
        # on one stream are ordered)
        G = self.n_heads // n_kv_heads
        self._attn_ws = torch.empty(max_batch * n_kv_heads * MAX_ATTN_SPLITS * G * (head_dim + 4),
                                    device=device, dtype=torch.float32)
        self.attn_plan = None      # (waves, splits) override; None = decode_plan()

    # ---- slot operations (kv_prealloc.py:43-84) ------------------------------------
    def set_slot_prefix(self, slot: int, legacy_kv, length: int) -> None:
        for li, (k, v) in enumerate(legacy_kv):
            self.k[li][slot, :length] = k[0].transpose(0, 1)
            self.v[li][slot, :length] = v[0].transpose(0, 1)
        self.lengths[slot] = length
        self._active = max(self._active, slot + 1)

    def _copy_slot(self, src: int, dst: int, length: int) -> None:
        call("omni_kv_copy_slot", ptr(self.storage), self.n_layers, self.max_batch, self.max_len,
             self.n_kv_heads * self.head_dim, int(src), int(dst), int(length), ptr(self.lengths),
             stream())

    def move_slot(self, src: int, dst: int) -> None:
        """Move a sequence's KV from slot src to dst (pool compaction on free): one launch
        over every layer's K and V copying the valid prefix, lengths[src] read on the
        device (no host synchronisation)."""
        self._copy_slot(src, dst, -1)

    def snapshot_slot(self, slot: int, length: int):
        ks = [self.k[li][slot, :length].clone() for li in range(self.n_layers)]
        vs = [self.v[li][slot, :length].clone() for li in range(self.n_layers)]
        return ks, vs

    def restore_slot(self, slot: int, snapshot, length: int) -> None:
        ks, vs = snapshot
        for li in range(self.n_layers):
            self.k[li][slot, :length] = ks[li]
            self.v[li][slot, :length] = vs[li]
        self.lengths[slot] = length
        self._active = max(self._active, slot + 1)

    def copy_slot_kv(self, src: int, dst: int, length: int) -> None:
        if not 0 <= length <= self.max_len:
            raise ValueError(f"length {length} outside [0, {self.max_len}]")
        self._copy_slot(src, dst, length)
        self._active = max(self._active, dst + 1)

    # ---- views ---------------------------------------------------------------------
    def view(self, n: int, rope_delta: torch.Tensor | None = None) -> "CacheView":
        return CacheView(self, n, rope_delta)

    def view_graph(self, n: int, write_pos: torch.Tensor, flat: torch.Tensor | None = None,
                   seqused: torch.Tensor | None = None,
                   rope_delta: torch.Tensor | None = None) -> "CacheView":
        """Static view for a captured step (kv_prealloc.py:90-92): write positions come
        from the caller's buffer ``write_pos`` [n] (int64, updated outside the graph) and
        lengths are not advanced.  ``flat`` / ``seqused`` (the reference's precomputed
        row * max_len + pos and pos + 1) are accepted and unused: the kernels derive both
        from write_pos."""
        return CacheView(self, n, rope_delta, write_pos=write_pos)

    def prefill_cache(self, slot: int) -> "ChunkedPrefillWriter":
        """One sequence's prefill into ``slot`` (kv_prealloc.py:94-97): its forward's tokens
        go to pool[slot, :L], lengths[slot] = L."""
        return ChunkedPrefillWriter(self, slot, 0)

    def packed_prefill_cache(self, slots: Sequence[int], seg_lengths: Sequence[int]):
        return PackedPrefillWriter(self, slots, seg_lengths)

    def chunked_prefill_cache(self, slot: int, start: int) -> "ChunkedPrefillWriter":
        """One prefill chunk appended at pool[slot, start:start+L] (kv_prealloc.py:104-108);
        L is the number of tokens the forward brings."""
        return ChunkedPrefillWriter(self, slot, start)

    def mixed_cache(self, slots: Sequence[int], new_lens: Sequence[int],
                    starts: Sequence[int]) -> "PackedPrefillWriter":
        """Decode tokens and a prefill chunk in one forward (kv_prealloc.py:110-116): segment
        s appends new_lens[s] tokens to slot slots[s] at starts[s]."""
        return PackedPrefillWriter(self, slots, new_lens, starts)

    # ---- kernel calls --------------------------------------------------------------
    def attend(self, q: torch.Tensor, q_stride: int, layer_idx: int, kv_len: torch.Tensor,
               kv_by_slot: bool, kv_add: int, out: torch.Tensor, n: int, scale: float,
               slots: torch.Tensor | None = None, plan: tuple | None = None) -> torch.Tensor:
        """omni_decode_attention over pool rows (slots or 0..n-1)."""
        nh = self.n_heads
        if out.numel() < n * nh * self.head_dim:
            raise ValueError("attention output buffer too small")
        w, s = self.checked_plan(n, plan)
        call("omni_decode_attention", ptr(q), q_stride, ptr(self.k[layer_idx]),
             ptr(self.v[layer_idx]), self.max_batch, self.max_len, ptr(slots), ptr(kv_len),
             int(kv_by_slot), kv_add, ptr(out), n, nh, self.n_kv_heads, self.head_dim,
             float(scale), w, s, ptr(self._attn_ws), self._attn_ws.numel(), stream())
        return out

    def checked_plan(self, n: int, plan: tuple | None = None) -> tuple:
        """(waves, splits) for n tokens: the given plan, the pool's override or decode_plan(),
        refused when its split states would not fit the pool's workspace (the library also
        checks the capacity it is given)."""
        w, s = plan or self.attn_plan or decode_plan(n, self.n_kv_heads, self.max_len)
        if n > self.max_batch or not 1 <= s <= MAX_ATTN_SPLITS or w not in (4, 8):
            raise ValueError(f"attention plan (waves {w}, splits {s}) for {n} tokens exceeds "
                             f"the pool workspace ({self.max_batch} rows, {MAX_ATTN_SPLITS} splits)")
        return w, s


class CacheView:
    """Single-forward decode adapter over pool rows [0, n) (kv_prealloc.py:232-290).

    Write positions are read on the device from ``pool.lengths`` (eager: advanced by one
    after the step, ``finish``) or, for a view made by ``view_graph``, from the caller's
    ``write_pos`` buffer (never advanced here); positions add the per-slot ``rope_delta``.
    Besides this build's fused protocol it has the reference's ``flash_decode`` and
    ``update`` (the SDPA route, :263-270) and the transformers-cache queries."""

    def __init__(self, pool: PreallocatedKVCache, n: int, rope_delta: torch.Tensor | None,
                 write_pos: torch.Tensor | None = None):
        self.pool = pool
        self.n = n
        self.rope_delta = rope_delta
        self._graph = write_pos is not None
        if self._graph and (write_pos.dtype != torch.int64 or write_pos.numel() < n):
            raise ValueError("write_pos must hold n int64 positions")
        self.kv_pos = write_pos if self._graph else pool.lengths
        self._snap = None                 # (write positions, window) for update()

    def finish(self) -> None:
        """After the step's last layer: eager views advance lengths[:n] by one (the graph
        runner advances them outside the graph)."""
        if not self._graph:
            self.pool.lengths[:self.n] += 1

    # ---- the reference's SDPA route and cache queries (kv_prealloc.py:240-300) -------
    def _window(self):
        if self._snap is None:
            wp = self.kv_pos[:self.n].clone()
            ret = self.pool.max_len if self._graph else int(wp.max().item()) + 1
            self._snap = (wp, ret)
        return self._snap

    def update(self, key, value, layer_idx, cache_kwargs=None):
        """key/value [n, n_kv, 1, hd] (rotated): written at each row's write position; on
        the last layer (eager) lengths[:n] = write position + 1.  Returns the valid K/V
        window [n, n_kv, L, hd] for SDPA (L = max write position + 1, or max_len)."""
        pool, n = self.pool, self.n
        wp, ret = self._window()
        rows = torch.arange(n, device=wp.device)
        flat = rows * pool.max_len + wp
        nkv, hd = pool.n_kv_heads, pool.head_dim
        pool.k[layer_idx].view(-1, nkv, hd).index_copy_(0, flat, key[:, :, 0, :].to(torch.float16))
        pool.v[layer_idx].view(-1, nkv, hd).index_copy_(0, flat, value[:, :, 0, :].to(torch.float16))
        if layer_idx == pool.n_layers - 1 and not self._graph:
            pool.lengths[:n] = wp + 1
        return (pool.k[layer_idx][:n, :ret].transpose(1, 2),
                pool.v[layer_idx][:n, :ret].transpose(1, 2))

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self._window()[1] - 1

    def get_mask_sizes(self, cache_position, layer_idx: int = 0):
        return self._window()[1], 0

    def get_max_cache_shape(self):
        return self.pool.max_len

    def rope_and_write(self, qkv: torch.Tensor, layer_idx: int, cos_tab, sin_tab,
                       mrope_section, parts=None) -> None:
        """Fused M-RoPE on q/k (in place in the qkv rows) + K/V write at lengths[row].

        ``parts = (partials fp32 [S, n, qkv], S, bias, bias_after_round)``: the qkv rows
        are first formed from the qkv projection's split-K partials (+ bias)."""
        pool = self.pool
        s0, s1, s2 = mrope_section
        if parts is None:
            call("omni_mrope_kv_write", ptr(qkv), qkv.stride(0), None, ptr(self.kv_pos),
                 ptr(self.rope_delta), ptr(cos_tab), ptr(sin_tab), cos_tab.shape[0],
                 ptr(pool.k[layer_idx]), ptr(pool.v[layer_idx]), None, None, pool.max_batch,
                 pool.max_len, self.n, pool.n_heads, pool.n_kv_heads, pool.head_dim, s0, s1, s2,
                 stream())
            return
        pbuf, S, bias, bar = parts
        call("omni_mrope_kv_write_partials", ptr(qkv), qkv.stride(0), ptr(pbuf), S, ptr(bias),
             int(bar), None, ptr(self.kv_pos), ptr(self.rope_delta), ptr(cos_tab), ptr(sin_tab),
             cos_tab.shape[0], ptr(pool.k[layer_idx]), ptr(pool.v[layer_idx]), None, None,
             pool.max_batch, pool.max_len, self.n, pool.n_heads, pool.n_kv_heads, pool.head_dim,
             s0, s1, s2, stream())

    def attend_qkv(self, qkv: torch.Tensor, layer_idx: int, scale: float, out: torch.Tensor,
                   plan: tuple | None = None) -> torch.Tensor:
        """Attention for rows [0, n): keys [0, write position] (the token just written)."""
        return self.pool.attend(qkv, qkv.stride(0), layer_idx, self.kv_pos, True, 1, out,
                                self.n, scale, plan=plan)

    def rope_rows(self, cos_tab, sin_tab, out: torch.Tensor) -> torch.Tensor:
        """out [n, 128] fp16 = cos | sin rows at each row's write position lengths[row] +
        rope_delta[row] (one per decode step, for every layer's attend_fused)."""
        pool = self.pool
        call("omni_rope_rows", None, ptr(self.kv_pos), ptr(self.rope_delta), ptr(cos_tab),
             ptr(sin_tab), cos_tab.shape[0], pool.max_batch, self.n, ptr(out), stream())
        return out

    def attend_fused(self, qparts, nparts: int, bias, bias_after_round: bool, layer_idx: int,
                     scale: float, cos_tab, sin_tab, mrope_section, out=None,
                     plan: tuple | None = None, rope_rows: torch.Tensor | None = None):
        """Decode attention fused with its producer's epilogue: q / new k, v from the qkv
        projection's fp32 split-K partials (+ bias), M-RoPE at lengths[row] + rope_delta
        (from ``rope_rows`` when given, see rope_rows()), new K/V row stored at
        lengths[row], attention over keys [0, lengths[row]].

        With ``out`` the merged fp16 output goes there and is returned; without it the
        split softmax states stay in the pool's workspace and (states, splits) is returned
        for the o_proj that merges them (forward_partial_attn)."""
        pool, n = self.pool, self.n
        w, s = pool.checked_plan(n, plan)
        s0, s1, s2 = mrope_section
        call("omni_decode_attention_fused", ptr(qparts), nparts, ptr(bias), int(bias_after_round),
             ptr(cos_tab), ptr(sin_tab), cos_tab.shape[0], ptr(self.rope_delta), s0, s1, s2,
             ptr(pool.k[layer_idx]), ptr(pool.v[layer_idx]), pool.max_batch, pool.max_len, None,
             ptr(self.kv_pos), ptr(out), n, pool.n_heads, pool.n_kv_heads, pool.head_dim,
             float(scale), w, s, ptr(pool._attn_ws), pool._attn_ws.numel(), int(out is not None),
             ptr(rope_rows), stream())
        return out if out is not None else (pool._attn_ws, s)

    def flash_decode(self, q, key, value, layer_idx, scale):
        """Reference protocol (kv_prealloc.py:272-290): q [n, nh, hd] (rotated), key/value
        [n, nkv, hd]; writes K/V at lengths[row], attends, advances lengths on the last
        layer."""
        pool, n = self.pool, self.n
        rows = torch.arange(n, device=q.device)
        flat = rows * pool.max_len + self.kv_pos[:n]
        nkv, hd = pool.n_kv_heads, pool.head_dim
        pool.k[layer_idx].view(-1, nkv, hd).index_copy_(0, flat, key.to(torch.float16))
        pool.v[layer_idx].view(-1, nkv, hd).index_copy_(0, flat, value.to(torch.float16))
        q = q.contiguous()
        out = torch.empty_like(q)
        pool.attend(q, q.shape[1] * q.shape[2], layer_idx, self.kv_pos, True, 1, out, n, scale)
        if layer_idx == pool.n_layers - 1:
            self.finish()
        return out


class PackedPrefillWriter:
    """Packed prefill adapter (kv_prealloc.py:177-215): segments of a packed batch go to
    their own slots; attention is causal within each segment.  With ``starts`` it is the
    append (mixed batching) adapter of kv_prealloc.py:118-146: segment s writes its tokens
    at pool[slot, start:start+L] and attends to the slot's cached prefix as well."""

    def __init__(self, pool: PreallocatedKVCache, slots: Sequence[int],
                 seg_lengths: Sequence[int] | None, starts: Sequence[int] | None = None):
        self.pool = pool
        self.slots = [int(s) for s in slots]
        self.starts = [0] * len(self.slots) if starts is None else [int(s) for s in starts]
        if len(self.starts) != len(self.slots):
            raise ValueError("one start per segment")
        self.seg = None
        if seg_lengths is not None:
            self._build([int(L) for L in seg_lengths])

    def _build(self, seg: List[int]) -> None:
        pool = self.pool
        if len(seg) != len(self.slots):
            raise ValueError("one length per segment")
        for slot, st, L in zip(self.slots, self.starts, seg):
            if not 0 <= slot < pool.max_batch:
                raise ValueError(f"slot {slot} outside the pool's {pool.max_batch} rows")
            if L < 1 or st < 0 or st + L > pool.max_len:
                raise ValueError(f"segment [{st}, {st + L}) outside [0, max_len={pool.max_len}]")
        if len(set(self.slots)) != len(self.slots):
            raise ValueError("a slot appears in two segments")
        self.seg = seg
        dev = pool.device
        slot_t, pos_t, cu = [], [], [0]
        for s, st, L in zip(self.slots, self.starts, seg):
            slot_t += [s] * L
            pos_t += list(range(st, st + L))
            cu.append(cu[-1] + L)
        self.T = cu[-1]
        # one staged upload (no host wait): token slots, write positions, then the slots and
        # new lengths finish() stores
        n = len(seg)
        meta = to_device(slot_t + pos_t + self.slots + [st + L for st, L in zip(self.starts, seg)],
                         torch.int64, dev)
        self.token_slot = meta[:self.T]
        self.token_pos = meta[self.T:2 * self.T]  # write positions
        self._fin_slots = meta[2 * self.T:2 * self.T + n]
        self._fin_lengths = meta[2 * self.T + n:]
        self.kv_len = self.token_pos + 1          # causal: token at position p sees keys [0, p]
        self.cu_seqlens = to_device(cu, torch.int32, dev)
        self.max_seg = max(seg) if seg else 0

    def bind(self, T: int) -> None:
        """Number of tokens the forward brings (fixed at construction here)."""
        if self.seg is None or self.T != T:
            raise ValueError(f"the forward brings {T} tokens, the adapter was built for "
                             f"{None if self.seg is None else self.T}")

    def rope_and_write(self, qkv: torch.Tensor, layer_idx: int, positions: torch.Tensor,
                       cos_tab, sin_tab, mrope_section, parts=None) -> None:
        """M-RoPE on q/k (in place in the qkv rows) + K/V write of the packed tokens.
        ``parts = (partials fp32 [S, T, qkv], S, bias, bias_after_round)``: the qkv rows are
        first formed from the qkv projection's split-K partials (+ bias)."""
        pool = self.pool
        s0, s1, s2 = mrope_section
        if parts is not None:
            pbuf, S, bias, bar = parts
            call("omni_mrope_kv_write_partials", ptr(qkv), qkv.stride(0), ptr(pbuf), S, ptr(bias),
                 int(bar), ptr(positions), None, None, ptr(cos_tab), ptr(sin_tab),
                 cos_tab.shape[0], ptr(pool.k[layer_idx]), ptr(pool.v[layer_idx]),
                 ptr(self.token_slot), ptr(self.token_pos), pool.max_batch, pool.max_len, self.T,
                 pool.n_heads, pool.n_kv_heads, pool.head_dim, s0, s1, s2, stream())
            return
        call("omni_mrope_kv_write", ptr(qkv), qkv.stride(0), ptr(positions), None, None,
             ptr(cos_tab), ptr(sin_tab), cos_tab.shape[0], ptr(pool.k[layer_idx]),
             ptr(pool.v[layer_idx]), ptr(self.token_slot), ptr(self.token_pos), pool.max_batch,
             pool.max_len, self.T, pool.n_heads, pool.n_kv_heads, pool.head_dim, s0, s1, s2,
             stream())

    def attend_qkv(self, qkv: torch.Tensor, layer_idx: int, scale: float,
                   out: torch.Tensor) -> torch.Tensor:
        from .attention import prefill_attention_pool
        return prefill_attention_pool(self, qkv, layer_idx, scale, out)

    def finish(self) -> None:
        # on the device from the uploaded values: a host scalar stored into the lengths
        # would wait for the queue
        if self.slots:
            self.pool.lengths.index_copy_(0, self._fin_slots, self._fin_lengths)
            self.pool._active = max(self.pool._active, max(self.slots) + 1)

    def update(self, k, v, layer_idx, cache_kwargs=None):
        """The reference's SDPA route (kv_prealloc.py:205-215, 222-229): k, v [1, n_kv, T, hd]
        (rotated) of the packed tokens, each segment's rows written to its slot at its start;
        lengths set on the last layer.  Returns k, v unchanged (the caller attends over the
        packed tokens with its own mask)."""
        pool = self.pool
        self.bind(k.shape[2])
        off = 0
        for slot, st, L in zip(self.slots, self.starts, self.seg):
            pool.k[layer_idx][slot, st:st + L] = k[0, :, off:off + L].transpose(0, 1)
            pool.v[layer_idx][slot, st:st + L] = v[0, :, off:off + L].transpose(0, 1)
            off += L
        if layer_idx == pool.n_layers - 1:
            self.finish()
        return k, v

    def flash_prefill(self, q, k, v, layer_idx, scale):
        """Reference protocol (kv_prealloc.py:181-203, 121-146): q [T, nh, hd], k/v
        [T, nkv, hd] (rotated).  Writes K/V to the slots at their starts, causal attention
        per segment over the cached prefix + the segment; lengths on the last layer."""
        pool = self.pool
        self.bind(q.shape[0])
        off = 0
        for slot, st, L in zip(self.slots, self.starts, self.seg):
            pool.k[layer_idx][slot, st:st + L] = k[off:off + L]
            pool.v[layer_idx][slot, st:st + L] = v[off:off + L]
            off += L
        q = q.contiguous()
        out = torch.empty_like(q)
        from .attention import prefill_attention_pool
        prefill_attention_pool(self, q, layer_idx, scale, out, q_stride=q.shape[1] * q.shape[2])
        if layer_idx == pool.n_layers - 1:
            self.finish()
        return out


class ChunkedPrefillWriter(PackedPrefillWriter):
    """_ChunkedPrefillWriter (kv_prealloc.py:149-174): one chunk of a long prompt appended
    at pool[slot, start:start+L]; its queries attend to pool[slot, 0:start+i] (the cached
    prefix + the chunk, causal).  L is taken from the forward that uses it."""

    def __init__(self, pool: PreallocatedKVCache, slot: int, start: int):
        super().__init__(pool, [slot], None, [start])

    def bind(self, T: int) -> None:
        if self.seg is None:
            self._build([int(T)])
        super().bind(T)
