"""Model runners: the drop-in boundary the engine/scheduler call every iteration.

``ModelRunner`` (omniserve/runners/base.py:26-57) is the abstract interface;
``StubRunner`` (:60-91) the no-GPU control-plane double; ``MultimodalRunner``
(runners/multimodal.py:19-379) the model-agnostic runner over the preallocated KV
pool; ``NativeQwenVLRunner`` (runners/qwen_vl_native.py:14-20) keeps the
reference's entry-point name and constructor signature.

Decode (multimodal.py:286-357): sequences sorted by slot must occupy slots [0, n);
one step advances each by one token.  With ``use_graph=True`` the whole step -
embedding gather + 28 layers + final norm + lm_head/argmax + length advance - is one
HIP-graph replay per batch size (captured lazily, static buffers kept alive; a batch with
non-greedy rows replays a second graph that also writes the fp16 logits, from which the
host samples, multimodal.py:306-313, 342-357).  The
host does at most one small H2D (token ids, only when the batch composition
changed) and one D2H (the new ids) per step.  While the batch can go on unchanged
(nobody has finished, every row has room) the next step's replay is enqueued before the
current step is waited for - its input ids are the current step's outputs, left on the
device by the graph - so the GPU never waits for the host's per-step bookkeeping.  Any
other call on the runner (a different batch, prefill, free, chunked prefill) first takes
that step back with ``settle()``: its length advance is undone and the K/V row it wrote
lies past the valid length, to be overwritten.

Chunked prefill and mixed batching (multimodal.py:200-284): a long text prompt is
prefilled chunk by chunk into the reserve slot (pool row ``max_running``), each chunk
attending to the chunks before it; ``mixed_step`` runs the running sequences' decode
tokens and one chunk in a single forward.  After the last chunk the prompt's KV prefix
is copied into the next decode slot.
"""

from __future__ import annotations

import abc
from typing import Dict, List

import numpy as np
import torch

from .hostio import to_device
from .kv_cache import PreallocatedKVCache
from .linear import weights_epoch
from .request import Sequence, Status


class ModelRunner(abc.ABC):
    @abc.abstractmethod
    def tokenize(self, seq: Sequence) -> None:
        """Fill seq.prompt_token_ids from the request prompt."""

    @abc.abstractmethod
    def prefill(self, seqs: List[Sequence]) -> None:
        """Prefill each sequence's prompt; append the first generated token."""

    @abc.abstractmethod
    def decode(self, seqs: List[Sequence]) -> None:
        """Advance every running sequence by exactly one token."""

    def chunk_prefill(self, seq: Sequence) -> None:
        raise NotImplementedError("this runner does not support chunked prefill")

    def mixed_step(self, chunk_seq: Sequence, decode_seqs: List[Sequence]) -> None:
        self.chunk_prefill(chunk_seq)
        self.decode(decode_seqs)

    @abc.abstractmethod
    def detokenize(self, seq: Sequence, new_token_ids: List[int]) -> str:
        """Render new token ids as text for streaming."""

    def free(self, seq: Sequence) -> None:
        """Release a finished sequence's resources (default: nothing)."""


class StubRunner(ModelRunner):
    """Deterministic no-GPU runner for exercising a scheduler/engine."""

    def __init__(self, reply: str = "ok " * 8):
        self._reply_tokens = reply.split()

    def tokenize(self, seq: Sequence) -> None:
        p = seq.request.prompt
        n = len(p.split()) if isinstance(p, str) else len(p)
        seq.prompt_token_ids = list(range(max(1, n)))

    def prefill(self, seqs: List[Sequence]) -> None:
        for seq in seqs:
            seq.kv_handle = {"len": seq.num_prompt_tokens}
            seq.append_token(0)
            seq.maybe_finish()

    def decode(self, seqs: List[Sequence]) -> None:
        for seq in seqs:
            seq.append_token(seq.num_output_tokens)
            seq.kv_handle["len"] += 1
            seq.maybe_finish()

    def detokenize(self, seq: Sequence, new_token_ids: List[int]) -> str:
        return " ".join(self._reply_tokens[t % len(self._reply_tokens)] for t in new_token_ids) + " "


class MultimodalRunner(ModelRunner):
    def __init__(self, adapter, max_running: int = 32, max_len: int = 1024, prefix_cache=None,
                 use_graph: bool = False):
        if prefix_cache is not None:
            raise NotImplementedError("prefix caching is not part of this build")
        self.adapter = adapter
        self.device = adapter.device
        self.max_running = max_running
        self.image_token_id = adapter.image_token_id
        self.eos_ids = adapter.eos_ids
        self._use_graph = use_graph
        self._reserve_slot = max_running       # kept for layout parity (multimodal.py:32-37)
        self._pool = PreallocatedKVCache(
            n_layers=adapter.num_layers, max_batch=max_running + 1,
            n_kv_heads=adapter.num_kv_heads, max_len=max_len, head_dim=adapter.head_dim,
            device=self.device, dtype=torch.float16, n_heads=adapter.num_heads)
        self._rope_delta = torch.zeros(max_running + 1, dtype=torch.int64, device=self.device)
        self._slot_seq: List[Sequence] = []
        self._kv_len: List[int] = []          # host mirror of pool.lengths for active slots
        self._graphs: Dict[int, tuple] = {}
        self._prefill_graphs: Dict[tuple, dict] = {}
        self._prefill_epoch = weights_epoch()
        self._graphs_sampled: Dict[int, tuple] = {}
        self._eager: Dict[int, dict] = {}
        self._dev_ids_for = None              # batch whose next ids already sit on device
        self._pinned_ids = torch.zeros(max_running + 1, dtype=torch.int64).pin_memory()
        # new ids come back through two pinned buffers (the step being collected and the
        # one enqueued ahead of it), each with its event
        self._pinned_out = [torch.zeros(max_running + 1, dtype=torch.int64).pin_memory()
                            for _ in range(2)]
        self._out_ready = [torch.cuda.Event() for _ in range(2)] if torch.cuda.is_available() else None
        self._pin_next = 0
        self._ahead = None                    # (batch key, n, buffer) of a step enqueued ahead

    @property
    def pool(self) -> PreallocatedKVCache:
        return self._pool

    # ---- ModelRunner interface -----------------------------------------------------
    def tokenize(self, seq: Sequence) -> None:
        if not seq.prompt_token_ids:
            seq.prompt_token_ids = self.adapter.encode_prompt(seq.request.prompt)
        sp = seq.request.sampling
        for e in self.eos_ids:
            if e not in sp.stop_token_ids:
                sp.stop_token_ids.append(e)

    # ---- the decode step enqueued ahead --------------------------------------------
    def steps_ahead(self) -> int:
        """1 while a decode step for the last batch has been enqueued ahead of the caller."""
        return 0 if self._ahead is None else 1

    def settle(self) -> None:
        """Take back a decode step enqueued ahead: undo its length advance and drop its
        ids (its K/V rows sit at the first position past each valid length)."""
        if self._ahead is None:
            return
        _, n, _ = self._ahead
        self._ahead = None
        self._pool.lengths[:n] -= 1
        self._dev_ids_for = None

    @torch.inference_mode()
    def prefill(self, seqs: List[Sequence]) -> None:
        """Packed prefill, compute branch (multimodal.py:116-144): every prompt in one
        forward, causal within its segment, K/V written to its slot, logits only at
        segment ends."""
        if not seqs:
            return
        self.settle()
        base = len(self._slot_seq)
        if base + len(seqs) > self.max_running:
            raise RuntimeError(f"KV pool full: {base} running + {len(seqs)} new > "
                               f"{self.max_running}")
        dev = self.device
        # The packed prompt's host-side inputs are gathered as numpy arrays and uploaded in
        # one pinned copy (ids, image row indices, positions, rope deltas): the GPU is idle
        # until the host has issued them, so per-token Python work and per-input uploads
        # would add to every prefill's latency.
        ids_l, pos_l, seg_lens, deltas, img_rows, vis = [], [], [], [], [], []
        T = 0
        for seq in seqs:
            if not seq.prompt_token_ids:
                self.tokenize(seq)
            ids = np.asarray(seq.prompt_token_ids, dtype=np.int64)
            L = int(ids.shape[0])
            if L == 0 or L >= self._pool.max_len:
                raise ValueError(f"prompt length {L} outside [1, max_len={self._pool.max_len})")
            images = seq.request.images
            grids = [im.grid for im in images] if images else None
            if images:
                # the image rows located on the host: a mask on the device would make the
                # host wait for the queue (its count, its nonzero rows)
                rows = np.flatnonzero(ids == self.image_token_id)
                v = self.adapter.vision_embed(images)
                if rows.shape[0] != v.shape[0]:
                    raise ValueError("image token count does not match the vision rows")
                img_rows.append(rows + T)
                vis.append(v)
            pos, delta = self.adapter.prefill_positions(ids, grids)
            ids_l.append(ids)
            pos_l.append(pos.numpy() if isinstance(pos, torch.Tensor) else np.asarray(pos))
            seg_lens.append(L)
            deltas.append(int(delta))
            T += L
        slots = [base + i for i in range(len(seqs))]
        nr = sum(int(r.shape[0]) for r in img_rows)
        host = np.concatenate(ids_l + img_rows + [np.concatenate(pos_l, axis=1).reshape(-1),
                                                  np.asarray(deltas, dtype=np.int64)])
        up = to_device(torch.from_numpy(host), torch.int64, dev)
        emb = self.adapter.embed_tokens(up[:T])
        if img_rows:
            emb.index_copy_(0, up[T:T + nr], torch.cat(vis, 0).to(emb.dtype))
        packed = emb.unsqueeze(0)
        pos = up[T + nr:T + nr + 3 * T].view(3, 1, T)                           # [3, 1, T]
        if self._use_graph and self.prefill_graph_layouts > 0:
            logits = self._prefill_graphed(packed, pos, slots, seg_lens)
        else:
            last = torch.tensor(seg_lens).cumsum(0) - 1
            cache = self._pool.packed_prefill_cache(slots, seg_lens)
            logits = self.adapter.llm(packed, pos, None, cache, logits_indices=last.tolist())[0]
        self._rope_delta[base:base + len(seqs)].copy_(up[T + nr + 3 * T:])
        toks = self._sample_rows(logits, seqs)
        for i, seq in enumerate(seqs):
            slot = slots[i]
            self._slot_seq.append(seq)
            self._kv_len.append(seg_lens[i])
            seq.kv_handle = {"slot": slot, "rope_delta": deltas[i]}
            seq.append_token(toks[i])
            seq.maybe_finish()
        self._dev_ids_for = None

    # Packed prefills run as HIP graphs keyed by their segment lengths (with use_graph): the
    # first prefill of a layout runs eagerly on the layout's static input buffers and is then
    # captured; a later prefill of the same layout copies its embeddings, positions and slots
    # into those buffers and replays.  Token positions, query blocks and new lengths depend
    # only on the layout; the slot of every token is rewritten on the device before a replay.
    # Up to this many layouts are kept (least recently used dropped); 0 disables.
    prefill_graph_layouts = 4

    def drop_prefill_graphs(self) -> None:
        """Forget the captured prefill graphs.  They launch on the device addresses of the
        weights they were captured with, so call this after replacing weight tensors (a
        GPTQ linear's release_f16 is noticed by itself: see _prefill_graphed)."""
        self._prefill_graphs.clear()

    def _prefill_graphed(self, packed, pos, slots, seg_lens):
        key = tuple(int(L) for L in seg_lens)
        graphs = self._prefill_graphs
        epoch = weights_epoch()
        if epoch != self._prefill_epoch:         # a resident fp16 expansion was released
            graphs.clear()
            self._prefill_epoch = epoch
        ent = graphs.pop(key, None)
        dev = self.device
        if ent is not None:
            graphs[key] = ent                                     # most recently used last
            ent["x"].copy_(packed)
            ent["pos"].copy_(pos)
            if ent["slots"] != slots:
                writer = ent["writer"]
                tok = [s for s, L in zip(slots, key) for _ in range(L)]
                new = to_device(tok + list(slots), torch.int64, dev)
                writer.token_slot.copy_(new[:len(tok)])
                writer._fin_slots.copy_(new[len(tok):])
                writer.slots = list(slots)
                ent["slots"] = list(slots)
            ent["graph"].replay()
            self._pool._active = max(self._pool._active, max(slots) + 1)
            return ent["out"]
        # first prefill of this layout: run it on static buffers, then capture (outside
        # inference mode, as the decode graphs are: a capture made inside it would leave the
        # generator's graph state as inference tensors that later captures cannot update)
        with torch.inference_mode(False):
            last = torch.tensor(key).cumsum(0) - 1
            ent = {"x": packed.clone(), "pos": pos.clone(), "slots": list(slots),
                   "idx": to_device(last, torch.int64, dev),
                   "writer": self._pool.packed_prefill_cache(slots, list(key))}
            run = lambda: self.adapter.llm(ent["x"], ent["pos"], None, ent["writer"],
                                           logits_indices=ent["idx"])[0]
            logits = run().clone()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                ent["out"] = run()
            ent["graph"] = g
        graphs[key] = ent
        while len(graphs) > self.prefill_graph_layouts:
            graphs.pop(next(iter(graphs)))
        return logits

    def attach_prefilled(self, seqs: List[Sequence], lengths: List[int],
                         rope_deltas: List[int] | None = None) -> List[int]:
        """Seat sequences whose KV prefix the caller already wrote into the pool (the
        set_slot_prefix contract, cache/kv_prealloc.py:43-49): each takes the next slot
        with lengths[slot] = L and decodes from there.  Returns the slots."""
        self.settle()
        base = len(self._slot_seq)
        if base + len(seqs) > self.max_running:
            raise RuntimeError("KV pool full")
        slots = []
        for i, (seq, L) in enumerate(zip(seqs, lengths)):
            if not 0 < L < self._pool.max_len:
                raise ValueError(f"length {L} outside (0, max_len)")
            slot = base + i
            d = 0 if rope_deltas is None else int(rope_deltas[i])
            self._pool.lengths[slot] = L
            self._rope_delta[slot] = d
            self._slot_seq.append(seq)
            self._kv_len.append(int(L))
            seq.kv_handle = {"slot": slot, "rope_delta": d}
            slots.append(slot)
        self._dev_ids_for = None
        return slots

    # ---- chunked prefill / mixed batching (multimodal.py:200-284) -------------------
    def _chunk_bounds(self, seq: Sequence):
        self.settle()
        if not seq.prompt_token_ids:
            self.tokenize(seq)
        P = len(seq.prompt_token_ids)
        start, L = seq.num_prefilled, seq.prefill_chunk
        if P == 0 or P >= self._pool.max_len:
            raise ValueError(f"prompt length {P} outside [1, max_len={self._pool.max_len})")
        if L < 1 or start < 0 or start + L > P:
            raise ValueError(f"chunk [{start}, {start + L}) outside the {P}-token prompt")
        if start == 0:
            # positions of the whole prompt once, sliced by later chunks (:212-216)
            if seq.request.images:
                raise AssertionError("chunked prefill supports text-only prompts (no images)")
            pos_full, delta = self.adapter.prefill_positions(seq.prompt_token_ids, None)
            seq.kv_handle = {"slot": self._reserve_slot, "rope_delta": int(delta),
                             "pos_full": pos_full}
        elif not seq.kv_handle or "pos_full" not in seq.kv_handle:
            raise ValueError("a later chunk of a prompt whose first chunk was not run")
        return start, L, start + L, P

    def _seat_prefilled(self, seq: Sequence, length: int, logits_row: torch.Tensor) -> None:
        """Last chunk done: move the reserve slot's KV into the decode region (valid prefix
        only) and emit the first token (:229-235)."""
        slot = len(self._slot_seq)
        if slot >= self.max_running:
            raise RuntimeError(f"KV pool full: {slot} running")
        delta = seq.kv_handle["rope_delta"]
        self._pool.copy_slot_kv(self._reserve_slot, slot, length)
        self._rope_delta[slot] = delta
        seq.kv_handle = {"slot": slot, "rope_delta": delta}
        self._slot_seq.append(seq)
        self._kv_len.append(length)
        seq.append_token(self._sample_rows(logits_row, [seq])[0])
        seq.maybe_finish()
        self._dev_ids_for = None

    def chunk_prefill(self, seq: Sequence) -> None:
        """One chunk [num_prefilled, num_prefilled + prefill_chunk) of a long text prompt
        (multimodal.py:200-235): appended to the reserve slot, attending to the chunks
        before it; after the last chunk the sequence joins the decode slots and emits its
        first token."""
        with torch.inference_mode():
            start, L, end, P = self._chunk_bounds(seq)
            dev = self.device
            ids = to_device(seq.prompt_token_ids[start:end], torch.int64, dev)
            emb = self.adapter.embed_tokens(ids).unsqueeze(0)                 # [1, L, H]
            pos = to_device(seq.kv_handle["pos_full"][:, start:end], torch.int64,
                            dev).unsqueeze(1)                                 # [3, 1, L]
            cache = self._pool.chunked_prefill_cache(self._reserve_slot, start)
            logits = self.adapter.llm(emb, pos, None, cache, logits_indices=[L - 1])[0]
            seq.num_prefilled = end
            if end == P:
                self._seat_prefilled(seq, end, logits[0:1])

    def mixed_step(self, chunk_seq: Sequence, decode_seqs: List[Sequence]) -> None:
        """Mixed batching (multimodal.py:237-284): the running sequences' decode tokens and
        one prefill chunk in a single forward - decode tokens first, the chunk after; each
        segment appends to its own slot and attends to its own KV."""
        with torch.inference_mode():
            decode_seqs = sorted(decode_seqs, key=lambda s: s.kv_handle["slot"])
            n = len(decode_seqs)
            if [s.kv_handle["slot"] for s in decode_seqs] != list(range(n)):
                raise AssertionError("mixed_step expects the running sequences in slots [0, n)")
            for b in range(n):
                if self._kv_len[b] >= self._pool.max_len:
                    raise RuntimeError(f"sequence in slot {b} reached max_len={self._pool.max_len}")
            start, L, end, P = self._chunk_bounds(chunk_seq)
            dev = self.device
            dec_len = [int(v) for v in self._kv_len[:n]]        # write positions = KV lengths
            ids = [s.last_token_id() for s in decode_seqs] + chunk_seq.prompt_token_ids[start:end]
            emb = self.adapter.embed_tokens(
                to_device(ids, torch.int64, dev)).unsqueeze(0)                   # [1, n+L, H]
            dec_pos = torch.tensor([dec_len[b] + int(s.kv_handle["rope_delta"])
                                    for b, s in enumerate(decode_seqs)], dtype=torch.int64)
            pos = torch.cat([dec_pos.view(1, n).expand(3, n),
                             chunk_seq.kv_handle["pos_full"][:, start:end].to(torch.int64)], 1)
            pos = to_device(pos, torch.int64, dev).unsqueeze(1)                   # [3, 1, n+L]
            cache = self._pool.mixed_cache(list(range(n)) + [self._reserve_slot],
                                           [1] * n + [L], dec_len + [start])
            final = end == P
            idx = list(range(n)) + ([n + L - 1] if final else [])
            logits = self.adapter.llm(emb, pos, None, cache, logits_indices=idx)[0]
            self._dev_ids_for = None
            if n:
                self._emit(decode_seqs, self._sample_rows(logits[:n], decode_seqs))
            chunk_seq.num_prefilled = end
            if final:
                self._seat_prefilled(chunk_seq, end, logits[n:n + 1])

    def decode(self, seqs: List[Sequence]) -> None:
        seqs = sorted(seqs, key=lambda s: s.kv_handle["slot"])
        n = len(seqs)
        if n == 0:
            return
        if [s.kv_handle["slot"] for s in seqs] != list(range(n)):
            raise AssertionError("decode expects the running sequences in slots [0, n)")
        for b in range(n):
            if self._kv_len[b] >= self._pool.max_len:
                raise RuntimeError(f"sequence in slot {b} reached max_len={self._pool.max_len}")
        greedy = all(s.request.sampling.greedy for s in seqs)
        fused = self.adapter.model.fused_decode_ready()
        if self._use_graph and fused:
            if greedy:
                self._decode_graph(seqs, n)
            else:
                self._decode_graph_sampled(seqs, n)
        else:
            self.settle()
            with torch.inference_mode():
                if fused:
                    self._decode_eager(seqs, n, greedy)
                else:
                    self._decode_forward(seqs, n)

    # ---- decode paths ----------------------------------------------------------------
    def _load_ids(self, seqs, n, dst: torch.Tensor) -> None:
        key = tuple(id(s) for s in seqs)
        if self._dev_ids_for == key:
            return                      # dst already holds the last step's outputs
        for b, s in enumerate(seqs):
            self._pinned_ids[b] = s.last_token_id()
        dst.copy_(self._pinned_ids[:n], non_blocking=True)

    def _decode_eager(self, seqs, n, greedy: bool):
        model = self.adapter.model
        if n not in self._eager:
            self._eager[n] = {
                "ids": torch.zeros(n, dtype=torch.int64, device=self.device),
                "out": torch.zeros(n, dtype=torch.int64, device=self.device),
                "logits": torch.empty(n, model.cfg.vocab_size, device=self.device,
                                      dtype=torch.float16),
            }
        b = self._eager[n]
        self._dev_ids_for = None
        self._load_ids(seqs, n, b["ids"])
        view = self._pool.view(n, self._rope_delta)
        model.decode_greedy(b["ids"], view, b["out"], None if greedy else b["logits"],
                            lengths=self._pool.lengths)
        if greedy:
            self._emit(seqs, b["out"].tolist())
        else:
            self._emit(seqs, self._sample_rows(b["logits"], seqs))

    def _decode_forward(self, seqs, n):
        """Decode through the model's forward (multimodal.py:286-313, eager): for linears
        the fused step cannot run (FP8 W8A8 modules, an fp8_out norm), the reference's
        per-op route - one token per row appended at its length, logits, then sampling."""
        model = self.adapter.model
        self._dev_ids_for = None
        ids = to_device([s.last_token_id() for s in seqs], torch.int64, self.device)
        emb = model.embed_tokens(ids).unsqueeze(1)                       # [n, 1, H]
        view = self._pool.view(n, self._rope_delta)
        pos = self.adapter.decode_positions(self._pool.lengths[:n], self._rope_delta[:n])
        logits = self.adapter.llm(emb, pos, None, view)[:, -1, :]
        self._emit(seqs, self._sample_rows(logits, seqs))

    def _capture_graph(self, n, sampled: bool = False):
        """Capture the step for rows [0, n).  Greedy: the final launch advances lengths[:n]
        and leaves the new ids in bufs["ids"] as the next step's input.  ``sampled``: the
        step also writes the fp16 logits to bufs["logits"] (the host samples from them and
        loads the next ids itself)."""
        model = self.adapter.model
        bufs = {"ids": torch.zeros(n, dtype=torch.int64, device=self.device),
                "out": torch.zeros(n, dtype=torch.int64, device=self.device)}
        if sampled:
            bufs["logits"] = torch.empty(n, model.cfg.vocab_size, device=self.device,
                                         dtype=torch.float16)
        view = self._pool.view(n, self._rope_delta)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):   # warm-up: writes K/V at the (not yet valid) next position only
                model.decode_greedy(bufs["ids"], view, bufs["out"], bufs.get("logits"))
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            model.decode_greedy(bufs["ids"], view, bufs["out"], bufs.get("logits"),
                                next_ids=None if sampled else bufs["ids"],
                                lengths=self._pool.lengths)
        # the view and buffers are referenced by the graph: keep them alive with it
        (self._graphs_sampled if sampled else self._graphs)[n] = (g, bufs, view)

    def _decode_graph_sampled(self, seqs, n):
        """A batch with non-greedy rows in graph mode (multimodal.py:306-313, 342-357):
        replay the step graph that also captures the logits, then sample every row from
        them on the host side of the step (greedy rows take the argmax, as _sample_rows
        does for the eager paths)."""
        self.settle()
        if n not in self._graphs_sampled:
            self._capture_graph(n, sampled=True)
        g, bufs, _view = self._graphs_sampled[n]
        self._dev_ids_for = None               # the next ids come from the host
        self._load_ids(seqs, n, bufs["ids"])
        g.replay()
        self._emit(seqs, self._sample_rows(bufs["logits"], seqs))

    def _launch(self, n: int) -> int:
        """Replay the step graph for rows [0, n) (inputs: bufs["ids"]) and start the new
        ids' copy to a pinned buffer; returns the buffer index."""
        g, bufs, _view = self._graphs[n]
        g.replay()
        i = self._pin_next
        self._pin_next ^= 1
        self._pinned_out[i][:n].copy_(bufs["out"], non_blocking=True)
        self._out_ready[i].record()
        return i

    def _decode_graph(self, seqs, n):
        key = tuple(id(s) for s in seqs)
        if self._ahead is not None and self._ahead[0] == key:
            cur = self._ahead[2]               # enqueued by the previous call
            self._ahead = None
        else:
            self.settle()
            if n not in self._graphs:
                self._capture_graph(n)
            self._load_ids(seqs, n, self._graphs[n][1]["ids"])
            cur = self._launch(n)
        # The next step goes out before this one is waited for, when the batch will decode
        # again as is unless this step finishes someone (nobody has finished, every row has
        # room): its inputs are this step's ids, which the graph leaves on the device.  If
        # this step does finish a sequence, the caller's free() takes the next one back.
        if (all(s.status not in (Status.FINISHED, Status.ABORTED) for s in seqs)
                and all(self._kv_len[b] + 1 < self._pool.max_len for b in range(n))):
            self._ahead = (key, n, self._launch(n))
        self._out_ready[cur].synchronize()
        toks = self._pinned_out[cur][:n].tolist()
        self._emit(seqs, toks)
        self._dev_ids_for = key

    def _emit(self, seqs, toks):
        for b, seq in enumerate(seqs):
            self._kv_len[b] += 1
            seq.append_token(int(toks[b]))
            seq.maybe_finish()

    def _sample_rows(self, logits: torch.Tensor, seqs) -> List[int]:
        """Greedy = argmax of the fp16 logits (multimodal.py:374-377); else temperature
        sampling."""
        out = []
        greedy_rows = logits.argmax(-1).tolist()      # first maximum, as on the fp32 copy
        for i, seq in enumerate(seqs):
            sp = seq.request.sampling
            if sp.greedy:
                out.append(int(greedy_rows[i]))
            else:
                probs = torch.softmax(logits[i].float() / sp.temperature, dim=-1)
                out.append(int(torch.multinomial(probs, 1).item()))
        return out

    # ---- release ----------------------------------------------------------------------
    def free(self, seq: Sequence) -> None:
        """Swap-compact the pool (multimodal.py:359-369): the last slot's sequence moves
        into the freed slot; only its valid KV prefix is copied."""
        self.settle()
        h = seq.kv_handle or {}
        slot = h.get("slot")
        if slot is None:
            return
        last = len(self._slot_seq) - 1
        if slot != last:
            L = self._kv_len[last]
            self._pool.copy_slot_kv(last, slot, L)
            self._rope_delta[slot] = self._rope_delta[last]
            moved = self._slot_seq[last]
            moved.kv_handle["slot"] = slot
            self._slot_seq[slot] = moved
            self._kv_len[slot] = L
        self._slot_seq.pop()
        self._kv_len.pop()
        self._dev_ids_for = None

    def detokenize(self, seq: Sequence, new_token_ids: List[int]) -> str:
        return self.adapter.detokenize(new_token_ids)


class NativeQwenVLRunner(MultimodalRunner):
    """Entry point with the reference's constructor (runners/qwen_vl_native.py:14-20).
    Extra keyword arguments go to the adapter (weights=, seed=, num_layers=, ...)."""

    def __init__(self, model_dir: str = None, max_running: int = 32, max_len: int = 1024,
                 prefix_cache=None, quant: str = None, gptq_dir: str = None,
                 use_graph: bool = False, **adapter_kwargs):
        from .adapter import Qwen2VLAdapter
        adapter = Qwen2VLAdapter(model_dir=model_dir, quant=quant, gptq_dir=gptq_dir,
                                 max_pos=max(8192, 2 * max_len), **adapter_kwargs)
        super().__init__(adapter, max_running=max_running, max_len=max_len,
                         prefix_cache=prefix_cache, use_graph=use_graph)
