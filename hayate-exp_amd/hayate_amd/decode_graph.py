"""Decode ticks replayed from captured HIP graphs.

A serving loop spends most of a decode tick launching small kernels: 36
layers of projections, norms, the fused decode attention and its merge,
the MLP. Every launch on this path enqueues only (no host synchronisation,
no allocation inside the kernels, fixed argument pointers), so a whole
36-layer decode forward can be captured once as a HIP graph and replayed
every tick. What changes from tick to tick is data: the token ids, the
page table, the lengths and the planner's work lists. ``StaticDecodeBatch``
keeps all of it in device buffers that never move and rewrites them in
place (one host-to-device copy per tick); the graph captured over one tick
then computes the next.

The decode grid is part of the captured launch, so it is fixed at the
largest chunk count a plan can have (one chunk per CU and kv head); a
tick whose plan has fewer chunks pads the list with empty chunk records,
whose workgroups leave at once. One graph per batch size therefore serves
every tick. The partial-result workspace and the work-list buffers are
sized for the largest plan of the batch size, and the kernels are told
that size (their workspace layout depends on it), so every tick's plan
fits the captured layout. A graph reads the fused q/k/v weights by
address; if a layer rebuilds them (its projection parameters were
replaced, not updated in place), the graphs are dropped and captured
again.

This is what the reference's ``Engine(compile=True)`` (engine.py:84-90,
torch.compile with CUDA graphs in "reduce-overhead" mode) buys on its path:
here the capture is explicit and covers the decode ticks, whose shapes
repeat; prefill and mixed ticks run eagerly.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np
import torch

from . import _native, attention
from .paged_cache import PagedCacheHandle, PagedKVBatch, PagedKVCacheManager, _require_hip


class _StaticPlan:
    """Decode work lists in fixed device buffers (the attributes of a tick's
    plan that the decode calls read)."""

    n_prefill = 0
    n_prefill_merge = 0
    n_prefill_slots = 0
    prefill_ptr = None
    prefill_merge_ptr = None
    prefill_workspace_ptr = None
    prefill_workspace_bytes = 0


class StaticDecodeBatch(PagedKVBatch):
    """A decode-only varlen batch of ``batch_size`` sequences whose device
    metadata lives in buffers that ``refresh`` rewrites in place.

    Layout: one int32 device buffer holding the page table (batch_size x
    max_pages, -1 padded), cache_lens, kv_lens, q_start, the decode records
    (chunks then pieces, 8 int32 each, up to ``record_capacity``) and the
    merge items (4 int32 per sequence); plus an fp32 workspace for
    ``slot_capacity`` partial slots."""

    def __init__(self, manager: PagedKVCacheManager, batch_size: int, num_q_heads: int,
                 max_tokens: int):
        _require_hip(manager.k_cache, "StaticDecodeBatch")
        if batch_size < 1:
            raise ValueError("batch_size must be positive")
        B = batch_size
        self.k_cache = manager.k_cache
        self.v_cache = manager.v_cache
        self.page_size = manager.page_size
        self.device = manager.device
        self.num_kv_heads = manager.num_kv_heads
        self.head_dim = manager.head_dim
        self.varlen = True
        self.q_lens = [1] * B
        self.num_seqs = B
        self.total_tokens = B
        self.query_len = None
        self.tokens_per_split = manager.tokens_per_split
        self._num_cus = manager.num_cus
        self._pool_ptrs: dict = {}
        self.launch_hook = None
        self._manager = manager
        self.num_q_heads = num_q_heads
        # a sequence never needs more pages than its longest context
        self.max_pages = max(1, min(manager.num_pages, math.ceil(max_tokens / self.page_size)))
        # decode records: at most one chunk per CU and kv head, and a piece per
        # (sequence, chunk) overlap: every cut adds at most one piece
        self.max_chunks = max(1, self._num_cus // self.num_kv_heads) if self._num_cus else 32
        self.record_capacity = 2 * self.max_chunks + B + 8
        # partial slots per piece, as the planner assigns them
        probe = _native.plan_tick(np.ones(1, dtype=np.int32), np.ones(1, dtype=np.int32),
                                  num_q_heads, self.num_kv_heads, self.page_size, 0, 0)
        slots_per_piece = probe.n_slots // max(1, len(probe.decode) - probe.n_chunks)
        self.slot_capacity = slots_per_piece * (self.max_chunks + B + 8)
        n_table = B * self.max_pages
        self._off_cache = n_table
        self._off_kv = n_table + B
        self._off_qs = n_table + 2 * B
        self._off_dec = n_table + 3 * B + 1
        self._off_merge = self._off_dec + 8 * self.record_capacity
        total = self._off_merge + 4 * B
        self._host = torch.empty(total, dtype=torch.int32, pin_memory=True)
        self._host_np = self._host.numpy()
        self._copied = None  # event after the last host-to-device copy
        self._dev = torch.zeros(total, dtype=torch.int32, device=self.device)
        d = self._dev
        self.page_table = d[:n_table].view(B, self.max_pages)
        self.cache_lens_i32 = d[self._off_cache : self._off_cache + B]
        self.kv_lens = d[self._off_kv : self._off_kv + B]
        self.q_start = d[self._off_qs : self._off_qs + B + 1]
        self.cache_lens = torch.zeros(B, dtype=torch.long, device=self.device)
        self._pt_ptr = self.page_table.data_ptr()
        self._pt_stride = self.page_table.stride(0)
        self._q_start_ptr = self.q_start.data_ptr()
        self._cache_lens_ptr = self.cache_lens_i32.data_ptr()
        self._kv_lens_ptr = self.kv_lens.data_ptr()
        plan = _StaticPlan()
        plan.decode = d[self._off_dec : self._off_merge]
        plan.merge = d[self._off_merge : total]
        plan.decode_ptr = plan.decode.data_ptr()
        plan.merge_ptr = plan.merge.data_ptr()
        plan.n_merge = B
        plan.n_slots = self.slot_capacity
        plan.workspace_bytes = _native.decode_workspace_bytes(self.slot_capacity, num_q_heads,
                                                              self.head_dim)
        plan.workspace = torch.empty(plan.workspace_bytes // 4, dtype=torch.float32,
                                     device=self.device)
        plan.workspace_ptr = plan.workspace.data_ptr()
        plan.n_decode = 0
        self._plan = plan
        self._plans = {num_q_heads: plan}
        self._max_kv = 0
        self.cache_lens_host: list[int] = []
        self.kv_lens_host: list[int] = []

    def plan(self, num_q_heads: int):
        if num_q_heads != self.num_q_heads:
            raise ValueError("a static decode batch is planned for one query-head count")
        return self._plan

    def refresh(self, handles: Sequence[PagedCacheHandle]) -> bool:
        """Rewrites the metadata and work lists for `handles` (whose append
        space is reserved) and enqueues the copy on the current stream.
        Returns False, changing nothing, when the tick does not fit the
        buffers (more pages per sequence, records or slots than sized)."""
        B = self.num_seqs
        if len(handles) != B:
            raise ValueError(f"static decode batch holds {B} sequences, got {len(handles)}")
        cache = [h.length for h in handles]
        kv = [c + 1 for c in cache]
        if any(len(h.pages) > self.max_pages for h in handles):
            return False
        host = _native.plan_tick(np.ones(B, dtype=np.int32), np.asarray(kv, dtype=np.int32),
                                 self.num_q_heads, self.num_kv_heads, self.page_size,
                                 self._num_cus, self.tokens_per_split)
        n_pieces = len(host.decode) - host.n_chunks
        if (host.n_chunks > self.max_chunks or self.max_chunks + n_pieces > self.record_capacity
                or host.n_slots > self.slot_capacity or len(host.merge) != B):
            return False
        if self._copied is not None:
            self._copied.synchronize()  # the staging buffer is free again
        buf = self._host_np
        table = buf[: B * self.max_pages].reshape(B, self.max_pages)
        table.fill(-1)
        for row, h in enumerate(handles):
            table[row, : len(h.pages)] = h.pages
        buf[self._off_cache : self._off_cache + B] = cache
        buf[self._off_kv : self._off_kv + B] = kv
        buf[self._off_qs : self._off_qs + B + 1] = np.arange(B + 1, dtype=np.int32)
        # chunk records, empty ones up to the fixed grid, then the pieces
        # (the kernel finds them after max_chunks records)
        nc = host.n_chunks
        dec = buf[self._off_dec : self._off_merge].reshape(-1, 8)
        dec[:nc] = host.decode[:nc]
        dec[nc : self.max_chunks] = 0
        dec[nc : self.max_chunks, 0:2] = n_pieces  # piece_begin == piece_end: empty
        dec[self.max_chunks : self.max_chunks + n_pieces] = host.decode[nc:]
        buf[self._off_merge : self._off_merge + 4 * B] = host.merge.reshape(-1)
        self._dev.copy_(self._host, non_blocking=True)
        self._copied = torch.cuda.Event()
        self._copied.record()
        self.cache_lens.copy_(self.cache_lens_i32, non_blocking=True)
        self._table_np = table
        self._plan.n_decode = self.max_chunks
        self.cache_lens_host = cache
        self.kv_lens_host = kv
        self._max_kv = max(kv)
        return True


class DecodeGraphRunner:
    """Captures and replays decode ticks of one model over one pool.

    ``run(handles, token_ids)`` returns the logits of one token per
    sequence (B, 1, vocab) for handles whose append space the caller has
    reserved, or None when the tick must run eagerly (it does not fit the
    static buffers)."""

    def __init__(self, model, manager: PagedKVCacheManager, max_tokens: int):
        self.model = model
        self.manager = manager
        self.max_tokens = max_tokens
        self._states: dict[int, dict] = {}
        self.captures = 0
        self.replays = 0

    def _state(self, batch_size: int) -> dict:
        st = self._states.get(batch_size)
        if st is None:
            st = {
                "batch": StaticDecodeBatch(self.manager, batch_size, self.model.num_heads,
                                           self.max_tokens),
                "ids": torch.zeros((1, batch_size), dtype=torch.long, device=self.manager.device),
                "graph": None,
            }
            self._states[batch_size] = st
        return st

    def drop_graphs(self) -> None:
        """Forgets every captured graph (their memory pools go with them)."""
        for st in self._states.values():
            st["graph"] = None

    def _forward(self, st):
        with torch.inference_mode():
            return self.model(st["ids"], paged_cache=st["batch"])[0]

    def run(self, handles: Sequence[PagedCacheHandle], token_ids: Sequence[int]
            ) -> Optional[torch.Tensor]:
        st = self._state(len(handles))
        batch = st["batch"]
        if not batch.refresh(handles):
            return None
        rope_rows = self.model.cos.shape[0] if self.model.cos is not None else 0
        if batch._max_kv > rope_rows:
            return None  # let the eager path raise its error
        st["ids"].copy_(torch.tensor(token_ids, dtype=torch.long).view(1, -1),
                        non_blocking=True)
        entry = st["graph"]
        if entry is not None and entry[2] != attention.qkv_rebuilds:
            self.drop_graphs()  # a fused q/k/v weight moved: recapture
            entry = None
        if entry is None:
            stream = torch.cuda.current_stream()
            side = torch.cuda.Stream()
            side.wait_stream(stream)
            with torch.cuda.stream(side):
                self._forward(st)  # warm-up: writes this tick's K/V rows (replays rewrite them)
            stream.wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                logits = self._forward(st)
            # the warm-up and the capture may build fused weights: key on
            # the count after them
            entry = (graph, logits, attention.qkv_rebuilds)
            st["graph"] = entry
            self.captures += 1
        graph, logits, _ = entry
        graph.replay()
        self.replays += 1
        return logits
