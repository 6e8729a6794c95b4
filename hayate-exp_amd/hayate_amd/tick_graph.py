"""Engine ticks replayed from captured HIP graphs.

A serving loop spends much of a tick launching kernels: 36 layers of
projections, norms, the attention calls and the MLP. Every launch on this
path only enqueues (no host synchronisation, no allocation inside the
kernels, fixed argument pointers), so a whole 36-layer forward can be
captured once as a HIP graph and replayed. What changes from one tick of a
shape to the next is data: the token ids, the page table, the lengths and
the planner's work lists. ``StaticTickBatch`` keeps all of it in device
buffers that never move and rewrites them in place (one host-to-device copy
per tick); the graph captured over one tick then computes the next tick of
the same shape.

A tick's shape is the tuple of its query lengths (1 for a decode token, the
chunk length for a prompt chunk). It fixes the token count, the GEMM shapes
and where each sequence's rows sit. The work lists vary with the cached
lengths, so their launches are captured at fixed sizes:

- decode: the grid is the largest chunk count a plan can have (one chunk
  per CU and kv head); a plan with fewer chunks pads the list with empty
  chunk records, whose workgroups leave at once;
- prefill: the item and merge lists are padded with empty records (the
  kernels skip a record whose query range is empty). A prefill item list
  holds at most one item per unsplit query tile plus one per partial slot,
  and a merge list one record per query tile, so both are sized from the
  shape's tile count and a partial-slot capacity: the first plan's slots
  plus one per tile. A later plan that needs more slots rebuilds the batch
  and captures again.

The partial-result workspaces are sized for those capacities, and the
kernels are told them (their workspace layouts depend on them).

Decode shapes (every length 1) repeat tick after tick and are captured the
first time they are seen. A shape with prompt chunks is captured the second
time: a chunk length that occurs once (a prompt's last chunk) runs eagerly
instead of paying for a capture that would never be replayed. At most
``max_graphs`` graphs are kept, the least recently used leaving first. A
graph reads the fused q/k/v weights by address; if a layer rebuilds them
(its projection parameters were replaced, not updated in place), every
graph is dropped and captured again.

This is what the reference's ``Engine(compile=True)`` (engine.py:84-90,
torch.compile with CUDA graphs in "reduce-overhead" mode) buys on its path;
here the capture is explicit.
"""

from __future__ import annotations

import math
from collections import OrderedDict
from typing import Optional, Sequence

import numpy as np
import torch

from . import _native, attention
from .paged_cache import PagedCacheHandle, PagedKVBatch, PagedKVCacheManager, _require_hip


def _prefill_tiles(q_lens: Sequence[int], num_q_heads: int, num_kv_heads: int) -> int:
    """Query tiles of the prompt chunks (q_len > 1), as the planner cuts them."""
    tile = max(1, int(_native.lib().hy_prefill_tile_rows()) // (num_q_heads // num_kv_heads))
    return sum(-(-q // tile) for q in q_lens if q > 1)


def _plan_for(manager: PagedKVCacheManager, q_lens: Sequence[int], num_q_heads: int,
              handles: Sequence[PagedCacheHandle]) -> "_native.TickPlan":
    """The planner's work lists for `handles` appending `q_lens` tokens."""
    kv = [h.length + q for h, q in zip(handles, q_lens)]
    return _native.plan_tick(np.asarray(q_lens, dtype=np.int32), np.asarray(kv, dtype=np.int32),
                             num_q_heads, manager.num_kv_heads, manager.page_size,
                             manager.num_cus, manager.tokens_per_split)


class _StaticPlan:
    """A tick's work lists in fixed device buffers, at their padded launch
    sizes (the attributes of a plan that the attention calls read)."""

    n_decode = 0
    n_merge = 0
    n_slots = 0
    decode_ptr = None
    merge_ptr = None
    workspace_ptr = None
    workspace_bytes = 0
    n_prefill = 0
    n_prefill_merge = 0
    n_prefill_slots = 0
    prefill_ptr = None
    prefill_merge_ptr = None
    prefill_workspace_ptr = None
    prefill_workspace_bytes = 0


class StaticTickBatch(PagedKVBatch):
    """A varlen tick of one shape (``q_lens``) whose device metadata lives in
    buffers that ``refresh`` rewrites in place.

    Layout: one int32 device buffer holding the page table (B x max_pages,
    -1 padded), cache_lens, kv_lens, q_start, the decode records (chunks
    then pieces, 8 int32 each), the decode merge items (4 int32 per decode
    sequence), the prefill items and the prefill merge items (8 int32
    each); plus fp32 workspaces for the decode and prefill partial slots.
    ``prefill_slots`` is the prefill partial-slot capacity."""

    def __init__(self, manager: PagedKVCacheManager, q_lens: Sequence[int], num_q_heads: int,
                 max_tokens: int, prefill_slots: int = 0):
        _require_hip(manager.k_cache, "StaticTickBatch")
        q_lens = [int(q) for q in q_lens]
        if not q_lens or min(q_lens) < 1:
            raise ValueError("a tick needs sequences with positive query lengths")
        if num_q_heads % manager.num_kv_heads:
            raise ValueError("query heads must be a multiple of kv heads")
        B = len(q_lens)
        self.k_cache = manager.k_cache
        self.v_cache = manager.v_cache
        self.page_size = manager.page_size
        self.device = manager.device
        self.num_kv_heads = manager.num_kv_heads
        self.head_dim = manager.head_dim
        self.varlen = True
        self.q_lens = q_lens
        self.num_seqs = B
        self.total_tokens = sum(q_lens)
        self.query_len = None
        self.tokens_per_split = manager.tokens_per_split
        self._num_cus = manager.num_cus
        self._pool_ptrs: dict = {}
        self.launch_hook = None
        self.num_q_heads = num_q_heads
        # a sequence never needs more pages than its longest context
        self.max_pages = max(1, min(manager.num_pages, math.ceil(max_tokens / self.page_size)))

        n_dec = sum(1 for q in q_lens if q == 1)
        if n_dec:
            # at most one chunk per CU and kv head, and a piece per
            # (sequence, chunk) overlap: every cut adds at most one piece
            self.max_chunks = max(1, self._num_cus // self.num_kv_heads) if self._num_cus else 32
            self.record_capacity = 2 * self.max_chunks + n_dec + 8
            # partial slots per piece, as the planner assigns them
            probe = _native.plan_tick(np.ones(1, dtype=np.int32), np.ones(1, dtype=np.int32),
                                      num_q_heads, self.num_kv_heads, self.page_size, 0, 0)
            slots_per_piece = probe.n_slots // max(1, len(probe.decode) - probe.n_chunks)
            self.slot_capacity = slots_per_piece * (self.max_chunks + n_dec + 8)
        else:
            self.max_chunks = self.record_capacity = self.slot_capacity = 0
        self.n_decode_seqs = n_dec
        self._manager = manager
        self.n_tiles = _prefill_tiles(q_lens, num_q_heads, self.num_kv_heads)
        self.prefill_slot_capacity = max(0, int(prefill_slots)) if self.n_tiles else 0
        # items: one per unsplit tile plus one per partial slot
        self.prefill_capacity = self.n_tiles + self.prefill_slot_capacity if self.n_tiles else 0
        # set by refresh when a plan needed more prefill partial slots
        self.prefill_slots_needed = 0

        n_table = B * self.max_pages
        self._off_cache = n_table
        self._off_kv = n_table + B
        self._off_qs = n_table + 2 * B
        self._off_dec = n_table + 3 * B + 1
        self._off_merge = self._off_dec + 8 * self.record_capacity
        self._off_pre = self._off_merge + 4 * n_dec
        self._off_pmerge = self._off_pre + 8 * self.prefill_capacity
        total = self._off_pmerge + 8 * self.n_tiles
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
        # query rows never move within a shape
        self._host_np[self._off_qs] = 0
        self._host_np[self._off_qs + 1 : self._off_qs + B + 1] = np.cumsum(q_lens)

        plan = _StaticPlan()
        if n_dec:
            plan.decode = d[self._off_dec : self._off_merge]
            plan.merge = d[self._off_merge : self._off_pre]
            plan.decode_ptr = plan.decode.data_ptr()
            plan.merge_ptr = plan.merge.data_ptr()
            plan.n_decode = self.max_chunks
            plan.n_merge = n_dec
            plan.n_slots = self.slot_capacity
            plan.workspace_bytes = _native.decode_workspace_bytes(self.slot_capacity, num_q_heads,
                                                                  self.head_dim)
            plan.workspace = torch.empty(plan.workspace_bytes // 4, dtype=torch.float32,
                                         device=self.device)
            plan.workspace_ptr = plan.workspace.data_ptr()
        if self.n_tiles:
            plan.prefill = d[self._off_pre : self._off_pmerge]
            plan.prefill_merge = d[self._off_pmerge : total]
            plan.prefill_ptr = plan.prefill.data_ptr()
            plan.prefill_merge_ptr = plan.prefill_merge.data_ptr()
            plan.n_prefill = self.prefill_capacity
            plan.n_prefill_merge = self.n_tiles
            plan.n_prefill_slots = self.prefill_slot_capacity
            plan.prefill_workspace_bytes = _native.prefill_workspace_bytes(
                self.prefill_slot_capacity, self.num_kv_heads, self.head_dim)
            if plan.prefill_workspace_bytes:
                plan.prefill_workspace = torch.empty(plan.prefill_workspace_bytes // 4,
                                                     dtype=torch.float32, device=self.device)
                plan.prefill_workspace_ptr = plan.prefill_workspace.data_ptr()
        self._plan = plan
        self._plans = {num_q_heads: plan}
        self._max_kv = 0
        self.cache_lens_host: list[int] = []
        self.kv_lens_host: list[int] = []

    def plan(self, num_q_heads: int):
        if num_q_heads != self.num_q_heads:
            raise ValueError("a static tick batch is planned for one query-head count")
        return self._plan

    def refresh(self, handles: Sequence[PagedCacheHandle],
                host: Optional["_native.TickPlan"] = None) -> bool:
        """Rewrites the metadata and work lists for `handles` (whose append
        space is reserved) and enqueues the copy on the current stream.
        Returns False, changing nothing, when the tick does not fit the
        buffers (more pages per sequence, records or slots than sized); if
        only the prefill partial slots ran short, ``prefill_slots_needed``
        then says how many the plan needs. `host` is the plan of `handles`
        when the caller already has it."""
        B = self.num_seqs
        if len(handles) != B:
            raise ValueError(f"static tick batch holds {B} sequences, got {len(handles)}")
        cache = [h.length for h in handles]
        kv = [c + q for c, q in zip(cache, self.q_lens)]
        if any(len(h.pages) > self.max_pages for h in handles):
            return False
        if host is None:
            host = _plan_for(self._manager, self.q_lens, self.num_q_heads, handles)
        n_pieces = len(host.decode) - host.n_chunks
        if (host.n_chunks > self.max_chunks or self.max_chunks + n_pieces > self.record_capacity
                or host.n_slots > self.slot_capacity or len(host.merge) != self.n_decode_seqs):
            return False
        if len(host.prefill_merge) > self.n_tiles:
            return False
        if (host.n_prefill_slots > self.prefill_slot_capacity
                or len(host.prefill) > self.prefill_capacity):
            self.prefill_slots_needed = host.n_prefill_slots
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
        if self.n_decode_seqs:
            # chunk records, empty ones up to the fixed grid, then the pieces
            # (the kernel finds them after max_chunks records)
            nc = host.n_chunks
            dec = buf[self._off_dec : self._off_merge].reshape(-1, 8)
            dec[:nc] = host.decode[:nc]
            dec[nc : self.max_chunks] = 0
            dec[nc : self.max_chunks, 0:2] = n_pieces  # piece_begin == piece_end: empty
            dec[self.max_chunks : self.max_chunks + n_pieces] = host.decode[nc:]
            buf[self._off_merge : self._off_pre] = host.merge.reshape(-1)
        if self.n_tiles:
            # real records first (the planner's longest-first order), then
            # empty ones (zero query range) up to the fixed launch sizes
            pre = buf[self._off_pre : self._off_pmerge].reshape(-1, 8)
            n_pre = len(host.prefill)
            pre[:n_pre] = host.prefill
            pre[n_pre:] = 0
            pm = buf[self._off_pmerge : self._off_pmerge + 8 * self.n_tiles].reshape(-1, 8)
            n_pm = len(host.prefill_merge)
            pm[:n_pm] = host.prefill_merge
            pm[n_pm:] = 0
        self._dev.copy_(self._host, non_blocking=True)
        self._copied = torch.cuda.Event()
        self._copied.record()
        self.cache_lens.copy_(self.cache_lens_i32, non_blocking=True)
        self._table_np = table
        self.cache_lens_host = cache
        self.kv_lens_host = kv
        self._max_kv = max(kv)
        return True


class StaticDecodeBatch(StaticTickBatch):
    """A decode tick of ``batch_size`` sequences (every query length 1)."""

    def __init__(self, manager: PagedKVCacheManager, batch_size: int, num_q_heads: int,
                 max_tokens: int):
        if batch_size < 1:
            raise ValueError("batch_size must be positive")
        super().__init__(manager, [1] * batch_size, num_q_heads, max_tokens)


class TickGraphRunner:
    """Captures and replays ticks of one model over one pool.

    ``run(handles, q_lens, token_ids)`` returns the logits of each sequence's
    last token (B, 1, vocab) for handles whose append space the caller has
    reserved, or None when the tick must run eagerly (a prompt shape seen
    for the first time, or a tick that does not fit the static buffers)."""

    def __init__(self, model, manager: PagedKVCacheManager, max_tokens: int,
                 max_graphs: int = 8):
        if max_graphs < 1:
            raise ValueError("max_graphs must be positive")
        self.model = model
        self.manager = manager
        self.max_tokens = max_tokens
        self.max_graphs = max_graphs
        self._states: OrderedDict[tuple, dict] = OrderedDict()
        self._seen: OrderedDict[tuple, None] = OrderedDict()  # prompt shapes run once
        self.captures = 0
        self.replays = 0
        self.prompt_replays = 0  # replays of ticks with prompt chunks

    def drop_graphs(self) -> None:
        """Forgets every captured graph (their memory pools go with them)."""
        for st in self._states.values():
            st["graph"] = None

    def _new_state(self, key: tuple, prefill_slots: int) -> dict:
        st = {
            "batch": StaticTickBatch(self.manager, key, self.model.num_heads, self.max_tokens,
                                     prefill_slots=prefill_slots),
            "ids": torch.zeros((1, sum(key)), dtype=torch.long, device=self.manager.device),
            "graph": None,
        }
        self._states[key] = st
        self._states.move_to_end(key)
        while len(self._states) > self.max_graphs:
            self._states.popitem(last=False)
        return st

    def _forward(self, st):
        with torch.inference_mode():
            return self.model(st["ids"], paged_cache=st["batch"])[0]

    def run(self, handles: Sequence[PagedCacheHandle], q_lens: Sequence[int],
            token_ids: Sequence[int]) -> Optional[torch.Tensor]:
        key = tuple(int(q) for q in q_lens)
        if len(key) != len(handles) or len(token_ids) != sum(key):
            raise ValueError("one query length per handle and one token id per query row")
        st = self._states.get(key)
        host = None
        if st is None:
            if any(q > 1 for q in key):
                if key not in self._seen:
                    self._seen[key] = None
                    while len(self._seen) > 64:
                        self._seen.popitem(last=False)
                    return None
                del self._seen[key]
            # size the prefill slots from this tick's plan, with room for one
            # more split per query tile
            host = _plan_for(self.manager, key, self.model.num_heads, handles)
            n_tiles = _prefill_tiles(key, self.model.num_heads, self.manager.num_kv_heads)
            st = self._new_state(key, host.n_prefill_slots + n_tiles)
        else:
            self._states.move_to_end(key)
        batch = st["batch"]
        if not batch.refresh(handles, host):
            if not batch.prefill_slots_needed:
                return None
            # more prefill splits than sized: a larger batch and a new capture
            st = self._new_state(key, batch.prefill_slots_needed + batch.n_tiles)
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
        self.prompt_replays += any(q > 1 for q in key)
        return logits
