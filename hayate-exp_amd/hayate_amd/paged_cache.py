"""Paged KV pool, per-tick metadata and the HIP attention calls.

Drop-in counterpart of the reference's hayate/engine/paged_cache.py:
``PagedCacheHandle`` (23-30), ``PagedKVBatch`` (33-71) and
``PagedKVCacheManager`` (74-385) keep their constructor arguments, methods,
attributes and exception types. What changes underneath:

* no FlexAttention BlockMask: a tick is described by an int32 page table,
  int32 ``cache_lens`` / ``kv_lens`` / ``q_start`` and the work lists of the
  native planner (``hy_plan_tick``), shipped to the device in one copy and
  shared by every layer of the forward pass;
* ``write_layer`` / ``attend_layer`` call the HIP kernels through the C ABI
  (``hy_kv_append``, ``hy_paged_decode``, ``hy_paged_prefill``), and the new
  ``norm_rope_write_layer`` fuses the q/k RMSNorm and RoPE of
  hayate/model/attention.py:62-71 with the append;
* pages are reference counted, so requests can share full prefix pages
  (``fork``); a shared page is never written: an append that would land in
  one first copies it (copy-on-write);
* ``begin_tick`` builds one varlen batch that mixes prefill chunks and decode
  tokens (the reference runs them as separate forwards, engine.py:303-312).

Data operations need the pool on a HIP device; on any other device they raise
(the allocator bookkeeping itself works anywhere).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np
import torch

from . import _native
from .cache import Cache
from .constants import MIN_KV_PAGE_SIZE


@dataclass
class PagedCacheHandle:
    """One request's physical KV pages and logical cache length
    (paged_cache.py:23-30)."""

    slot: int
    pages: list[int] = field(default_factory=list)
    length: int = 0
    released: bool = False


class PagedPrefix:
    """The first `length` tokens of a cache as references to its physical
    pages: the zero-copy form of a prefix snapshot (the reference gathers a
    compact copy, paged_cache.py:180-190, and clones it again for the prefix
    cache, prefix_cache.py:72).

    Holding a PagedPrefix keeps its pages alive (one reference each).
    Shared pages are copy-on-write for every handle that appends into them,
    so the tokens a PagedPrefix covers never change: it is as immutable as
    the reference's cloned Cache. It offers the part of the Cache interface
    the prefix cache and the engine use (``length``, ``capacity``,
    ``slice``, ``reset``); ``to_cache()`` gathers a compact Cache copy.
    """

    __slots__ = ("manager", "pages", "_length")

    def __init__(self, manager: "PagedKVCacheManager", pages: list[int], length: int):
        # the caller has already taken one reference per page for this object
        self.manager = manager
        self.pages = pages
        self._length = length

    @property
    def length(self) -> int:
        return self._length

    @property
    def capacity(self) -> int:
        return self._length

    def slice(self, end: int, clone: bool = False) -> "PagedPrefix":
        """The first `end` tokens, sharing the pages (clone or not: shared
        pages are never written, so a slice is already independent)."""
        if end < 0:
            raise ValueError("cache slice end must be non-negative")
        if end > self._length:
            raise ValueError(f"cache slice end {end} exceeds cache length {self._length}")
        pages = self.pages[: -(-end // self.manager.page_size)]
        self.manager._ref_pages(pages)
        return PagedPrefix(self.manager, list(pages), end)

    def reset(self) -> None:
        """Drop the page references (idempotent)."""
        if self.pages:
            self.manager._drop_pages(self.pages)
        self.pages = []
        self._length = 0

    def to_cache(self) -> Cache:
        """A compact (layers, Hkv, length, D) copy gathered from the pages."""
        return self.manager._gather(self.pages, self._length)


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_hip(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{what} runs only on a HIP device (tensor is on {t.device}); "
            "there is no CPU implementation"
        )


def _row_strides(t: torch.Tensor, layout: str, q_len: int):
    """(stride_seq, stride_tok, stride_head) for the kernels' addressing
    base + b*seq + (q_start[b] + i)*tok + h*head with q_start[b] = b * q_len.

    layout "bhtd": (B, H, T, D); "bthd": (B, T, H, D); "thd": packed (N, H, D).
    """
    st = t.stride()
    if layout == "thd":
        s_tok, s_head, s_el = st
        s_seq = 0
    elif layout == "bhtd":
        s_b, s_head, s_tok, s_el = st
        s_seq = s_b - q_len * s_tok
    elif layout == "bthd":
        s_b, s_tok, s_head, s_el = st
        s_seq = s_b - q_len * s_tok
    else:
        raise ValueError(layout)
    if s_el != 1 or (s_tok | s_head | s_seq) & 7 or t.data_ptr() & 15:
        raise ValueError("rows must be contiguous in the last dim and 16-byte aligned")
    return s_seq, s_tok, s_head


def _aligned_rows(t: torch.Tensor) -> torch.Tensor:
    st = t.stride()
    if st[-1] != 1 or t.data_ptr() & 15:
        return t.contiguous()
    acc = 0
    for x in st[:-1]:
        acc |= x
    return t.contiguous() if acc & 7 else t


@dataclass
class _AppendInputs:
    q: torch.Tensor
    q_out: torch.Tensor
    num_q_heads: int
    keep: tuple  # tensors whose addresses are in head / tables
    head: tuple  # q .. k_norm_weight arguments of the C call
    tables: tuple  # cos, sin, max_positions


class _DevicePlan:
    """One tick's work lists on the device plus the split workspaces."""

    def __init__(self, host: "_native.TickPlan", num_q_heads: int, num_kv_heads: int,
                 head_dim: int, device: torch.device):
        self.host = host
        self.n_decode = host.n_chunks
        self.n_merge = len(host.merge)
        self.n_slots = host.n_slots
        self.n_prefill = len(host.prefill)
        self.n_prefill_merge = len(host.prefill_merge)
        self.n_prefill_slots = host.n_prefill_slots
        parts = [host.decode, host.merge, host.prefill, host.prefill_merge]
        packed = np.concatenate([p.reshape(-1) for p in parts])
        dev = torch.from_numpy(np.ascontiguousarray(packed, dtype=np.int32)).to(device)
        views, off = [], 0
        for p in parts:
            views.append(dev[off : off + p.size])
            off += p.size
        self.decode, self.merge, self.prefill, self.prefill_merge = views
        self.workspace_bytes = _native.decode_workspace_bytes(self.n_slots, num_q_heads, head_dim)
        self.workspace = (
            torch.empty(self.workspace_bytes // 4, dtype=torch.float32, device=device)
            if self.workspace_bytes
            else None
        )
        self.prefill_workspace_bytes = _native.prefill_workspace_bytes(
            self.n_prefill_slots, num_kv_heads, head_dim
        )
        self.prefill_workspace = (
            torch.empty(self.prefill_workspace_bytes // 4, dtype=torch.float32, device=device)
            if self.prefill_workspace_bytes
            else None
        )
        # raw addresses for the C calls (None for an empty list)
        def addr(t):
            return t.data_ptr() if t is not None and t.numel() else None

        self.decode_ptr = addr(self.decode)
        self.merge_ptr = addr(self.merge)
        self.prefill_ptr = addr(self.prefill)
        self.prefill_merge_ptr = addr(self.prefill_merge)
        self.workspace_ptr = addr(self.workspace)
        self.prefill_workspace_ptr = addr(self.prefill_workspace)


class PagedKVBatch:
    """Per-forward metadata shared by every layer (paged_cache.py:33-71).

    Attributes kept from the reference: ``k_cache``, ``v_cache``,
    ``page_table`` (int32 here, -1 padded, width = the batch's largest page
    count), ``cache_lens`` (int64, used by callers for positions) and
    ``page_size``. ``block_mask``/``score_mod`` are gone; the kernels read
    ``kv_lens``, ``q_start`` and the planner's work lists instead.

    Uniform batches (``begin_batch``) use the reference's tensor shapes:
    k/v (B, Hkv, T, D) for ``write_layer``, q (B, Hq, T, D) for
    ``attend_layer``. Varlen ticks (``begin_tick``) use packed (N, H, D).
    """

    def __init__(
        self,
        manager: "PagedKVCacheManager",
        q_lens: list[int],
        cache_lens_host: list[int],
        page_lists: list[list[int]],
        varlen: bool,
        num_q_heads: Optional[int],
        tokens_per_split: int = 0,
    ):
        self.k_cache = manager.k_cache
        self.v_cache = manager.v_cache
        self.page_size = manager.page_size
        self.device = manager.device
        self.num_kv_heads = manager.num_kv_heads
        self.head_dim = manager.head_dim
        self.varlen = varlen
        self.q_lens = list(q_lens)
        self.cache_lens_host = list(cache_lens_host)
        self.kv_lens_host = [c + q for c, q in zip(cache_lens_host, q_lens)]
        self.num_seqs = len(q_lens)
        self.total_tokens = int(sum(q_lens))
        self.query_len = q_lens[0] if not varlen else None
        self.tokens_per_split = tokens_per_split
        self._num_cus = manager.num_cus
        self._max_kv = max(self.kv_lens_host) if self.kv_lens_host else 0
        self._pool_ptrs: dict = {}
        # optional per-kernel timing hook, see _launch
        self.launch_hook = None

        width = max(1, max(len(p) for p in page_lists))
        table = np.full((self.num_seqs, width), -1, dtype=np.int32)
        for row, pages in enumerate(page_lists):
            table[row, : len(pages)] = pages
        if table.size and (table >= manager.num_pages).any():
            raise RuntimeError("page table holds a page id outside the pool")
        q_start = np.zeros(self.num_seqs + 1, dtype=np.int32)
        q_start[1:] = np.cumsum(q_lens)
        self._table_np = table
        self._meta_np = np.concatenate(
            [
                table.reshape(-1),
                np.asarray(cache_lens_host, dtype=np.int32),
                np.asarray(self.kv_lens_host, dtype=np.int32),
                q_start,
            ]
        )
        meta = torch.from_numpy(self._meta_np).to(self.device)
        n, b = table.size, self.num_seqs
        self.page_table = meta[:n].view(self.num_seqs, width)
        self.cache_lens_i32 = meta[n : n + b]
        self.kv_lens = meta[n + b : n + 2 * b]
        self.q_start = meta[n + 2 * b : n + 3 * b + 1]
        self.cache_lens = self.cache_lens_i32.to(torch.long)
        self._meta = meta
        self._pt_ptr = self.page_table.data_ptr()
        self._pt_stride = self.page_table.stride(0)
        self._q_start_ptr = self.q_start.data_ptr()
        self._cache_lens_ptr = self.cache_lens_i32.data_ptr()
        self._kv_lens_ptr = self.kv_lens.data_ptr()
        self._plans: dict[int, tuple] = {}
        if num_q_heads is not None and self.device.type == "cuda":
            self.plan(num_q_heads)

    # ------------------------------------------------------------------ plan
    def plan(self, num_q_heads: int) -> "_DevicePlan":
        """Work lists for this tick (built once per query-head count)."""
        cached = self._plans.get(num_q_heads)
        if cached is not None:
            return cached
        host = _native.plan_tick(
            np.asarray(self.q_lens, dtype=np.int32),
            np.asarray(self.kv_lens_host, dtype=np.int32),
            num_q_heads,
            self.num_kv_heads,
            self.page_size,
            self._num_cus,
            self.tokens_per_split,
        )
        plan = _DevicePlan(host, num_q_heads, self.num_kv_heads, self.head_dim, self.device)
        self._plans[num_q_heads] = plan
        return plan

    def _layer_pools(self, layer_idx: int):
        """(k_ptr, v_ptr, head_stride) of one layer's pool slice, cached
        per batch (the pool tensors outlive the batch)."""
        hit = self._pool_ptrs.get(layer_idx)
        if hit is not None:
            return hit
        num_layers = self.k_cache.shape[0]
        if not -num_layers <= layer_idx < num_layers:
            raise IndexError(f"layer {layer_idx} out of range for {num_layers} layers")
        layer = layer_idx % num_layers
        el = self.k_cache.element_size()
        hit = (
            self.k_cache.data_ptr() + layer * self.k_cache.stride(0) * el,
            self.v_cache.data_ptr() + layer * self.v_cache.stride(0) * el,
            self.k_cache.stride(2),
        )
        self._pool_ptrs[layer_idx] = hit
        return hit

    def _layout(self, t: torch.Tensor, uniform_layout: str) -> tuple:
        if self.varlen:
            if t.dim() != 3 or t.shape[0] != self.total_tokens:
                raise ValueError(
                    f"varlen batch expects packed (tokens={self.total_tokens}, heads, dim)"
                )
            return _row_strides(t, "thd", 0)
        if t.dim() != 4:
            raise ValueError("uniform batch expects 4-D tensors")
        return _row_strides(t, uniform_layout, self.query_len)

    # ----------------------------------------------------------- write path
    def write_layer(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append new (already rotated) keys and values into their pages
        (paged_cache.py:44-60): k, v are (B, Hkv, T, D), or packed (N, Hkv, D)
        for a varlen tick."""
        _require_hip(k, "write_layer")
        k = _aligned_rows(k)
        v = _aligned_rows(v)
        self._check_kv(k, v, head_axis=1)
        k_ptr, v_ptr, hs = self._layer_pools(layer_idx)
        ks = self._layout(k, "bhtd")
        vs = self._layout(v, "bhtd")
        rc = _native.lib().hy_kv_append(
            k_ptr, v_ptr, hs,
            k.data_ptr(), *ks, v.data_ptr(), *vs,
            self._q_start_ptr, self._cache_lens_ptr, self._pt_ptr, self._pt_stride,
            self.num_seqs, self.total_tokens, self.num_kv_heads, self.head_dim,
            self.page_size, _stream_handle(self.device),
        )
        _native.check(rc, "hy_kv_append")

    def norm_rope_write_layer(
        self,
        layer_idx: int,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        q_norm_weight: Optional[torch.Tensor],
        k_norm_weight: Optional[torch.Tensor],
        eps: float,
        cos: Optional[torch.Tensor],
        sin: Optional[torch.Tensor],
        k_eps: Optional[float] = None,
    ) -> torch.Tensor:
        """Fused q/k RMSNorm + RoPE + paged append of k and v
        (attention.py:62-75 with rope.py:31-47). Inputs are the projection
        outputs, (B, T, H, D) (or packed (N, H, D) for a varlen tick); positions
        are cache_lens + token index. `eps` is the q norm's epsilon and
        `k_eps` the k norm's (default: `eps`). Returns the rotated q in the
        same layout; k and v go to the pool only."""
        a = self._append_inputs("norm_rope_write_layer", q, k, v, q_norm_weight,
                                k_norm_weight, cos, sin)
        k_ptr, v_ptr, hs = self._layer_pools(layer_idx)
        rc = _native.lib().hy_qknorm_rope_append(
            *a.head, float(eps), float(eps if k_eps is None else k_eps), *a.tables,
            k_ptr, v_ptr, hs,
            self._q_start_ptr, self._cache_lens_ptr, self._pt_ptr, self._pt_stride,
            self.num_seqs, self.total_tokens, a.num_q_heads, self.num_kv_heads,
            self.head_dim, self.page_size, _stream_handle(self.device),
        )
        _native.check(rc, "hy_qknorm_rope_append")
        return a.q_out

    def _append_inputs(self, what, q, k, v, q_norm_weight, k_norm_weight, cos, sin):
        """Checked, 16-byte-aligned inputs of the fused norm + rope + append
        and the C arguments they map to (shared by norm_rope_write_layer and
        decode_layer)."""
        _require_hip(q, what)
        q = _aligned_rows(q)
        k = _aligned_rows(k)
        v = _aligned_rows(v)
        self._check_kv(k, v, head_axis=2)
        if q.dtype != torch.bfloat16:
            raise TypeError("q must be bfloat16")
        num_q_heads = q.shape[-2]
        q_out = torch.empty_like(q, memory_format=torch.contiguous_format)
        qs = self._layout(q, "bthd")
        qos = self._layout(q_out, "bthd")
        ks = self._layout(k, "bthd")
        vs = self._layout(v, "bthd")
        if (cos is None) != (sin is None):
            raise ValueError("cos and sin rope tables go together (both or neither)")
        if cos is not None:
            if cos.dtype != torch.float32 or sin.dtype != torch.float32:
                raise TypeError("rope tables must be float32")
            cos = cos.contiguous()
            sin = sin.contiguous()
            max_pos = cos.shape[0]
            if self._max_kv > max_pos:
                raise ValueError(
                    f"positions up to {self._max_kv - 1} exceed the rope "
                    f"table ({max_pos} positions)"
                )
        else:
            max_pos = 0
        qw = None if q_norm_weight is None else q_norm_weight.contiguous()
        kw = None if k_norm_weight is None else k_norm_weight.contiguous()
        for w in (qw, kw):
            if w is not None and (w.dtype != torch.bfloat16 or w.numel() != self.head_dim):
                raise TypeError("norm weights must be bfloat16 (head_dim,)")
        return _AppendInputs(
            q=q, q_out=q_out, num_q_heads=num_q_heads, keep=(k, v, qw, kw, cos, sin),
            head=(q.data_ptr(), *qs, q_out.data_ptr(), *qos, k.data_ptr(), *ks,
                  v.data_ptr(), *vs, None if qw is None else qw.data_ptr(),
                  None if kw is None else kw.data_ptr()),
            tables=(None if cos is None else cos.data_ptr(),
                    None if sin is None else sin.data_ptr(), max_pos),
        )

    def decode_layer(
        self,
        layer_idx: int,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        q_norm_weight: Optional[torch.Tensor],
        k_norm_weight: Optional[torch.Tensor],
        eps: float,
        cos: Optional[torch.Tensor],
        sin: Optional[torch.Tensor],
        scale: Optional[float] = None,
        no_alloc: bool = False,
        k_eps: Optional[float] = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """norm_rope_write_layer then attend_layer, for a batch whose
        sequences all decode one token, in one kernel launch plus the merge
        (attention.py:62-75 then paged_cache.py:62-71). Inputs as for
        norm_rope_write_layer; returns (q_rot, out) exactly as the two calls
        would: q_rot in the input layout, out as attend_layer returns it.
        Pool contents and q_rot are bit-identical to the two-call path.
        `eps` / `k_eps` are the q and k norms' epsilons, as there.

        no_alloc=True runs both launches through
        hy_paged_decode_append_noalloc, whose partials live in the library's
        static device scratch instead of the plan's workspace (same
        results; raises MemoryError if the tick's partials do not fit)."""
        if any(ql != 1 for ql in self.q_lens):
            raise ValueError("decode_layer needs q_len == 1 for every sequence")
        a = self._append_inputs("decode_layer", q, k, v, q_norm_weight, k_norm_weight, cos,
                                sin)
        num_q_heads = a.num_q_heads
        if num_q_heads % self.num_kv_heads:
            raise ValueError("query heads must be a multiple of kv heads")
        if self.varlen:
            out = torch.empty((self.total_tokens, num_q_heads, self.head_dim),
                              dtype=q.dtype, device=q.device)
            result = out
            os_ = self._layout(out, "thd")
        else:
            B, T = self.num_seqs, self.query_len
            buf = torch.empty((B, T, num_q_heads, self.head_dim), dtype=q.dtype,
                              device=q.device)
            result = buf.transpose(1, 2)
            os_ = self._layout(result, "bhtd")
        if scale is None:
            scale = 1.0 / math.sqrt(self.head_dim)
        plan = self.plan(num_q_heads)
        k_ptr, v_ptr, hs = self._layer_pools(layer_idx)
        stream = _stream_handle(self.device)
        lib = _native.lib()
        eps_pair = (float(eps), float(eps if k_eps is None else k_eps))
        if no_alloc:
            self._launch("hy_paged_decode_append_noalloc", lib.hy_paged_decode_append_noalloc,
                *a.head, *eps_pair, *a.tables, result.data_ptr(), *os_, k_ptr, v_ptr, hs,
                self._pt_ptr, self._pt_stride, self._q_start_ptr, self._cache_lens_ptr,
                plan.decode_ptr, plan.n_decode, plan.merge_ptr, plan.n_merge, plan.n_slots,
                self.num_seqs, num_q_heads, self.num_kv_heads, self.head_dim, self.page_size,
                float(scale), stream,
            )
            return a.q_out, result
        self._launch("hy_paged_decode_append", lib.hy_paged_decode_append,
            *a.head, *eps_pair, *a.tables, result.data_ptr(), k_ptr, v_ptr, hs,
            self._pt_ptr, self._pt_stride, self._q_start_ptr, self._cache_lens_ptr,
            plan.decode_ptr, plan.n_decode, plan.n_slots, plan.workspace_ptr,
            plan.workspace_bytes, self.num_seqs, num_q_heads, self.num_kv_heads,
            self.head_dim, self.page_size, float(scale), stream,
        )
        self._launch("hy_paged_decode_merge", lib.hy_paged_decode_merge,
            result.data_ptr(), *os_, self._q_start_ptr,
            plan.merge_ptr, plan.n_merge, plan.n_slots,
            plan.workspace_ptr, plan.workspace_bytes, num_q_heads,
            self.head_dim, stream,
        )
        return a.q_out, result

    def _check_kv(self, k: torch.Tensor, v: torch.Tensor, head_axis: int) -> None:
        if k.shape != v.shape:
            raise ValueError("k and v must have the same shape")
        if k.dtype != self.k_cache.dtype or v.dtype != self.v_cache.dtype:
            raise TypeError("k/v dtype must match the pool dtype")
        if k.shape[-1] != self.head_dim:
            raise ValueError("k/v head_dim does not match the pool")
        if self.varlen:
            head_axis = 1
        if k.shape[head_axis] != self.num_kv_heads:
            raise ValueError("k/v head count does not match the pool")

    # ---------------------------------------------------------- attend path
    def _launch(self, name: str, fn, *args) -> None:
        """Enqueues one C-ABI call. A `launch_hook(name, after)` set on the
        batch is called right before (after=False) and right after
        (after=True) the call, so a caller can bracket one kernel with
        events on the launch stream."""
        hook = self.launch_hook
        if hook is not None:
            hook(name, False)
        rc = fn(*args)
        if rc:
            _native.check(rc, name)
        if hook is not None:
            hook(name, True)

    def attend_layer(
        self, q: torch.Tensor, layer_idx: int, scale: Optional[float] = None
    ) -> torch.Tensor:
        """Causal GQA attention over this layer's pages (paged_cache.py:62-71).

        q is (B, Hq, T, D) for a uniform batch (returns (B, Hq, T, D), a
        transposed view of a (B, T, Hq, D) buffer so the caller's
        transpose + reshape is free) or packed (N, Hq, D) for a varlen tick.
        """
        _require_hip(q, "attend_layer")
        q = _aligned_rows(q)
        if q.dtype != self.k_cache.dtype:
            raise TypeError("q dtype must match the pool dtype")
        if self.varlen:
            num_q_heads = q.shape[1]
            out = torch.empty((self.total_tokens, num_q_heads, self.head_dim),
                              dtype=q.dtype, device=q.device)
            qs = self._layout(q, "thd")
            os_ = self._layout(out, "thd")
            result = out
        else:
            B, num_q_heads, T, D = q.shape
            if B != self.num_seqs or T != self.query_len:
                raise ValueError("q does not match the batch shape")
            buf = torch.empty((B, T, num_q_heads, D), dtype=q.dtype, device=q.device)
            result = buf.transpose(1, 2)
            qs = self._layout(q, "bhtd")
            os_ = self._layout(result, "bhtd")
        if num_q_heads % self.num_kv_heads:
            raise ValueError("query heads must be a multiple of kv heads")
        if scale is None:
            scale = 1.0 / math.sqrt(self.head_dim)
        plan = self.plan(num_q_heads)
        k_ptr, v_ptr, hs = self._layer_pools(layer_idx)
        stream = _stream_handle(self.device)
        lib = _native.lib()
        if plan.n_decode:
            self._launch("hy_paged_decode", lib.hy_paged_decode,
                q.data_ptr(), *qs, result.data_ptr(), *os_,
                k_ptr, v_ptr, hs,
                self._pt_ptr, self._pt_stride, self._q_start_ptr, plan.decode_ptr,
                plan.n_decode, plan.n_slots, plan.workspace_ptr, plan.workspace_bytes, self.num_seqs, num_q_heads,
                self.num_kv_heads, self.head_dim, self.page_size, float(scale),
                stream,
            )
        if plan.n_merge:
            self._launch("hy_paged_decode_merge", lib.hy_paged_decode_merge,
                result.data_ptr(), *os_, self._q_start_ptr,
                plan.merge_ptr, plan.n_merge, plan.n_slots,
                plan.workspace_ptr, plan.workspace_bytes, num_q_heads,
                self.head_dim, stream,
            )
        if plan.n_prefill:
            self._launch("hy_paged_prefill", lib.hy_paged_prefill,
                q.data_ptr(), *qs, result.data_ptr(), *os_,
                k_ptr, v_ptr, hs,
                self._pt_ptr, self._pt_stride, self._q_start_ptr, self._kv_lens_ptr,
                plan.prefill_ptr, plan.n_prefill, plan.n_prefill_slots,
                plan.prefill_workspace_ptr, plan.prefill_workspace_bytes, self.num_seqs, num_q_heads,
                self.num_kv_heads, self.head_dim, self.page_size, float(scale),
                stream,
            )
        if plan.n_prefill_merge:
            self._launch("hy_paged_prefill_merge", lib.hy_paged_prefill_merge,
                result.data_ptr(), *os_, self._q_start_ptr,
                plan.prefill_merge_ptr, plan.n_prefill_merge, plan.n_prefill_slots,
                plan.prefill_workspace_ptr, plan.prefill_workspace_bytes,
                num_q_heads, self.num_kv_heads, self.head_dim, stream,
            )
        return result


class PagedKVCacheManager:
    """Fixed-size pages of one shared K and one shared V tensor
    (paged_cache.py:74-200). Same constructor, same LIFO page order, same
    exceptions; adds per-page reference counts for prefix sharing."""

    def __init__(
        self,
        num_layers: int,
        num_kv_heads: int,
        head_dim: int,
        max_cache_tokens: int,
        page_size: int,
        max_requests: int,
        dtype: torch.dtype,
        device: torch.device | str,
        num_q_heads: Optional[int] = None,
        tokens_per_split: int = 0,
    ):
        if max_cache_tokens < 1:
            raise ValueError("max_cache_tokens must be positive")
        if page_size < 1 or page_size & (page_size - 1):
            raise ValueError("page_size must be a positive power of two")
        if max_requests < 1:
            raise ValueError("max_requests must be positive")

        self.page_size = page_size
        self.num_pages = math.ceil(max_cache_tokens / page_size)
        self.capacity_tokens = self.num_pages * page_size
        self.max_requests = max_requests
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.num_q_heads = num_q_heads
        self.tokens_per_split = tokens_per_split
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self._free_slots = list(range(max_requests - 1, -1, -1))
        self._free_pages = list(range(self.num_pages - 1, -1, -1))
        self._refs = [0] * self.num_pages
        self.num_cus = (
            torch.cuda.get_device_properties(self.device).multi_processor_count
            if self.device.type == "cuda"
            else 256
        )

        # (layers, 1, kv_heads, capacity, head_dim), head-major: one
        # (page, head) is page_size * head_dim contiguous elements.
        self.k_cache = torch.empty(
            (num_layers, 1, num_kv_heads, self.capacity_tokens, head_dim),
            dtype=dtype,
            device=self.device,
        )
        self.v_cache = torch.empty_like(self.k_cache)

    # ------------------------------------------------------------ allocator
    def _take_pages(self, count: int) -> list[int]:
        pages = [self._free_pages.pop() for _ in range(count)]
        for p in pages:
            self._refs[p] = 1
        return pages

    def _ref_pages(self, pages: Sequence[int]) -> None:
        for p in pages:
            self._refs[p] += 1

    def _drop_pages(self, pages: Sequence[int]) -> None:
        for p in pages:
            self._refs[p] -= 1
            if self._refs[p] == 0:
                self._free_pages.append(p)

    def page_refcount(self, page: int) -> int:
        return self._refs[page]

    @property
    def free_page_count(self) -> int:
        return len(self._free_pages)

    def allocate(self) -> PagedCacheHandle:
        """Reserve a request slot without pages (paged_cache.py:111-117)."""
        if not self._free_slots:
            raise MemoryError(
                f"paged cache supports at most {self.max_requests} active requests"
            )
        return PagedCacheHandle(slot=self._free_slots.pop())

    def reserve(self, handle: PagedCacheHandle, required_tokens: int) -> None:
        """Own enough pages for required_tokens positions (119-140)."""
        if handle.released:
            raise RuntimeError("cannot reserve pages for a released cache handle")
        if required_tokens < 0:
            raise ValueError("required_tokens must be non-negative")
        if required_tokens > self.capacity_tokens:
            raise MemoryError(
                f"request needs {required_tokens} cache tokens, but the paged cache "
                f"capacity is {self.capacity_tokens} tokens"
            )
        required_pages = math.ceil(required_tokens / self.page_size)
        missing = required_pages - len(handle.pages)
        if missing <= 0:
            return
        if len(self._free_pages) < missing:
            raise MemoryError(
                f"paged KV cache is full: need {missing} additional pages, "
                f"but only {len(self._free_pages)} remain"
            )
        handle.pages.extend(self._take_pages(missing))

    def allocate_for_request(self, cache: "Cache | PagedPrefix | None" = None) -> PagedCacheHandle:
        """Allocate a handle and optionally import a prefix (142-151): a
        contiguous Cache is copied into fresh pages; a PagedPrefix is
        shared without a copy (its pages gain a reference)."""
        handle = self.allocate()
        try:
            if isinstance(cache, PagedPrefix):
                if cache.manager is not self:
                    raise ValueError("a PagedPrefix belongs to the pool that made it")
                if cache.length:
                    self._ref_pages(cache.pages)
                    handle.pages = list(cache.pages)
                    handle.length = cache.length
            elif cache is not None and cache.length:
                self.import_cache(handle, cache)
        except Exception:
            self.release(handle)
            raise
        return handle

    def import_cache(self, handle: PagedCacheHandle, cache: Cache) -> None:
        """Copy a contiguous (layers, Hkv, len, D) prefix into the handle's
        pages with hy_page_scatter (153-166)."""
        if cache.k is None or cache.v is None:
            return
        _require_hip(self.k_cache, "import_cache")
        self.reserve(handle, cache.length)
        self._make_private(handle, 0, cache.length)
        pages = torch.tensor(handle.pages, dtype=torch.int32, device=self.device)
        layers = cache.k.shape[0]
        for pool, src in ((self.k_cache, cache.k), (self.v_cache, cache.v)):
            src = src.to(device=self.device, dtype=pool.dtype)
            src = _aligned_rows(src)
            rc = _native.lib().hy_page_scatter(
                pool.data_ptr(), pool.stride(0), pool.stride(2), pages.data_ptr(),
                cache.length, src.data_ptr(), src.stride(0), src.stride(1),
                src.stride(2), layers, self.num_kv_heads, self.head_dim,
                self.page_size, _stream_handle(self.device),
            )
            _native.check(rc, "hy_page_scatter")
        handle.length = cache.length

    def truncate(self, handle: PagedCacheHandle, length: int) -> None:
        """Shorten a cache, returning whole pages past the end (168-178)."""
        if handle.released:
            raise RuntimeError("cannot truncate a released cache handle")
        if length < 0 or length > handle.length:
            raise ValueError("truncate length must be within the current cache length")
        keep = math.ceil(length / self.page_size)
        released = handle.pages[keep:]
        handle.pages = handle.pages[:keep]
        self._drop_pages(released)
        handle.length = length

    def snapshot(self, handle: PagedCacheHandle, length: int | None = None) -> Cache:
        """Gather the first `length` positions into a compact Cache with
        hy_page_gather (180-190)."""
        if handle.released:
            raise RuntimeError("cannot snapshot a released cache handle")
        snapshot_len = handle.length if length is None else length
        if snapshot_len < 0 or snapshot_len > handle.length:
            raise ValueError("snapshot length must be within the current cache length")
        return self._gather(handle.pages, snapshot_len)

    def share(self, handle: PagedCacheHandle, length: int | None = None) -> PagedPrefix:
        """Zero-copy snapshot: the first `length` tokens (default: all) as a
        PagedPrefix that references the handle's pages. Later appends by
        the handle copy a shared page first, so the prefix never changes."""
        if handle.released:
            raise RuntimeError("cannot snapshot a released cache handle")
        share_len = handle.length if length is None else length
        if share_len < 0 or share_len > handle.length:
            raise ValueError("snapshot length must be within the current cache length")
        pages = handle.pages[: -(-share_len // self.page_size)]
        self._ref_pages(pages)
        return PagedPrefix(self, list(pages), share_len)

    def _gather(self, page_list: Sequence[int], snapshot_len: int) -> Cache:
        _require_hip(self.k_cache, "snapshot")
        shape = (self.num_layers, self.num_kv_heads, snapshot_len, self.head_dim)
        k = torch.empty(shape, dtype=self.k_cache.dtype, device=self.device)
        v = torch.empty_like(k)
        if snapshot_len:
            pages = torch.tensor(list(page_list), dtype=torch.int32, device=self.device)
            for pool, dst in ((self.k_cache, k), (self.v_cache, v)):
                rc = _native.lib().hy_page_gather(
                    pool.data_ptr(), pool.stride(0), pool.stride(2), pages.data_ptr(),
                    snapshot_len, dst.data_ptr(), self.num_layers,
                    self.num_kv_heads, self.head_dim, self.page_size,
                    _stream_handle(self.device),
                )
                _native.check(rc, "hy_page_gather")
        return Cache.from_tensors(k, v)

    def release(self, handle: PagedCacheHandle) -> None:
        """Return the handle's pages and slot (192-200)."""
        if handle.released:
            return
        self._drop_pages(handle.pages)
        handle.pages.clear()
        handle.length = 0
        handle.released = True
        self._free_slots.append(handle.slot)

    def claim_pages(self, handle: PagedCacheHandle, pages: Sequence[int]) -> None:
        """Append specific free page ids to a handle (restores a saved or
        seeded page placement; `reserve` takes pages in LIFO order)."""
        if handle.released:
            raise RuntimeError("cannot claim pages for a released cache handle")
        wanted = [int(p) for p in pages]
        if len(set(wanted)) != len(wanted):
            raise ValueError("page ids must be distinct")
        free = set(self._free_pages)
        missing = [p for p in wanted if p not in free]
        if missing:
            raise ValueError(f"pages {missing[:8]} are not free")
        taken = set(wanted)
        self._free_pages = [p for p in self._free_pages if p not in taken]
        for p in wanted:
            self._refs[p] = 1
        handle.pages.extend(wanted)

    # -------------------------------------------------------------- sharing
    def fork(self, handle: PagedCacheHandle, length: int | None = None) -> PagedCacheHandle:
        """New handle whose first `length` tokens (default: all of them)
        reference the same physical pages, a partly filled last page
        included. Shared pages are read-only; the first append into one (by
        either handle) copies it."""
        if handle.released:
            raise RuntimeError("cannot fork a released cache handle")
        if length is None:
            length = handle.length
        if length < 0 or length > handle.length:
            raise ValueError("fork length must be within the current cache length")
        child = self.allocate()
        shared = handle.pages[: -(-length // self.page_size)]
        self._ref_pages(shared)
        child.pages = list(shared)
        child.length = length
        return child

    def _make_private(self, handle: PagedCacheHandle, start: int, end: int) -> None:
        """Copy-on-write every shared page that positions [start, end) touch."""
        if end <= start:
            return
        first = start // self.page_size
        last = (end - 1) // self.page_size
        for idx in range(first, min(last + 1, len(handle.pages))):
            page = handle.pages[idx]
            if self._refs[page] <= 1:
                continue
            _require_hip(self.k_cache, "copy-on-write of a shared page")
            if not self._free_pages:
                raise MemoryError("paged KV cache is full: no page for copy-on-write")
            (new_page,) = self._take_pages(1)
            lo, hi = page * self.page_size, (page + 1) * self.page_size
            nlo, nhi = new_page * self.page_size, (new_page + 1) * self.page_size
            self.k_cache[:, :, :, nlo:nhi].copy_(self.k_cache[:, :, :, lo:hi])
            self.v_cache[:, :, :, nlo:nhi].copy_(self.v_cache[:, :, :, lo:hi])
            self._refs[page] -= 1
            handle.pages[idx] = new_page

    # ---------------------------------------------------------- tick setup
    def _validate_handles(self, handles: Sequence[PagedCacheHandle]) -> None:
        if not handles:
            raise ValueError("cannot build paged cache metadata for an empty batch")
        if any(h.released for h in handles):
            raise RuntimeError("cannot use a released cache handle in an attention batch")
        if len({id(h) for h in handles}) != len(handles):
            raise ValueError("an attention batch cannot contain the same cache handle twice")

    def _cow_pages_needed(self, handles: Sequence[PagedCacheHandle],
                          q_lens: Sequence[int]) -> int:
        """Pages that _make_private will copy for this batch: shared pages
        (refcount > 1) that [length, length + q) of a handle touches,
        counted in the order _make_private visits them (a copy drops the
        original's count, so the last sharer in the batch writes in place)."""
        refs: dict[int, int] = {}
        copies = 0
        for h, q in zip(handles, q_lens):
            if q <= 0:
                continue
            first = h.length // self.page_size
            last = (h.length + q - 1) // self.page_size
            for idx in range(first, min(last + 1, len(h.pages))):
                page = h.pages[idx]
                r = refs.get(page, self._refs[page])
                if r > 1:
                    copies += 1
                    refs[page] = r - 1
        return copies

    def _reserve_all(self, handles: Sequence[PagedCacheHandle], q_lens: Sequence[int]) -> None:
        """Reserve every handle's append space and copy the shared pages the
        appends touch, or raise before changing anything."""
        kv_lengths = [h.length + q for h, q in zip(handles, q_lens)]
        additional = sum(
            max(0, math.ceil(kv / self.page_size) - len(h.pages))
            for h, kv in zip(handles, kv_lengths)
        )
        if any(kv > self.capacity_tokens for kv in kv_lengths):
            raise MemoryError(
                f"request needs more than the paged cache capacity of "
                f"{self.capacity_tokens} tokens"
            )
        copies = self._cow_pages_needed(handles, q_lens)
        if copies:
            _require_hip(self.k_cache, "copy-on-write of a shared page")
        if additional + copies > len(self._free_pages):
            raise MemoryError(
                f"paged KV cache is full: batch needs {additional + copies} "
                f"additional pages, but only {len(self._free_pages)} remain"
            )
        for h, kv in zip(handles, kv_lengths):
            self.reserve(h, kv)
        for h, q in zip(handles, q_lens):
            self._make_private(h, h.length, h.length + q)

    def begin_batch(
        self, handles: Sequence[PagedCacheHandle], query_len: int
    ) -> PagedKVBatch:
        """Reserve append space for `query_len` tokens per request and build
        the tick metadata (paged_cache.py:202-293)."""
        self._validate_handles(handles)
        if query_len < 1:
            raise ValueError("query_len must be positive")
        q_lens = [query_len] * len(handles)
        self._reserve_all(handles, q_lens)
        if self.page_size < MIN_KV_PAGE_SIZE:
            raise ValueError(
                f"page_size must be at least {MIN_KV_PAGE_SIZE} tokens"
            )
        return PagedKVBatch(
            self, q_lens, [h.length for h in handles], [list(h.pages) for h in handles],
            varlen=False, num_q_heads=self.num_q_heads,
            tokens_per_split=self.tokens_per_split,
        )

    def begin_tick(
        self, handles: Sequence[PagedCacheHandle], query_lens: Sequence[int]
    ) -> PagedKVBatch:
        """One varlen batch mixing prefill chunks (q_len > 1) and decode
        tokens (q_len == 1); tensors are packed (total_tokens, heads, dim)
        in handle order. Commit with ``commit_tick``."""
        q_lens = self.reserve_tick(handles, query_lens)
        return PagedKVBatch(
            self, q_lens, [h.length for h in handles], [list(h.pages) for h in handles],
            varlen=True, num_q_heads=self.num_q_heads,
            tokens_per_split=self.tokens_per_split,
        )

    def reserve_tick(self, handles: Sequence[PagedCacheHandle],
                     query_lens: Sequence[int]) -> list[int]:
        """The checks and reservations of begin_tick without building a
        batch (for callers that keep their own tick metadata, such as a
        replayed decode graph); returns the query lengths as ints."""
        self._validate_handles(handles)
        q_lens = [int(q) for q in query_lens]
        if len(q_lens) != len(handles):
            raise ValueError("one query length per handle is required")
        if any(q < 1 for q in q_lens):
            raise ValueError("query lengths must be positive")
        self._reserve_all(handles, q_lens)
        if self.page_size < MIN_KV_PAGE_SIZE:
            raise ValueError(
                f"page_size must be at least {MIN_KV_PAGE_SIZE} tokens"
            )
        return q_lens

    def commit_batch(self, handles: Sequence[PagedCacheHandle], query_len: int) -> None:
        """Advance lengths after every layer wrote its states (295-304)."""
        self.commit_tick(handles, [query_len] * len(handles))

    def commit_tick(self, handles: Sequence[PagedCacheHandle], query_lens: Sequence[int]) -> None:
        """Advance each handle by its query length after a begin_tick batch
        ran through every layer."""
        if len(query_lens) != len(handles):
            raise ValueError("one query length per handle is required")
        for handle, q in zip(handles, query_lens):
            if handle.released:
                raise RuntimeError("cannot commit a released cache handle")
            if handle.length + q > len(handle.pages) * self.page_size:
                raise RuntimeError("paged cache append space was not reserved")
            handle.length += q

    def _physical_positions(self, handle: PagedCacheHandle, length: int) -> np.ndarray:
        """Physical token index of logical positions 0..length-1 (306-315)."""
        if length == 0:
            return np.zeros(0, dtype=np.int64)
        logical = np.arange(length, dtype=np.int64)
        pages = np.asarray(handle.pages, dtype=np.int64)
        return pages[logical // self.page_size] * self.page_size + logical % self.page_size
