"""Seeded synthetic workloads for the five paged-attention configurations
(Qwen3-4B geometry: 32 query heads, 8 kv heads, head_dim 128, bf16, 128-token
pages). Used by the tests and the benchmark; no data comes from a checkpoint.

Every configuration is one attention step of one transformer layer:
the fused q/k RMSNorm + RoPE + append of this step's tokens, then attention
over the page table. The whole pool is filled with N(0, 1) so that a read of a
wrong page changes the result. Page placement is a seeded permutation of the
pool's pages consumed request by request.

  decode_b1      batch 1, context 512 (4 pages of a 16,384-token pool)
  decode_b32     batch 32, contexts uniform in [256, 4096], 262,144-token pool
  prefill_4x512  4 chunks of 512 at cached offsets {0, 1024, 2048, 3584}
  mixed_tick     8 prefill chunks of 512 + 56 decode tokens (contexts uniform
                 in [512, 8192]); 16 requests share 8 prefix pages
  decode_32k     batch 8, context 32,768 each, all 2,048 pages of the pool
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import torch

from .constants import HEAD_DIM, MAX_POSITION_EMBEDDINGS, NUM_KV_HEADS, NUM_Q_HEADS, ROPE_THETA
from .paged_cache import PagedCacheHandle, PagedKVBatch, PagedKVCacheManager
from .rope import compute_rope_params

PAGE = 128
KV_BYTES_PER_TOKEN = 2 * NUM_KV_HEADS * HEAD_DIM * 2  # K + V, all kv heads, bf16
FLOPS_PER_PAIR = 4 * NUM_Q_HEADS * HEAD_DIM  # QK^T + PV, all query heads


@dataclass
class ConfigSpec:
    name: str
    index: int
    pool_tokens: int
    seed: int
    description: str


SPECS = {
    "decode_b1": ConfigSpec("decode_b1", 1, 16_384, 1001,
                            "decode, batch 1, context 512, 16,384-token pool"),
    "decode_b32": ConfigSpec("decode_b32", 2, 262_144, 1002,
                             "decode, batch 32, context U[256, 4096], 262,144-token pool"),
    "prefill_4x512": ConfigSpec("prefill_4x512", 3, 262_144, 1003,
                                "chunked prefill, 4 x 512 at offsets {0, 1024, 2048, 3584}"),
    "mixed_tick": ConfigSpec("mixed_tick", 4, 524_288, 1004,
                             "mixed tick, 8 x 512 prefill + 56 decode, 16 share 8 prefix pages"),
    "decode_32k": ConfigSpec("decode_32k", 5, 262_144, 1005,
                             "decode, batch 8, context 32,768, 262,144-token pool"),
}
ORDER = ["decode_b1", "decode_b32", "prefill_4x512", "mixed_tick", "decode_32k"]


@dataclass
class Workload:
    spec: ConfigSpec
    manager: PagedKVCacheManager
    handles: list[PagedCacheHandle]
    q_lens: list[int]
    cache_lens: list[int]
    page_lists: list[list[int]]
    q: torch.Tensor          # raw projections, packed (N, Hq, D) bf16
    k: torch.Tensor          # (N, Hkv, D)
    v: torch.Tensor          # (N, Hkv, D)
    q_norm_w: torch.Tensor   # (D,) bf16
    k_norm_w: torch.Tensor
    cos: torch.Tensor        # (max_pos, D) fp32
    sin: torch.Tensor
    shared_pages: list[int] = field(default_factory=list)
    batch: Optional[PagedKVBatch] = None

    @property
    def kv_lens(self) -> list[int]:
        return [c + q for c, q in zip(self.cache_lens, self.q_lens)]

    def begin(self) -> PagedKVBatch:
        self.batch = self.manager.begin_tick(self.handles, self.q_lens)
        return self.batch

    # Algorithmic work of one step (numerators of the roofline fractions).
    def decode_bytes(self, include_append: bool = True) -> int:
        """HBM bytes a decode step must move: every K/V row of every decode
        context once (shared pages once), q and output rows and, with
        include_append, the appended K/V rows (written by the append
        kernel, not by attention)."""
        seen = set()
        tokens = 0
        n_dec = 0
        for pages, c, ql in zip(self.page_lists, self.cache_lens, self.q_lens):
            if ql != 1:
                continue
            n_dec += 1
            kv = c + ql
            for j in range(math.ceil(kv / PAGE)):
                used = min(PAGE, kv - j * PAGE)
                if pages[j] in seen:
                    continue
                seen.add(pages[j])
                tokens += used
        qo = n_dec * 2 * NUM_Q_HEADS * HEAD_DIM * 2
        append = n_dec * KV_BYTES_PER_TOKEN if include_append else 0
        return tokens * KV_BYTES_PER_TOKEN + qo + append

    def prefill_pairs(self) -> int:
        """(query, key) pairs visible under the causal mask, prefill rows."""
        pairs = 0
        for c, ql in zip(self.cache_lens, self.q_lens):
            if ql > 1:
                pairs += ql * c + ql * (ql + 1) // 2
        return pairs

    def decode_pairs(self) -> int:
        return sum(c + 1 for c, ql in zip(self.cache_lens, self.q_lens) if ql == 1)

    def prefill_flops(self) -> int:
        return FLOPS_PER_PAIR * self.prefill_pairs()


def _lengths(name: str, gen: torch.Generator):
    """(cache_lens, q_lens) of a configuration, drawn from `gen`."""
    if name == "decode_b1":
        return [511], [1]
    if name == "decode_b32":
        ctx = torch.randint(256, 4097, (32,), generator=gen).tolist()
        return [c - 1 for c in ctx], [1] * 32
    if name == "prefill_4x512":
        return [0, 1024, 2048, 3584], [512] * 4
    if name == "mixed_tick":
        offs = (torch.randint(8, 33, (8,), generator=gen) * PAGE).tolist()  # 1024..4096
        ctx = torch.randint(512, 8193, (56,), generator=gen).tolist()
        return offs + [c - 1 for c in ctx], [512] * 8 + [1] * 56
    if name == "decode_32k":
        return [32_767] * 8, [1] * 8
    raise KeyError(name)


def fill_pool(manager: PagedKVCacheManager, seed: int) -> None:
    """N(0, 1) bf16 in every position of every layer (on the pool's device)."""
    gen = torch.Generator(device=manager.device)
    gen.manual_seed(seed)
    for pool in (manager.k_cache, manager.v_cache):
        flat = pool.view(-1)
        step = 1 << 26
        for i in range(0, flat.numel(), step):
            n = min(step, flat.numel() - i)
            flat[i : i + n] = torch.randn(n, generator=gen, device=manager.device,
                                          dtype=torch.float32).to(torch.bfloat16)


def make_workload(name: str, device: torch.device | str = "cuda", num_layers: int = 1,
                  pool_tokens: Optional[int] = None, seed: Optional[int] = None,
                  fill: bool = True, tokens_per_split: int = 0,
                  lengths: Optional[tuple[list[int], list[int]]] = None) -> Workload:
    """The named configuration; `lengths` = (cache_lens, q_lens) replaces its
    request lengths (same pool, seed and placement rule)."""
    spec = SPECS[name]
    seed = spec.seed if seed is None else seed
    gen = torch.Generator().manual_seed(seed)
    cache_lens, q_lens = _lengths(name, gen)
    if lengths is not None:
        cache_lens, q_lens = list(lengths[0]), list(lengths[1])
    pool_tokens = pool_tokens or spec.pool_tokens
    n_pages_pool = pool_tokens // PAGE
    manager = PagedKVCacheManager(
        num_layers=num_layers, num_kv_heads=NUM_KV_HEADS, head_dim=HEAD_DIM,
        max_cache_tokens=pool_tokens, page_size=PAGE, max_requests=len(q_lens),
        dtype=torch.bfloat16, device=device, num_q_heads=NUM_Q_HEADS,
        tokens_per_split=tokens_per_split,
    )
    perm = torch.randperm(n_pages_pool, generator=gen).tolist()
    need = [math.ceil((c + q) / PAGE) for c, q in zip(cache_lens, q_lens)]

    handles: list[PagedCacheHandle] = []
    shared: list[int] = []
    cursor = 0
    if name == "mixed_tick":
        # Requests 0..7 (prefill, offsets >= 1024) and the first 8 decode
        # requests with a cached length >= 1024 share 8 prefix pages.
        sharers = list(range(8)) + [i for i in range(8, len(q_lens)) if cache_lens[i] >= 1024][:8]
        shared = perm[cursor : cursor + 8]
        cursor += 8
    else:
        sharers = []
    owner: Optional[PagedCacheHandle] = None
    for i, (c, n) in enumerate(zip(cache_lens, q_lens)):
        if i in sharers:
            if owner is None:
                h = manager.allocate()
                manager.claim_pages(h, shared)
                h.length = 8 * PAGE
                owner = h
            else:
                h = manager.fork(owner, 8 * PAGE)
            own = need[i] - 8
        else:
            h = manager.allocate()
            own = need[i]
        manager.claim_pages(h, perm[cursor : cursor + own])
        cursor += own
        h.length = c
        handles.append(h)
    if cursor > n_pages_pool:
        raise MemoryError("workload needs more pages than the pool holds")

    if fill:
        fill_pool(manager, seed + 7)

    n_tok = sum(q_lens)
    q = torch.randn((n_tok, NUM_Q_HEADS, HEAD_DIM), generator=gen).to(torch.bfloat16)
    k = torch.randn((n_tok, NUM_KV_HEADS, HEAD_DIM), generator=gen).to(torch.bfloat16)
    v = torch.randn((n_tok, NUM_KV_HEADS, HEAD_DIM), generator=gen).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(HEAD_DIM, generator=gen)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(HEAD_DIM, generator=gen)).to(torch.bfloat16)
    cos, sin = compute_rope_params(HEAD_DIM, ROPE_THETA, MAX_POSITION_EMBEDDINGS, device=device)
    dev = manager.device
    return Workload(
        spec=spec, manager=manager, handles=handles, q_lens=q_lens, cache_lens=cache_lens,
        page_lists=[list(h.pages) for h in handles],
        q=q.to(dev), k=k.to(dev), v=v.to(dev), q_norm_w=qw.to(dev), k_norm_w=kw.to(dev),
        cos=cos, sin=sin, shared_pages=shared,
    )
