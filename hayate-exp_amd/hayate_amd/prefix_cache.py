"""Prompt-prefix cache over shared KV pages, indexed by page-sized blocks.

Observable policy of the reference's hayate/engine/prefix_cache.py:
* ``get(tokens, max_prefix_len)`` (:32-59) returns the longest common
  prefix of `tokens` with any stored prompt, at most max_prefix_len tokens;
  among stored prompts that share that longest prefix, the least recently
  used one is returned (the reference scans in LRU order and keeps the
  first strict improvement), and it becomes the most recently used;
* ``put(tokens, cache)`` (:61-80) stores the first
  min(len(tokens), cache.length, max_tokens) tokens, replacing an identical
  key, and then drops least recently used entries until the stored tokens
  fit the budget (:96-100).

The structure is different. The reference compares the prompt with every
stored key, token by token. Here stored prompts hang in a trie whose edges
are whole blocks of `block_tokens` tokens (the pool's page size, so one
trie level is one shared page): a lookup follows the prompt's full blocks
by hashing each block once, and only at the deepest node it reaches
compares the next, partial block with that node's outgoing blocks and the
short tails of prompts that end inside it. Every node knows which entries
pass through it, so the candidates for the longest match are found without
visiting any other entry.

An entry is what the caller stores: with the paged engine a PagedPrefix
(references to the prompt's pool pages: ``slice`` takes more references,
nothing is copied, and a request that reuses it shares the pages through
``PagedKVCacheManager.allocate_for_request``); a reference-format Cache is
cloned as the reference does. Entries are immutable: shared pages are
copy-on-write.
"""

from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass
from typing import Any, Optional, Sequence


@dataclass(frozen=True)
class PrefixCacheMatch:
    """Cached token count and cache found for one prompt (prefix_cache.py:10-15)."""

    length: int
    cache: Any


def _shared_len(a: Sequence[int], b: Sequence[int]) -> int:
    n = min(len(a), len(b))
    i = 0
    while i < n and a[i] == b[i]:
        i += 1
    return i


class _Block:
    """A trie node: the prompts whose first `depth` blocks are this path."""

    __slots__ = ("parent", "edge", "depth", "next", "tails", "through")

    def __init__(self, parent: Optional["_Block"], edge: tuple, depth: int):
        self.parent = parent
        self.edge = edge            # the block of tokens leading here
        self.depth = depth          # full blocks from the root
        self.next: dict[tuple, _Block] = {}  # full next block -> node
        self.tails: dict[int, tuple] = {}     # entry -> its last, partial block
        self.through: set[int] = set()        # entries on this path (ending here or below)


class _Entry:
    __slots__ = ("key", "cache", "node")

    def __init__(self, key: tuple, cache: Any, node: _Block):
        self.key = key
        self.cache = cache
        self.node = node  # deepest node of the key's full blocks


def _release(cache) -> None:
    reset = getattr(cache, "reset", None)
    if reset is not None:
        reset()


class PrefixCache:
    """Least-recently-used prompt-prefix cache with a token budget."""

    def __init__(self, max_tokens: int, block_tokens: int = 128):
        if max_tokens < 0:
            raise ValueError("prefix cache token budget must be non-negative")
        if block_tokens < 1:
            raise ValueError("block_tokens must be positive")
        self.max_tokens = max_tokens
        self.block_tokens = block_tokens
        self.total_tokens = 0
        self._root = _Block(None, (), 0)
        self._lru: OrderedDict[int, _Entry] = OrderedDict()  # least recent first
        self._ids: dict[tuple, int] = {}
        self._next_id = 0

    def __len__(self) -> int:
        return len(self._lru)

    # ------------------------------------------------------------- lookup
    def get(self, tokens: Sequence[int], max_prefix_len: int | None = None) -> PrefixCacheMatch:
        """Longest cached prefix of `tokens` (at most max_prefix_len). The
        returned cache is the caller's: with paged entries it holds page
        references until its reset()."""
        if self.max_tokens == 0 or not tokens or not self._lru:
            return PrefixCacheMatch(0, None)
        limit = len(tokens) if max_prefix_len is None else min(len(tokens), max_prefix_len)
        if limit <= 0:
            return PrefixCacheMatch(0, None)
        bt = self.block_tokens
        node = self._root
        while (node.depth + 1) * bt <= limit:
            start = node.depth * bt
            child = node.next.get(tuple(tokens[start : start + bt]))
            if child is None:
                break
            node = child
        base = node.depth * bt
        probe = tuple(tokens[base : min(limit, base + bt)])
        # the longest extension into the next block, and who reaches it
        best, reach = 0, []
        for block, child in node.next.items():
            n = _shared_len(probe, block)
            if n > best:
                best, reach = n, [child.through]
            elif n == best and n > 0:
                reach.append(child.through)
        for eid, tail in node.tails.items():
            n = _shared_len(probe, tail)
            if n > best:
                best, reach = n, [(eid,)]
            elif n == best and n > 0:
                reach.append((eid,))
        length = base + best
        if length == 0:
            return PrefixCacheMatch(0, None)
        if best == 0:
            reach = [node.through]  # every prompt below this node shares `base` tokens
        winner = self._least_recent(reach)
        self._lru.move_to_end(winner)
        return PrefixCacheMatch(length, self._lru[winner].cache.slice(length))

    def _least_recent(self, groups) -> int:
        ids = set().union(*groups)
        for eid in self._lru:  # least recent first
            if eid in ids:
                return eid
        raise AssertionError("prefix index out of step with its entries")

    # ------------------------------------------------------------ storage
    def put(self, tokens: Sequence[int], cache) -> None:
        """Store the first min(len(tokens), cache.length, max_tokens) tokens.
        A paged entry takes its own page references (no copy); a Cache entry
        is cloned, as in the reference."""
        if self.max_tokens == 0 or not tokens or cache.length == 0:
            return
        n = min(len(tokens), cache.length, self.max_tokens)
        if n <= 0:
            return
        key = tuple(tokens[:n])
        stored = cache.slice(n, clone=True)
        old = self._ids.get(key)
        if old is not None:
            self._drop(old)
        eid = self._next_id
        self._next_id += 1
        bt = self.block_tokens
        node = self._root
        node.through.add(eid)
        for b in range(n // bt):
            edge = key[b * bt : (b + 1) * bt]
            child = node.next.get(edge)
            if child is None:
                child = _Block(node, edge, node.depth + 1)
                node.next[edge] = child
            node = child
            node.through.add(eid)
        if n % bt:
            node.tails[eid] = key[(n // bt) * bt :]
        self._lru[eid] = _Entry(key, stored, node)
        self._ids[key] = eid
        self.total_tokens += n
        while self.total_tokens > self.max_tokens and self._lru:
            self.evict_lru()

    def _drop(self, eid: int) -> None:
        """Unlinks entry `eid` from the index and releases its cache."""
        entry = self._lru.pop(eid)
        del self._ids[entry.key]
        self.total_tokens -= len(entry.key)
        node = entry.node
        node.tails.pop(eid, None)
        while node is not None:
            node.through.discard(eid)
            parent = node.parent
            if parent is not None and not node.through:
                del parent.next[node.edge]
            node = parent
        _release(entry.cache)

    def evict_lru(self) -> bool:
        """Drop the least recently used entry (returning its pages to the
        pool once no request shares them); False if the cache is empty."""
        if not self._lru:
            return False
        self._drop(next(iter(self._lru)))
        return True

    def clear(self) -> None:
        while self._lru:
            self._drop(next(iter(self._lru)))
