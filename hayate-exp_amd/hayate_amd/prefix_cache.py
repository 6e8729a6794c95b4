"""LRU prompt-prefix cache over shared KV pages.

Same interface and policy as the reference's hayate/engine/prefix_cache.py:
``get(tokens, max_prefix_len)`` returns the longest cached prefix
(:32-59), ``put(tokens, cache)`` stores an entry under a token budget
(:61-80) and the least recently used entries are evicted past the budget
(:96-100). The difference is the entry: the reference stores a cloned
contiguous Cache (``cache.slice(store_len, clone=True)``, :72) and every hit
copies it back into the pool (paged_cache.py:153-166); here an entry is a
PagedPrefix that holds references to the pool pages of the prompt, a hit
is another reference (``slice``), and the request that reuses it shares the
pages (``PagedKVCacheManager.allocate_for_request``). Entries stay
immutable because shared pages are copy-on-write.

Entries given as a plain Cache (the reference's format) are kept as they
are, so the class also works as a drop-in for the reference's.
"""

from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass
from typing import Any, Sequence


@dataclass(frozen=True)
class PrefixCacheMatch:
    """Cached token count and cache found for one prompt (prefix_cache.py:10-15)."""

    length: int
    cache: Any


def _release(entry) -> None:
    reset = getattr(entry, "reset", None)
    if reset is not None:
        reset()


class PrefixCache:
    """Least-recently-used prompt-prefix cache with a token budget."""

    def __init__(self, max_tokens: int):
        if max_tokens < 0:
            raise ValueError("prefix cache token budget must be non-negative")
        self.max_tokens = max_tokens
        self.total_tokens = 0
        self._entries: OrderedDict[tuple[int, ...], Any] = OrderedDict()

    def __len__(self) -> int:
        return len(self._entries)

    def get(self, tokens: Sequence[int], max_prefix_len: int | None = None) -> PrefixCacheMatch:
        """Longest cached prefix of `tokens` (at most max_prefix_len). The
        returned cache is the caller's: with paged entries it holds page
        references until its reset()."""
        if self.max_tokens == 0 or not tokens or not self._entries:
            return PrefixCacheMatch(0, None)
        token_tuple = tuple(tokens)
        limit = len(token_tuple) if max_prefix_len is None else min(len(token_tuple),
                                                                    max_prefix_len)
        if limit <= 0:
            return PrefixCacheMatch(0, None)
        best_key = None
        best_len = 0
        for cached_tokens, cache in self._entries.items():
            common = self._common_prefix_len(token_tuple, cached_tokens, limit)
            if common > best_len and common <= cache.length:
                best_key = cached_tokens
                best_len = common
                if best_len == limit:
                    break
        if best_key is None:
            return PrefixCacheMatch(0, None)
        self._entries.move_to_end(best_key)
        return PrefixCacheMatch(best_len, self._entries[best_key].slice(best_len))

    def put(self, tokens: Sequence[int], cache) -> None:
        """Store the first min(len(tokens), cache.length, max_tokens) tokens.
        A paged entry takes its own page references (no copy); a Cache entry
        is cloned, as in the reference."""
        if self.max_tokens == 0 or not tokens or cache.length == 0:
            return
        store_len = min(len(tokens), cache.length, self.max_tokens)
        if store_len <= 0:
            return
        key = tuple(tokens[:store_len])
        entry = cache.slice(store_len, clone=True)
        existing = self._entries.pop(key, None)
        if existing is not None:
            self.total_tokens -= len(key)
            _release(existing)
        self._entries[key] = entry
        self.total_tokens += len(key)
        self._evict_to_budget()

    def evict_lru(self) -> bool:
        """Drop the least recently used entry (returning its pages to the
        pool once no request shares them); False if the cache is empty."""
        if not self._entries:
            return False
        tokens, entry = self._entries.popitem(last=False)
        self.total_tokens -= len(tokens)
        _release(entry)
        return True

    def clear(self) -> None:
        for entry in self._entries.values():
            _release(entry)
        self._entries.clear()
        self.total_tokens = 0

    @staticmethod
    def _common_prefix_len(left: Sequence[int], right: Sequence[int], limit: int) -> int:
        count = 0
        max_len = min(len(left), len(right), limit)
        while count < max_len and left[count] == right[count]:
            count += 1
        return count

    def _evict_to_budget(self) -> None:
        while self.total_tokens > self.max_tokens and self._entries:
            self.evict_lru()
