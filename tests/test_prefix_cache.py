"""PrefixCache (hayate_amd/prefix_cache.py) on the CPU: the reference's
policy (hayate/engine/prefix_cache.py: longest match, LRU, token budget) and
its immutability test (tests/test_cache.py:26-39), for both entry kinds —
a cloned Cache as in the reference, and PagedPrefix page references."""

import pytest
import torch

from hayate_amd import Cache, PagedKVCacheManager, PrefixCache


def test_cache_entries_are_immutable_compact_copies():
    """tests/test_cache.py:26-39: an entry does not change when the active
    cache it came from changes, and it is compact (capacity == length)."""
    values = torch.arange(24).reshape(1, 2, 3, 4)
    storage = torch.zeros(1, 2, 8, 4, dtype=values.dtype)
    storage[:, :, :3] = values
    active = Cache.from_tensors(storage[:, :, :3], storage[:, :, :3])
    prefixes = PrefixCache(max_tokens=16)
    prefixes.put([1, 2, 3], active)
    storage.zero_()
    match = prefixes.get([1, 2, 3, 4])
    assert match.length == 3
    assert match.cache.capacity == 3
    torch.testing.assert_close(match.cache.k, values)


def test_longest_match_limit_and_lru_budget():
    c = PrefixCache(max_tokens=8)
    mk = lambda n: Cache.from_tensors(torch.zeros(1, 1, n, 2), torch.zeros(1, 1, n, 2))
    c.put([1, 2, 3], mk(3))
    c.put([1, 2, 9, 9], mk(4))
    assert c.total_tokens == 7
    m = c.get([1, 2, 3, 4])
    assert m.length == 3
    assert c.get([1, 2, 3, 4], max_prefix_len=2).length == 2
    assert c.get([7]).cache is None
    # the limited lookup stopped at [1, 2, 9, 9] (first entry reaching the
    # limit), so [1, 2, 3] is now the least recently used and goes first
    c.put([5, 6, 7, 8], mk(4))
    assert c.total_tokens == 8 and len(c) == 2
    assert c.get([1, 2, 3, 4]).length == 2  # only [1, 2] of [1, 2, 9, 9] is left
    c.clear()
    assert c.total_tokens == 0 and c.get([1, 2, 3]).cache is None
    with pytest.raises(ValueError):
        PrefixCache(-1)


def test_paged_entries_hold_and_release_page_references():
    m = PagedKVCacheManager(2, 1, 4, 32, 4, 4, torch.float32, "cpu")
    h = m.allocate()
    m.reserve(h, 10)
    h.length = 10  # pages: 3 (10 tokens)
    c = PrefixCache(max_tokens=12)
    shared = m.share(h, 10)
    c.put(list(range(10)), shared)
    shared.reset()
    assert [m.page_refcount(p) for p in h.pages] == [2, 2, 2]
    hit = c.get(list(range(10)) + [99], max_prefix_len=9)
    assert hit.length == 9 and hit.cache.pages == h.pages[:3]
    assert [m.page_refcount(p) for p in h.pages] == [3, 3, 3]
    req = m.allocate_for_request(hit.cache)  # the request shares the pages
    hit.cache.reset()
    assert req.length == 9 and [m.page_refcount(p) for p in h.pages] == [3, 3, 3]
    m.release(h)
    m.release(req)
    assert [m.page_refcount(p) for p in range(3)] == [1, 1, 1]  # the entry's
    # a second entry past the budget evicts the first and frees its pages
    g = m.allocate()
    m.reserve(g, 4)
    g.length = 4
    other = m.share(g)
    c.put([50, 51, 52, 53], other)
    other.reset()
    assert len(c) == 1 and c.total_tokens == 4
    assert m.free_page_count == m.num_pages - 1
    assert c.evict_lru() and not c.evict_lru()
    m.release(g)
    assert m.free_page_count == m.num_pages
