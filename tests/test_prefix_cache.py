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


class _Stored:
    """A stand-in entry: remembers which put() it came from and its length;
    reset() records that the cache let go of it."""

    released = []

    def __init__(self, tag, length):
        self.tag, self.length = tag, length

    def slice(self, n, clone=False):
        return _Stored(self.tag, n)

    def reset(self):
        _Stored.released.append(self.tag)


class _LinearScan:
    """The reference's lookup, restated as the plain scan it is
    (prefix_cache.py:32-100): compare the prompt with every stored key in
    least-recently-used order, keep the first strictly longer common prefix
    (at most the limit), move the hit to the most recent end; put replaces
    an identical key and evicts from the least recent end past the budget."""

    def __init__(self, budget):
        self.budget, self.keys, self.tags = budget, [], []

    def get(self, tokens, limit):
        limit = len(tokens) if limit is None else min(len(tokens), limit)
        best, at = 0, None
        for i, key in enumerate(self.keys):
            n = 0
            while n < min(len(key), limit) and key[n] == tokens[n]:
                n += 1
            if n > best:
                best, at = n, i
        if at is None:
            return 0, None
        self.keys.append(self.keys.pop(at))
        self.tags.append(self.tags.pop(at))
        return best, self.tags[-1]

    def put(self, tokens, tag, length):
        n = min(len(tokens), length, self.budget)
        key = tuple(tokens[:n])
        if key in self.keys:
            i = self.keys.index(key)
            del self.keys[i], self.tags[i]
        self.keys.append(key)
        self.tags.append(tag)
        while sum(map(len, self.keys)) > self.budget:
            del self.keys[0], self.tags[0]


@pytest.mark.parametrize("block", [1, 3, 16, 128])
def test_block_index_agrees_with_a_linear_scan(block):
    """Random prompt families (shared stems, branches inside and at block
    edges, exact repeats, prompts longer than the budget) through a random
    mix of put/get/evict: the block-indexed cache returns the same match
    length and the same entry as the linear scan, holds the same keys in
    the same LRU order and releases exactly the entries it drops."""
    import random

    rng = random.Random(block)
    stems = [[rng.randrange(6) for _ in range(rng.randrange(1, 300))] for _ in range(5)]

    def prompt():
        s = rng.choice(stems)
        cut = rng.randrange(len(s) + 1)
        tail = [rng.randrange(6) for _ in range(rng.randrange(0, 200))]
        return s[:cut] + tail or [1]

    for budget in (0, 50, 700, 5000):
        cache, scan = PrefixCache(budget, block_tokens=block), _LinearScan(budget)
        _Stored.released = []
        live, stored = set(), set()
        for step in range(400):
            op = rng.random()
            if op < 0.45:
                p = prompt()
                length = rng.randrange(1, len(p) + 2)
                cache.put(p, _Stored(step, length))
                if budget > 0:
                    scan.put(p, step, length)
                    stored.add(step)
            elif op < 0.95:
                p = prompt()
                limit = rng.choice([None, rng.randrange(0, len(p) + 3)])
                got = cache.get(p, max_prefix_len=limit)
                want_len, want_tag = scan.get(p, limit) if budget else (0, None)
                assert got.length == want_len, (step, got.length, want_len)
                assert (got.cache.tag if got.cache else None) == want_tag
                if got.cache is not None:
                    assert got.cache.length == want_len
            elif budget and scan.keys:
                assert cache.evict_lru()
                del scan.keys[0], scan.tags[0]
            assert len(cache) == len(scan.keys) or budget == 0
            assert cache.total_tokens == sum(map(len, scan.keys)) or budget == 0
            live = set(scan.tags) if budget else set()
        assert [e.cache.tag for e in cache._lru.values()] == list(live and scan.tags)
        released = set(_Stored.released)
        assert not released & live and released == stored - live
        cache.clear()
        assert len(cache) == 0 and cache.total_tokens == 0
        assert not cache._root.next and not cache._root.tails and not cache._root.through
