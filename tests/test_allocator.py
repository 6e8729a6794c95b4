"""Host-side pool bookkeeping of PagedKVCacheManager (CPU, no kernels).

Mirrors the reference's CPU allocator tests (tests/test_paged_cache.py:9-51:
page size 2, 2 layers, 1 kv head, head_dim 4, fp32) and the error
conditions of paged_cache.py (88-93, 113-139, 170-186, 206-234, 300-303),
plus the reference-counted prefix sharing this library adds.
"""

import pytest
import torch

from hayate_amd.paged_cache import PagedKVCacheManager


def make_manager(max_cache_tokens=8, page_size=2, max_requests=2):
    return PagedKVCacheManager(
        num_layers=2, num_kv_heads=1, head_dim=4, max_cache_tokens=max_cache_tokens,
        page_size=page_size, max_requests=max_requests, dtype=torch.float32, device="cpu",
    )


def test_constructor_validation():
    with pytest.raises(ValueError):
        make_manager(max_cache_tokens=0)
    with pytest.raises(ValueError):
        make_manager(page_size=3)
    with pytest.raises(ValueError):
        make_manager(max_requests=0)
    m = make_manager(max_cache_tokens=7)
    assert m.num_pages == 4 and m.capacity_tokens == 8
    assert tuple(m.k_cache.shape) == (2, 1, 1, 8, 4)


def test_lifo_page_order_and_release_reuses_the_same_pages():
    m = make_manager()
    h = m.allocate()
    m.reserve(h, 3)
    assert h.pages == [0, 1]  # fresh free list pops 0, 1, 2, ...
    original = list(h.pages)
    m.release(h)
    replacement = m.allocate()
    m.reserve(replacement, 3)
    assert set(replacement.pages) == set(original)  # test_paged_cache.py:39-42


def test_pool_reports_exhausted_pages():
    m = make_manager(max_cache_tokens=4)  # test_paged_cache.py:44-51
    first, second = m.allocate(), m.allocate()
    m.reserve(first, 4)
    with pytest.raises(MemoryError):
        m.reserve(second, 1)


def test_slots_capacity_and_handle_errors():
    m = make_manager(max_requests=1)
    h = m.allocate()
    with pytest.raises(MemoryError):
        m.allocate()
    with pytest.raises(MemoryError):
        m.reserve(h, 9)  # beyond capacity_tokens
    with pytest.raises(ValueError):
        m.reserve(h, -1)
    m.reserve(h, 2)
    h.length = 2
    with pytest.raises(ValueError):
        m.truncate(h, 3)
    m.release(h)
    m.release(h)  # idempotent
    for call in (lambda: m.reserve(h, 1), lambda: m.truncate(h, 0), lambda: m.snapshot(h)):
        with pytest.raises(RuntimeError):
            call()
    assert m.allocate().slot == h.slot


def test_truncate_returns_whole_pages():
    m = make_manager()
    h = m.allocate()
    m.reserve(h, 7)
    h.length = 7
    m.truncate(h, 3)
    assert len(h.pages) == 2 and h.length == 3
    assert m.free_page_count == 2


def test_begin_batch_validation_order_and_types():
    m = PagedKVCacheManager(1, 1, 4, 1024, 128, 3, torch.float32, "cpu")
    a, b = m.allocate(), m.allocate()
    with pytest.raises(ValueError):
        m.begin_batch([], 1)
    with pytest.raises(ValueError):
        m.begin_batch([a], 0)
    with pytest.raises(ValueError):
        m.begin_batch([a, a], 1)
    m.release(b)
    with pytest.raises(RuntimeError):
        m.begin_batch([a, b], 1)
    c = m.allocate()
    with pytest.raises(MemoryError):
        m.begin_batch([a, c], 1025)  # beyond capacity
    m.reserve(a, 1024)
    with pytest.raises(MemoryError):
        m.begin_batch([c], 1)  # pool full


def test_begin_batch_rejects_small_pages_like_the_reference():
    m = make_manager()
    h = m.allocate()
    with pytest.raises(ValueError):
        m.begin_batch([h], 1)


def test_commit_requires_reserved_space():
    m = make_manager()
    h = m.allocate()
    with pytest.raises(RuntimeError):
        m.commit_batch([h], 1)
    m.reserve(h, 1)
    m.commit_batch([h], 1)
    assert h.length == 1


def test_fork_shares_pages_and_refcounts():
    m = make_manager(max_cache_tokens=16, max_requests=4)
    parent = m.allocate()
    m.reserve(parent, 5)
    parent.length = 5
    child = m.fork(parent)  # all 5 tokens: 3 pages, the last one partly filled
    assert child.length == 5 and child.pages == parent.pages
    assert [m.page_refcount(p) for p in parent.pages] == [2, 2, 2]
    half = m.fork(parent, 3)  # 3 tokens: the first 2 pages
    assert half.length == 3 and half.pages == parent.pages[:2]
    assert [m.page_refcount(p) for p in parent.pages] == [3, 3, 2]
    with pytest.raises(ValueError):
        m.fork(parent, 6)
    m.release(parent)
    m.release(half)
    assert [m.page_refcount(p) for p in child.pages] == [1, 1, 1]
    assert m.free_page_count == 8 - 3
    m.release(child)
    assert m.free_page_count == 8


def test_shared_prefix_references_pages_without_copies():
    """share() / PagedPrefix / allocate_for_request(prefix): the zero-copy
    path of the prefix cache is pure page bookkeeping."""
    m = make_manager(max_cache_tokens=16, max_requests=4)
    owner = m.allocate()
    m.reserve(owner, 5)
    owner.length = 5
    prefix = m.share(owner, 4)
    assert prefix.length == 4 and prefix.pages == owner.pages[:2]
    assert [m.page_refcount(p) for p in owner.pages] == [2, 2, 1]
    part = prefix.slice(3, clone=True)
    assert part.length == 3 and part.pages == owner.pages[:2]
    assert [m.page_refcount(p) for p in owner.pages] == [3, 3, 1]
    with pytest.raises(ValueError):
        prefix.slice(5)
    req = m.allocate_for_request(part)  # no copy: the request shares the pages
    assert req.length == 3 and req.pages == owner.pages[:2]
    assert [m.page_refcount(p) for p in owner.pages] == [4, 4, 1]
    part.reset()
    part.reset()  # idempotent
    prefix.reset()
    m.release(owner)
    assert [m.page_refcount(p) for p in req.pages] == [1, 1]
    assert m.free_page_count == 8 - 2
    m.release(req)
    assert m.free_page_count == 8
    # a prefix only attaches to the pool its pages belong to
    h = m.allocate()
    m.reserve(h, 2)
    h.length = 2
    with pytest.raises(ValueError):
        make_manager().allocate_for_request(m.share(h))


def test_claim_pages_takes_specific_free_pages():
    m = make_manager(max_cache_tokens=16)
    h = m.allocate()
    m.claim_pages(h, [5, 2])
    assert h.pages == [5, 2] and m.free_page_count == 6
    g = m.allocate()
    with pytest.raises(ValueError):
        m.claim_pages(g, [2])
    m.reserve(g, 2)
    assert g.pages == [0]


def test_data_operations_refuse_a_cpu_pool():
    """No CPU implementation exists: data movement needs the HIP library."""
    m = PagedKVCacheManager(1, 1, 128, 1024, 128, 2, torch.bfloat16, "cpu")
    h = m.allocate()
    m.reserve(h, 10)
    h.length = 10
    with pytest.raises(RuntimeError):
        m.snapshot(h)
    batch = m.begin_batch([h], 1)
    k = torch.zeros(1, 1, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        batch.write_layer(0, k, k)
    with pytest.raises(RuntimeError):
        batch.attend_layer(torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16), 0)


def test_copy_on_write_needs_a_device_pool():
    m = PagedKVCacheManager(1, 1, 128, 1024, 128, 3, torch.bfloat16, "cpu")
    parent = m.allocate()
    m.reserve(parent, 256)
    parent.length = 256
    child = m.fork(parent, 256)
    m.truncate(child, 200)  # the next append would land in a shared page
    with pytest.raises(RuntimeError):
        m.begin_batch([child], 1)


def test_begin_batch_counts_copy_on_write_pages_before_changing_anything(monkeypatch):
    """A batch whose appends need new pages and a copy of a shared page
    either gets all of them or raises before any handle changes (the
    reference's begin_batch checks its page need up front,
    paged_cache.py:218-234). The copy itself is a device operation; the
    device check is stubbed so the bookkeeping runs on a CPU pool."""
    import hayate_amd.paged_cache as pc

    monkeypatch.setattr(pc, "_require_hip", lambda t, what: None)
    m = PagedKVCacheManager(1, 1, 128, 640, 128, 4, torch.bfloat16, "cpu")
    parent = m.allocate()
    m.reserve(parent, 256)
    parent.length = 256
    child = m.fork(parent, 256)
    m.truncate(child, 200)  # its next append lands in the shared second page
    a = m.allocate()
    m.reserve(a, 128)
    a.length = 128  # its next append needs a new page
    spare = m.allocate()
    m.reserve(spare, 1)
    assert m.free_page_count == 1
    before = (list(a.pages), list(child.pages), [m.page_refcount(p) for p in range(5)])
    with pytest.raises(MemoryError):
        m.begin_batch([a, child], 1)
    assert (list(a.pages), list(child.pages), [m.page_refcount(p) for p in range(5)]) == before
    assert m.free_page_count == 1
    # with a second free page both the new page and the copy fit
    m.release(spare)
    shared = parent.pages[1]
    m.begin_batch([a, child], 1)
    assert len(a.pages) == 2 and child.pages[1] != shared
    assert m.page_refcount(shared) == 1 and m.page_refcount(child.pages[1]) == 1
    assert m.page_refcount(child.pages[0]) == 2
    assert m.free_page_count == 0


def test_copy_on_write_batch_with_two_sharers_copies_once(monkeypatch):
    """Two handles sharing one page both append into it in one batch: the
    first copies it, the last sharer then writes the original in place, so
    the pre-check needs exactly one free page."""
    import hayate_amd.paged_cache as pc

    monkeypatch.setattr(pc, "_require_hip", lambda t, what: None)
    m = PagedKVCacheManager(1, 1, 128, 384, 128, 3, torch.bfloat16, "cpu")
    parent = m.allocate()
    m.reserve(parent, 256)
    parent.length = 256
    child = m.fork(parent, 256)
    m.truncate(parent, 200)
    m.truncate(child, 150)
    assert m.free_page_count == 1
    m.begin_batch([parent, child], 1)
    assert parent.pages[1] != child.pages[1]
    assert m.free_page_count == 0
    assert m.page_refcount(parent.pages[1]) == 1 and m.page_refcount(child.pages[1]) == 1
    assert m.page_refcount(parent.pages[0]) == 2


def test_commit_tick_needs_one_length_per_handle():
    m = make_manager(max_requests=2)
    a, b = m.allocate(), m.allocate()
    m.reserve(a, 2)
    m.reserve(b, 2)
    with pytest.raises(ValueError):
        m.commit_tick([a, b], [1])
    assert a.length == 0 and b.length == 0
