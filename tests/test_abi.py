"""The C ABI without a GPU: the library loads, exports every function the
header declares, the host-only planner behaves, and argument validation
returns error codes before any device work."""

import ctypes
import os
import re

import numpy as np
import pytest

from hayate_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hayate_attn.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(hy_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_function():
    lib = _native.lib()
    names = declared_functions()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_native.EXPORTED_SYMBOLS)
    assert lib.hy_version() >= 1


def test_symbols_are_plain_c_in_the_dynamic_table():
    out = os.popen(f"nm -D --defined-only {_native.LIB_PATH}").read()
    for name in declared_functions():
        assert re.search(rf"\bT {name}$", out, re.M), name


def plan(q, kv, hq=32, hkv=8, page=128, cus=256, split=0):
    return _native.plan_tick(np.array(q), np.array(kv), hq, hkv, page, cus, split)


W = 2  # waves per decode workgroup: partials per piece
PIECE_COST = 64  # tokens the planner charges a decode piece after a chunk's first


def chunks_and_pieces(p):
    return p.decode[: p.n_chunks], p.decode[p.n_chunks :]


@pytest.mark.parametrize("split", [0, 96, 256, 1000])
def test_plan_decode_covers_every_token_once(split):
    rng = np.random.default_rng(0)
    kv = rng.integers(1, 9000, size=40)
    p = plan([1] * 40, kv, split=split)
    assert len(p.prefill) == 0
    chunks, pieces = chunks_and_pieces(p)
    # chunks own consecutive runs of pieces; slice offsets restart per chunk
    assert chunks[0, 0] == 0 and chunks[-1, 1] == len(pieces)
    assert (chunks[1:, 0] == chunks[:-1, 1]).all() and (chunks[:, 1] > chunks[:, 0]).all()
    nsl = (pieces[:, 2] - pieces[:, 1] + 31) // 32
    for c in chunks:
        part = slice(c[0], c[1])
        assert (pieces[part, 4] == np.concatenate([[0], np.cumsum(nsl[part])[:-1]])).all()
        assert c[2] == nsl[part].sum()
    assert (pieces[:, 3] == W * np.arange(len(pieces))).all()
    # chunk records repeat their first piece
    first = pieces[chunks[:, 0]]
    assert (chunks[:, 3:6] == first[:, 0:3]).all() and (chunks[:, 6] == first[:, 3]).all()
    assert (chunks[:, 7] == first[:, 5]).all()
    assert (pieces[:, 5] == pieces[:, 0]).all()  # q row of sequence b is b (q_len 1)
    assert (pieces[:, 6] == kv[pieces[:, 0]] - 1).all()  # position of the query token
    assert (pieces[:, 7] == (pieces[:, 2] == kv[pieces[:, 0]])).all()  # holds that token
    merged = {int(m[0]): m for m in p.merge}
    assert sorted(merged) == list(range(40))
    for b in range(40):
        idx = np.nonzero(pieces[:, 0] == b)[0]
        rows = pieces[idx]
        assert (np.diff(idx) == 1).all()
        assert rows[0, 1] == 0 and rows[-1, 2] == kv[b]
        assert (rows[1:, 1] == rows[:-1, 2]).all()
        assert (rows[:, 1] % 32 == 0).all() and (rows[:, 2] > rows[:, 1]).all()
        m = merged[b]
        assert m[1] == W * idx[0] and m[2] == W * len(idx)
        assert m[3] == b  # the sequence's query row (q_start[b], q_len 1)
    assert p.n_slots == W * len(pieces) == int(p.merge[:, 2].sum())
    tokens = [int((pieces[c[0]:c[1], 2] - pieces[c[0]:c[1], 1]).sum()) for c in chunks]
    if split:
        assert len(chunks) == -(-int(kv.sum()) // split)
    else:
        assert len(chunks) == 256 // 8
    # equal chunk costs (slices' tokens plus 64 per piece after a chunk's
    # first) up to the rounding of each cut to 32 tokens at either end and a
    # partial last slice
    cost = chunks[:, 2] * 32 + PIECE_COST * (chunks[:, 1] - chunks[:, 0] - 1)
    assert cost.max() - cost.min() <= 128


def test_plan_decode_chunks_with_more_pieces_get_fewer_tokens():
    """Batch-32 decode lengths (256-4,096): each piece after a chunk's first
    costs a partial flush and a query switch, so the cut gives chunks with
    more pieces fewer tokens, and no chunk costs more than an equal-token
    cut's costliest chunk would."""
    rng = np.random.default_rng(1002)
    kv = rng.integers(256, 4097, size=32)
    p = plan([1] * 32, kv)
    chunks, pieces = chunks_and_pieces(p)
    n = chunks[:, 1] - chunks[:, 0]
    tokens = np.array([int((pieces[c[0]:c[1], 2] - pieces[c[0]:c[1], 1]).sum()) for c in chunks])
    assert n.max() >= 3 and n.min() == 1
    assert tokens[n == 1].mean() > tokens[n >= 3].mean() + 64
    cost = chunks[:, 2] * 32 + PIECE_COST * (n - 1)
    equal_share = -(-int(kv.sum()) // len(chunks))
    assert cost.max() <= equal_share + 32 + PIECE_COST * (n.max() - 1)


def test_plan_chunk_holds_at_most_the_query_table():
    # 1000 one-token contexts: chunks close at 32 pieces (G = 4)
    p = plan([1] * 1000, [1] * 1000)
    chunks, pieces = chunks_and_pieces(p)
    assert len(pieces) == 1000
    assert ((chunks[:, 1] - chunks[:, 0]) <= 32).all()
    assert chunks[0, 0] == 0 and chunks[-1, 1] == 1000
    assert (chunks[1:, 0] == chunks[:-1, 1]).all()


@pytest.mark.parametrize("seed", range(3))
def test_plan_chunks_stay_balanced_when_the_piece_limit_closes_chunks(seed):
    """G = 16 (32 q heads over 2 kv heads): the query table holds 8 pieces,
    so 256 sequences close chunks early; the cuts after such a close follow
    the stream position, so the largest chunk stays near the mean (cut
    targets counted in closed chunks made it 1.34x)."""
    rng = np.random.default_rng(seed)
    kv = rng.integers(256, 4097, size=256)
    p = plan([1] * 256, kv, hq=32, hkv=2)
    chunks, pieces = chunks_and_pieces(p)
    assert ((chunks[:, 1] - chunks[:, 0]) <= 8).all()
    tokens = np.array([int((pieces[c[0]:c[1], 2] - pieces[c[0]:c[1], 1]).sum()) for c in chunks])
    assert tokens.sum() == kv.sum()
    assert tokens.max() <= 1.05 * tokens.mean()


def test_plan_chunk_cut_rounds_to_32_tokens():
    p = plan([1], [300], split=256)
    chunks, pieces = chunks_and_pieces(p)
    assert [tuple(r[1:3]) for r in pieces] == [(0, 160), (160, 300)]
    assert [tuple(c[:3]) for c in chunks] == [(0, 1, 5), (1, 2, 5)]
    assert p.n_slots == 2 * W


def check_prefill_cover(q, kv, p):
    """Every query tile's key range [0, cache + q1) is covered once by its
    parts, which start on 64-key steps, carry the sequence's query row and
    cached length, and are dispatched longest first; a split tile has one
    merge item over its parts' partial slots."""
    pre = p.prefill
    tile = _native.lib().hy_prefill_tile_rows() // 4
    lengths = pre[:, 4] - pre[:, 3]
    assert (lengths[:-1] >= lengths[1:]).all()  # longest first
    assert (pre[:, 3] % 64 == 0).all()
    merges = {(int(m[0]), int(m[1])): m for m in p.prefill_merge}
    n_parts = 0
    for s_, ql in enumerate(q):
        if ql <= 1:
            assert not (pre[:, 0] == s_).any()
            continue
        cache = kv[s_] - ql
        rows = pre[pre[:, 0] == s_]
        for q0 in range(0, ql, tile):
            q1 = min(ql, q0 + tile)
            parts = rows[(rows[:, 1] == q0)]
            n_parts += len(parts)
            assert (parts[:, 2] == q1).all()
            assert (parts[:, 6] == sum(q[:s_])).all()  # packed query row of the sequence
            assert (parts[:, 7] == cache).all()  # cached keys before the chunk
            parts = parts[np.argsort(parts[:, 3])]
            assert parts[0, 3] == 0 and parts[-1, 4] == cache + q1
            assert (parts[1:, 3] == parts[:-1, 4]).all() and (parts[:, 4] > parts[:, 3]).all()
            if len(parts) == 1:
                assert parts[0, 5] == -1 and (s_, q0) not in merges
            else:
                m = merges[(s_, q0)]
                assert m[2] == q1 and m[4] == len(parts)
                assert m[5] == sum(q[:s_])  # q_start of the sequence
                assert sorted(parts[:, 5]) == list(range(m[3], m[3] + len(parts)))
    assert n_parts == len(pre)
    assert p.n_prefill_slots == int((pre[:, 5] >= 0).sum())
    return merges


def test_plan_prefill_tiles_cover_every_query_and_key_once():
    q = [512, 512, 1, 3, 512]
    kv = [512, 4096, 700, 10, 8192]
    p = plan(q, kv)
    _, pieces = chunks_and_pieces(p)
    assert len(pieces) >= 1 and (pieces[:, 0] == 2).all()
    # the 8192-token tile must have been split to balance the tick
    assert len(check_prefill_cover(q, kv, p)) > 0


@pytest.mark.parametrize("seed", range(6))
def test_plan_list_sizes_fit_a_fixed_launch(seed):
    """The bounds a replayed graph sizes its padded lists by
    (hayate_amd/tick_graph.py): a plan has at most one decode chunk per CU
    and kv head, at most one prefill item per unsplit query tile plus one per
    partial slot, at most one prefill merge item per query tile, and one
    decode merge item per decode sequence."""
    rng = np.random.default_rng(300 + seed)
    n = int(rng.integers(1, 20))
    q = [1 if rng.random() < 0.5 else int(rng.integers(2, 1025)) for _ in range(n)]
    kv = [x + int(rng.integers(0, 16000)) for x in q]
    for cus in (64, 256):
        p = plan(q, kv, cus=cus)
        tile = _native.lib().hy_prefill_tile_rows() // 4
        n_tiles = sum(-(-x // tile) for x in q if x > 1)
        split_tiles = len(p.prefill_merge)
        assert len(p.prefill) == (n_tiles - split_tiles) + p.n_prefill_slots
        assert split_tiles <= n_tiles
        assert p.n_chunks <= max(1, cus // 8)
        assert len(p.merge) == sum(1 for x in q if x == 1)


@pytest.mark.parametrize("shape", ["prefill_4x512", "mixed_tick", "random0", "random1", "random2"])
def test_plan_prefill_cover_across_shapes(shape):
    """The split rules the planner picks from (even parts, or full parts of
    a cap plus a shorter remainder) on the benchmark shapes and on random
    chunked prefills."""
    if shape == "prefill_4x512":
        q, kv = [512] * 4, [512, 1536, 2560, 4096]
    elif shape == "mixed_tick":
        offs = [1280, 1920, 1280, 3072, 2944, 1152, 3968, 4096]
        q, kv = [512] * 8 + [1] * 56, [o + 512 for o in offs] + [3000] * 56
    else:
        rng = np.random.default_rng(int(shape[-1]))
        n = int(rng.integers(1, 12))
        q = rng.integers(2, 1025, size=n).tolist()
        kv = [x + int(rng.integers(0, 20000)) for x in q]
    merges = check_prefill_cover(q, kv, plan(q, kv))
    if shape == "prefill_4x512":
        # the offset-3584 tiles (57-64 steps) cannot run whole on 32 CUs per kv head
        assert any(k[0] == 3 for k in merges)


def test_plan_rejects_bad_input():
    with pytest.raises(ValueError):
        plan([2], [1])  # kv_len < q_len
    with pytest.raises(ValueError):
        plan([1], [5], hq=6, hkv=4)
    with pytest.raises(NotImplementedError):
        plan([1], [5], page=48)


def test_workspace_size():
    assert _native.decode_workspace_bytes(0, 32, 128) == 0
    n = _native.decode_workspace_bytes(3, 32, 128)
    assert n % 256 == 0 and n >= 3 * 32 * 130 * 4


def test_entry_points_validate_before_touching_the_device():
    lib = _native.lib()
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    # head_dim 64 is not built
    rc = lib.hy_kv_append(fake, fake, 0, fake, 0, 0, 0, fake, 0, 0, 0, fake, fake, fake, 0,
                          1, 1, 8, 64, 128, None)
    assert rc == _native.HY_EUNSUPPORTED and "head_dim" in _native.last_error()
    # null pointers
    rc = lib.hy_kv_append(None, fake, 0, fake, 0, 0, 0, fake, 0, 0, 0, fake, fake, fake, 0,
                          1, 1, 8, 128, 128, None)
    assert rc == _native.HY_EINVAL
    # page size not a multiple of 32
    rc = lib.hy_page_gather(fake, 0, 0, fake, 10, fake, 1, 8, 128, 100, None)
    assert rc == _native.HY_EUNSUPPORTED
    # GQA group 3 is not built
    rc = lib.hy_paged_decode(fake, 0, 0, 0, fake, 0, 0, 0, fake, fake, 0, fake, 0, fake,
                             fake, 1, 0, None, 0, 1, 6, 2, 128, 128, 0.1, None)
    assert rc == _native.HY_EUNSUPPORTED
    # workspace too small for the slots
    rc = lib.hy_paged_decode(fake, 0, 0, 0, fake, 0, 0, 0, fake, fake, 0, fake, 0, fake,
                             fake, 2, 2, fake, 100, 1, 32, 8, 128, 128, 0.1, None)
    assert rc == _native.HY_ENOSPACE
    with pytest.raises(MemoryError):
        _native.check(rc, "hy_paged_decode")
    rc = lib.hy_paged_decode_merge(fake, 0, 0, 0, fake, fake, 1, 2, fake, 100, 32, 128, None)
    assert rc == _native.HY_ENOSPACE
    rc = lib.hy_paged_prefill_merge(fake, 0, 0, 0, fake, fake, 1, 2, fake, 100, 32, 8, 128,
                                    None)
    assert rc == _native.HY_ENOSPACE
    rc = lib.hy_paged_prefill_merge(fake, 0, 0, 0, fake, fake, 1, 2, fake, 1 << 30, 24, 8, 128,
                                    None)
    assert rc == _native.HY_EUNSUPPORTED
    # nothing to do is success, even with null buffers
    assert lib.hy_paged_prefill(None, 0, 0, 0, None, 0, 0, 0, None, None, 0, None, 0, None,
                                None, None, 0, 0, None, 0, 1, 32, 8, 128, 128, 0.1,
                                None) == 0
    assert lib.hy_paged_decode_merge(None, 0, 0, 0, None, None, 0, 0, None, 0, 32, 128,
                                     None) == 0
    assert lib.hy_paged_prefill_merge(None, 0, 0, 0, None, None, 0, 0, None, 0, 32, 8, 128,
                                      None) == 0
    assert lib.hy_last_error() == b""


def test_plan_short_decode_spreads_over_64_token_chunks():
    """A lone short context still uses many workgroups: chunks of at least
    64 tokens (two 32-token slices), one per CU and kv head at most."""
    p = plan([1], [512])
    chunks, pieces = chunks_and_pieces(p)
    assert len(chunks) == 512 // 64
    assert (pieces[:, 2] - pieces[:, 1] == 64).all()
    p = plan([1] * 4, [4096] * 4)
    assert len(plan([1] * 4, [4096] * 4).decode) - p.n_chunks >= 4
    assert p.n_chunks == 256 // 8  # capped at one chunk per CU and kv head


def test_noalloc_rejects_merge_items_without_decode_items():
    """With no decode items the static scratch holds the previous call's
    partials; merging them would be silent garbage, so it is an argument
    error, returned before any device work."""
    lib = _native.lib()
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    args = [fake, 0, 0, 0, fake, 0, 0, 0, fake, 0, 0, 0, fake, 0, 0, 0, fake, fake, 1e-6, 1e-6,
            fake, fake, 40960, fake, 0, 0, 0, fake, fake, 0, fake, 0, fake, fake,
            fake, 0, fake, 3, 4, 1, 32, 8, 128, 128, 0.1, None]
    rc = lib.hy_paged_decode_append_noalloc(*args)
    assert rc == _native.HY_EINVAL
    assert "stale" in _native.last_error()
    with pytest.raises(ValueError):
        _native.check(rc, "hy_paged_decode_append_noalloc")


def test_plan_with_default_cu_count_sizes_its_buffers():
    """num_cus <= 0 means 256 CUs to the planner; the record buffers are
    sized the same way, so a deep decode batch plans without ENOSPACE."""
    rng = np.random.default_rng(5)
    for n in (1, 7, 32, 64):
        kv = rng.integers(1, 12000, size=n)
        p = plan([1] * n, kv, cus=0)
        ref = plan([1] * n, kv, cus=256)
        assert p.n_chunks == ref.n_chunks
        assert np.array_equal(p.decode, ref.decode) and np.array_equal(p.merge, ref.merge)
