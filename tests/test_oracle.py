"""Pins the oracle (oracle/paged_ref.py) before anything is compared with it.

Each oracle function is checked against something that does not share its
code: a torch library routine (bf16 casts, F.rms_norm, index ops,
scaled_dot_product_attention with a boolean mask and enable_gqa, exactly the
comparison of the reference's tests/test_paged_cache.py:95-112), a brute-force
loop, or a closed form (rotation as complex multiplication, single-key and
uniform-score attention, permutation invariance). Mutation checks show that
a dropped term, a swapped operand or a wrong page fails the checks.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import paged_ref as R


def rng(seed):
    return np.random.default_rng(seed)


# ----------------------------------------------------------------- bf16 casts
def test_bf16_cast_matches_torch_bit_for_bit():
    g = torch.Generator().manual_seed(0)
    x = torch.cat([
        torch.randn(20000, generator=g) * 10,
        torch.randn(2000, generator=g) * 1e-38,      # subnormal range
        torch.tensor([0.0, -0.0, float("inf"), -float("inf"), 3.3e38, -3.3e38]),
        # exact ties: bf16 value + half an ulp, both parities
        torch.tensor([1.0 + 2**-8, 1.0 + 3 * 2**-8, -(1.0 + 2**-8), 2.0 + 2**-7]),
    ])
    ours = R.f32_to_bf16(x.numpy())
    theirs = R.torch_bf16_to_bits(x.to(torch.bfloat16))
    assert np.array_equal(ours, theirs)
    assert np.array_equal(R.bf16_to_f32(theirs), x.to(torch.bfloat16).float().numpy())


def test_bf16_nan_stays_nan():
    x = np.array([np.nan, -np.nan], dtype=np.float32)
    assert np.isnan(R.bf16_to_f32(R.f32_to_bf16(x))).all()


# --------------------------------------------------------- page index math
def brute_positions(pages, length, page_size):
    out = []
    for t in range(length):
        out.append(pages[t // page_size] * page_size + t % page_size)
    return out


@pytest.mark.parametrize("page_size", [2, 4, 128])
def test_physical_positions_brute_force(page_size):
    r = rng(1)
    pages = r.permutation(50)[:7].tolist()
    for length in [0, 1, page_size - 1, page_size, page_size + 1, 7 * page_size]:
        assert R.physical_positions(pages, length, page_size).tolist() == brute_positions(
            pages, length, page_size
        )


def test_append_matches_torch_index_put_of_write_layer():
    """The reference's write_layer (paged_cache.py:49-60) expressed with the
    same torch indexing, on a uniform batch; the oracle must agree bitwise."""
    P, H, D, cap = 4, 2, 8, 64
    r = rng(2)
    page_lists = [[5, 2, 9], [0, 14, 3]]
    cache_lens = [5, 9]
    T = 2
    pool = r.integers(0, 65535, size=(1, 1, H, cap, D), dtype=np.uint16)
    k = r.integers(0, 65535, size=(2, H, T, D), dtype=np.uint16)
    # torch version of write_layer
    tp = torch.from_numpy(pool.astype(np.int32))
    table = torch.tensor(page_lists)
    cl = torch.tensor(cache_lens)
    logical = cl[:, None] + torch.arange(T)[None, :]
    phys = torch.gather(table, 1, logical // P) * P + logical % P
    tp[0, 0, :, phys, :] = torch.from_numpy(k.astype(np.int32)).permute(1, 0, 2, 3)
    # oracle, packed (N, H, D)
    pk = pool[0, 0].copy()
    pv = pool[0, 0].copy()
    packed = np.transpose(k, (0, 2, 1, 3)).reshape(2 * T, H, D)
    R.kv_append(pk, pv, packed, packed, page_lists, cache_lens, [T, T], P)
    assert np.array_equal(pk, tp[0, 0].numpy().astype(np.uint16))


def test_append_brute_force_loop():
    P, H, D, cap = 2, 1, 4, 16
    pool_k = np.zeros((H, cap, D), dtype=np.uint16)
    pool_v = np.zeros((H, cap, D), dtype=np.uint16)
    page_lists = [[3, 1], [6, 0, 2]]
    cache_lens, q_lens = [1, 3], [2, 2]
    new = np.arange(4 * H * D, dtype=np.uint16).reshape(4, H, D) + 1
    R.kv_append(pool_k, pool_v, new, new + 100, page_lists, cache_lens, q_lens, P)
    expect = np.zeros_like(pool_k)
    tok = 0
    for pages, c, q in zip(page_lists, cache_lens, q_lens):
        for i in range(q):
            t = c + i
            expect[:, pages[t // P] * P + t % P, :] = new[tok]
            tok += 1
    assert np.array_equal(pool_k, expect)
    assert np.array_equal(pool_v[pool_v != 0], (expect + 100)[expect != 0])


def test_gather_scatter_round_trip_mirrors_reference_test():
    """tests/test_paged_cache.py:25-38 of the reference: 2 layers, 1 head,
    head_dim 4, page 2, values arange(24) over 3 tokens -> 2 pages; the
    snapshot equals what was imported."""
    pool = np.zeros((2, 1, 8, 4), dtype=np.uint16)
    values = np.arange(24, dtype=np.uint16).reshape(2, 1, 3, 4)
    pages = [0, 1]  # LIFO free list of a fresh pool pops 0 then 1
    R.page_scatter(pool, pages, values, 2)
    assert np.array_equal(R.page_gather(pool, pages, 3, 2), values)
    # the same with scattered pages, against torch index_select (paged_cache.py:188)
    pool2 = np.zeros((2, 1, 16, 4), dtype=np.uint16)
    pages2 = [6, 2]
    R.page_scatter(pool2, pages2, values, 2)
    pos = torch.tensor(R.physical_positions(pages2, 3, 2))
    sel = torch.from_numpy(pool2.astype(np.int32)).index_select(2, pos).numpy()
    assert np.array_equal(sel.astype(np.uint16), values)


# ------------------------------------------------------------------- norm
def test_rms_norm_matches_torch_rms_norm_bitwise():
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(3000, 128, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    ref = F.rms_norm(x, (128,), w, 1e-6)
    ours = R.rms_norm(R.torch_bf16_to_bits(x), R.torch_bf16_to_bits(w), 1e-6)
    assert np.array_equal(ours, R.torch_bf16_to_bits(ref))


def test_rms_norm_closed_form_constant_row():
    # x = c everywhere: mean(x^2) = c^2, y = w * c / sqrt(c^2 + eps) ~ w * sign(c)
    for c in [0.5, -3.0, 100.0]:
        x = R.f32_to_bf16(np.full((1, 128), c, dtype=np.float32))
        w = R.f32_to_bf16(np.linspace(0.5, 1.5, 128, dtype=np.float32))
        y = R.bf16_to_f32(R.rms_norm(x, w, 1e-6))[0]
        expect = R.bf16_to_f32(w) * np.sign(c) * abs(c) / math.sqrt(c * c + 1e-6)
        np.testing.assert_allclose(y, expect, rtol=2**-7)


def test_rms_norm_mutation_is_caught():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(64, 128, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    ref = R.torch_bf16_to_bits(F.rms_norm(x, (128,), w, 1e-6))
    xb = R.torch_bf16_to_bits(x)
    wrong = R.f32_to_bf16(R.bf16_to_f32(R.rms_norm(xb, R.f32_to_bf16(np.ones(128, np.float32)), 1e-6))
                          * R.bf16_to_f32(R.torch_bf16_to_bits(w)) * 1.01)
    assert not np.array_equal(wrong, ref)


# ------------------------------------------------------------------- rope
def test_rope_tables_closed_form():
    cos, sin = R.rope_tables(128, 1_000_000, 4096)
    assert cos.dtype == np.float32 and cos.shape == (4096, 128)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    assert np.array_equal(cos[:, :64], cos[:, 64:])
    p = np.arange(4096, dtype=np.float64)[:, None]
    inv = 1_000_000.0 ** (-np.arange(0, 128, 2, dtype=np.float64) / 128)
    np.testing.assert_allclose(cos[:, :64], np.cos(p * inv), atol=2e-3)
    np.testing.assert_allclose(sin[:, :64], np.sin(p * inv), atol=2e-3)


def test_rope_is_identity_at_position_zero_and_matches_complex_rotation():
    cos, sin = R.rope_tables(128, 1_000_000, 4096)
    r = rng(5)
    x = R.f32_to_bf16(r.standard_normal((50, 3, 128)).astype(np.float32))
    pos0 = np.zeros(50, dtype=np.int64)
    assert np.array_equal(R.apply_rope(x, cos, sin, pos0), x)
    pos = r.integers(0, 4096, size=50)
    y = R.bf16_to_f32(R.apply_rope(x, cos, sin, pos)).astype(np.float64)
    xf = R.bf16_to_f32(x).astype(np.float64)
    z = (xf[..., :64] + 1j * xf[..., 64:]) * (cos[pos][:, None, :64] + 1j * sin[pos][:, None, :64])
    np.testing.assert_allclose(y[..., :64], z.real, atol=3e-2, rtol=2**-7)
    np.testing.assert_allclose(y[..., 64:], z.imag, atol=3e-2, rtol=2**-7)
    # a rotation keeps the norm
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(xf, axis=-1), rtol=1e-2)


def test_rope_matches_torch_ops_bitwise():
    cos, sin = R.rope_tables(128, 1_000_000, 2048)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 4, 7, 128, generator=g).to(torch.bfloat16)  # (B, H, T, D)
    pos = torch.randint(0, 2048, (2, 7), generator=g)
    ct, st = torch.from_numpy(cos), torch.from_numpy(sin)
    rotated = torch.cat((-x[..., 64:], x[..., :64]), dim=-1)
    ref = ((x * ct[pos].unsqueeze(1)) + (rotated * st[pos].unsqueeze(1))).to(torch.bfloat16)
    xb = R.torch_bf16_to_bits(x.transpose(1, 2))  # (B, T, H, D)
    ours = R.apply_rope(xb, cos, sin, pos.numpy())
    assert np.array_equal(ours, R.torch_bf16_to_bits(ref.transpose(1, 2)))


# -------------------------------------------------------------- attention
def sdpa_reference(q_bits, pool_k, pool_v, page_lists, cache_lens, q_lens, page_size, group):
    """torch SDPA over concatenated logical K/V with the boolean causal mask
    `key <= cache_len + i` and enable_gqa (test_paged_cache.py:95-112)."""
    outs = []
    start = 0
    q = torch.from_numpy(R.bf16_to_f32(q_bits)).double()
    for pages, c, ql in zip(page_lists, cache_lens, q_lens):
        kv = c + ql
        pos = R.physical_positions(pages, kv, page_size)
        k = torch.from_numpy(R.bf16_to_f32(pool_k[:, pos, :])).double()[None]
        v = torch.from_numpy(R.bf16_to_f32(pool_v[:, pos, :])).double()[None]
        qq = q[start : start + ql].transpose(0, 1)[None]  # (1, Hq, ql, D)
        allowed = torch.arange(kv)[None, :] <= (c + torch.arange(ql))[:, None]
        o = F.scaled_dot_product_attention(qq, k, v, attn_mask=allowed[None, None], enable_gqa=True)
        outs.append(o[0].transpose(0, 1).numpy())
        start += ql
    return np.concatenate(outs, axis=0)


def random_case(seed, hq, hkv, d, page, cache_lens, q_lens, n_pages):
    r = rng(seed)
    pool_k = R.f32_to_bf16(r.standard_normal((hkv, n_pages * page, d)).astype(np.float32))
    pool_v = R.f32_to_bf16(r.standard_normal((hkv, n_pages * page, d)).astype(np.float32))
    perm = r.permutation(n_pages).tolist()
    page_lists, cur = [], 0
    for c, q in zip(cache_lens, q_lens):
        n = math.ceil((c + q) / page)
        page_lists.append(perm[cur : cur + n])
        cur += n
    q = R.f32_to_bf16(r.standard_normal((sum(q_lens), hq, d)).astype(np.float32))
    return q, pool_k, pool_v, page_lists


@pytest.mark.parametrize(
    "hq,hkv,d,cache_lens,q_lens",
    [
        (4, 2, 16, [130, 200], [2, 2]),           # the reference test's shapes
        (32, 8, 128, [511], [1]),                 # decode, batch 1
        (32, 8, 128, [0, 300, 129], [40, 1, 17]),  # mixed, with an empty history
    ],
)
def test_attention_matches_sdpa(hq, hkv, d, cache_lens, q_lens):
    q, pk, pv, pl = random_case(7, hq, hkv, d, 128, cache_lens, q_lens, 16)
    ours = R.paged_attention(q, pk, pv, pl, cache_lens, q_lens, 128)
    ref = sdpa_reference(q, pk, pv, pl, cache_lens, q_lens, 128, hq // hkv)
    np.testing.assert_allclose(ours, ref, atol=1e-10, rtol=1e-9)


def test_attention_closed_forms():
    hq, hkv, d = 8, 2, 128
    q, pk, pv, pl = random_case(8, hq, hkv, d, 128, [0, 257], [1, 1], 8)
    # a first token sees only itself: output = its V row, for every head of a group
    out = R.paged_attention(q, pk, pv, pl, [0, 257], [1, 1], 128)
    v0 = R.bf16_to_f32(pv[:, pl[0][0] * 128, :])
    np.testing.assert_allclose(out[0], np.repeat(v0, hq // hkv, axis=0), rtol=1e-12)
    # q = 0: uniform weights, output = mean of the visible V rows
    qz = np.zeros_like(q)
    out = R.paged_attention(qz, pk, pv, pl, [0, 257], [1, 1], 128)
    pos = R.physical_positions(pl[1], 258, 128)
    mean_v = R.bf16_to_f32(pv[:, pos, :]).astype(np.float64).mean(axis=1)
    np.testing.assert_allclose(out[1], np.repeat(mean_v, hq // hkv, axis=0), rtol=1e-10)


def test_attention_page_placement_invariance_and_wrong_page_mutation():
    hq, hkv, d = 32, 8, 128
    cache_lens, q_lens = [900, 40], [1, 60]
    q, pk, pv, pl = random_case(9, hq, hkv, d, 128, cache_lens, q_lens, 20)
    base = R.paged_attention(q, pk, pv, pl, cache_lens, q_lens, 128)
    # move every page of request 0 to fresh physical pages: same result
    free = [p for p in range(20) if p not in pl[0] and p not in pl[1]]
    pk2, pv2 = pk.copy(), pv.copy()
    moved = free[: len(pl[0])]
    for old, new in zip(pl[0], moved):
        pk2[:, new * 128 : (new + 1) * 128] = pk[:, old * 128 : (old + 1) * 128]
        pv2[:, new * 128 : (new + 1) * 128] = pv[:, old * 128 : (old + 1) * 128]
    out2 = R.paged_attention(q, pk2, pv2, [moved, pl[1]], cache_lens, q_lens, 128)
    assert np.array_equal(out2, base)
    # pointing one page of request 0 at the wrong physical page must fail the
    # tolerances the GPU kernels are held to
    wrong = list(pl[0])
    wrong[3] = free[-1]
    bad = R.paged_attention(q, pk, pv, [wrong, pl[1]], cache_lens, q_lens, 128)
    stats = R.compare(R.f32_to_bf16(bad[:1].astype(np.float32)), base[:1])
    assert stats["rel_rms"] > R.REL_RMS_TOL


def test_attention_mutations_are_caught():
    hq, hkv, d = 32, 8, 128
    q, pk, pv, pl = random_case(10, hq, hkv, d, 128, [300], [5], 8)
    ref = sdpa_reference(q, pk, pv, pl, [300], [5], 128, 4)
    # wrong GQA mapping (h % Hkv instead of h // G) must be far off
    perm = np.array([(h % hkv) * 4 + h // hkv for h in range(hq)])
    out = R.paged_attention(q[:, perm, :], pk, pv, pl, [300], [5], 128)[:, np.argsort(perm), :]
    assert R.compare(R.f32_to_bf16(out.astype(np.float32)), ref)["rel_rms"] > R.REL_RMS_TOL
    # dropping the causal diagonal (one key fewer) must be visible
    out = R.paged_attention(q, pk, pv, pl, [299], [5], 128)
    assert R.compare(R.f32_to_bf16(out.astype(np.float32)), ref)["max_abs"] > 1e-3


# ------------------------------------------------- fused norm + rope + append
def _reference_chain(q, k, v, q_w, k_w, cos, sin, pool_k, pool_v, page_lists, cache_lens,
                     page_size, rope_first=False, positions_from_zero=False, q_eps=1e-6,
                     k_eps=1e-6):
    """The reference's op chain for one paged layer on a uniform (B, T)
    batch, written with the torch ops it uses:
    nn.RMSNorm on (B, T, H, D) (attention.py:34-35, 62-63), transpose to
    (B, H, T, D) (66-68), apply_rope_vectorized at position_ids =
    arange(T) + cache_lens (rope.py:31-47, qwen.py:97-109), then
    write_layer's indexing (paged_cache.py:49-60) for k and the un-normed v.
    Mutations (for the sensitivity checks): rope_first rotates before the
    norm; positions_from_zero drops cache_lens from the positions."""
    B, T, _, D = q.shape
    qn = torch.nn.RMSNorm(D, eps=q_eps, dtype=torch.bfloat16)
    kn = torch.nn.RMSNorm(D, eps=k_eps, dtype=torch.bfloat16)
    with torch.no_grad():
        qn.weight.copy_(q_w)
        kn.weight.copy_(k_w)
    cl = torch.tensor(cache_lens, dtype=torch.long)
    position_ids = torch.arange(T, dtype=torch.long).unsqueeze(0)
    if not positions_from_zero:
        position_ids = position_ids + cl.view(-1, 1)

    def rope(x):  # x (B, H, T, D)
        x1, x2 = x[..., : D // 2], x[..., D // 2 :]
        rotated = torch.cat((-x2, x1), dim=-1)
        out = (x * cos[position_ids].unsqueeze(1)) + (rotated * sin[position_ids].unsqueeze(1))
        return out.to(dtype=x.dtype)

    with torch.no_grad():
        if rope_first:
            q = rope(q.transpose(1, 2)).transpose(1, 2)
            k = rope(k.transpose(1, 2)).transpose(1, 2)
            q, k = qn(q), kn(k)
            q, k = q.transpose(1, 2), k.transpose(1, 2)
        else:
            q, k = qn(q), kn(k)
            q, k = rope(q.transpose(1, 2)), rope(k.transpose(1, 2))
        v = v.transpose(1, 2)
        # page table (B, num_pages), -1 padded (paged_cache.py:238-250)
        width = max(len(pl) for pl in page_lists)
        table = torch.full((B, width), -1, dtype=torch.long)
        for row, pl in enumerate(page_lists):
            table[row, : len(pl)] = torch.tensor(pl, dtype=torch.long)
        logical = cl[:, None] + torch.arange(T, dtype=torch.long).view(1, -1)
        phys = torch.gather(table, 1, logical // page_size) * page_size + logical % page_size
        pool_k[:, phys, :] = k.permute(1, 0, 2, 3)
        pool_v[:, phys, :] = v.permute(1, 0, 2, 3)
    return q  # (B, Hq, T, D)


def test_qknorm_rope_append_matches_reference_op_chain():
    """qknorm_rope_append (the oracle of the fused append kernels) against
    the reference's own op chain on a uniform batch with non-zero, unaligned
    cache lengths: rotated q, K pool and V pool bit for bit. Two plausible
    mistakes — rope before the norm, positions without cache_lens — change
    the result, so the check would catch them in the oracle."""
    B, T, Hq, Hkv, D, P = 3, 6, 4, 2, 128, 8
    cache_lens = [0, 77, 130]
    page_lists = [[11, 3], [20, 7, 14, 1, 9, 30, 25, 4, 12, 17, 2], [5, 8, 16, 0, 29, 31, 6, 10,
                                                                     13, 15, 18, 19, 21, 22,
                                                                     23, 24, 26, 27]]
    g = torch.Generator().manual_seed(41)
    q = (torch.randn(B, T, Hq, D, generator=g) * 2).to(torch.bfloat16)
    k = (torch.randn(B, T, Hkv, D, generator=g) * 2).to(torch.bfloat16)
    v = torch.randn(B, T, Hkv, D, generator=g).to(torch.bfloat16)
    q_w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    k_w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    cos_np, sin_np = R.rope_tables(D, 1_000_000, 4096)
    cos, sin = torch.from_numpy(cos_np), torch.from_numpy(sin_np)
    cap = 32 * P
    pool0_k = torch.randn(Hkv, cap, D, generator=g).to(torch.bfloat16)
    pool0_v = torch.randn(Hkv, cap, D, generator=g).to(torch.bfloat16)

    tk, tv = pool0_k.clone(), pool0_v.clone()
    q_ref = _reference_chain(q, k, v, q_w, k_w, cos, sin, tk, tv, page_lists, cache_lens, P)

    ok_k, ok_v = R.torch_bf16_to_bits(pool0_k).copy(), R.torch_bf16_to_bits(pool0_v).copy()
    q_ours = R.qknorm_rope_append(
        R.torch_bf16_to_bits(q.reshape(B * T, Hq, D)), R.torch_bf16_to_bits(k.reshape(B * T, Hkv, D)),
        R.torch_bf16_to_bits(v.reshape(B * T, Hkv, D)), R.torch_bf16_to_bits(q_w),
        R.torch_bf16_to_bits(k_w), 1e-6, cos_np, sin_np, ok_k, ok_v, page_lists, cache_lens,
        [T] * B, P)
    assert np.array_equal(q_ours, R.torch_bf16_to_bits(q_ref.transpose(1, 2).reshape(B * T, Hq, D)))
    assert np.array_equal(ok_k, R.torch_bf16_to_bits(tk)), "K pool"
    assert np.array_equal(ok_v, R.torch_bf16_to_bits(tv)), "V pool (v is appended un-normed)"

    for mutation in ({"rope_first": True}, {"positions_from_zero": True}):
        mk, mv = pool0_k.clone(), pool0_v.clone()
        q_mut = _reference_chain(q, k, v, q_w, k_w, cos, sin, mk, mv, page_lists, cache_lens, P,
                                 **mutation)
        assert not np.array_equal(
            q_ours, R.torch_bf16_to_bits(q_mut.transpose(1, 2).reshape(B * T, Hq, D))), mutation
        assert not np.array_equal(ok_k, R.torch_bf16_to_bits(mk)), mutation


def test_qknorm_rope_append_separate_q_and_k_eps():
    """The q and k norms are separate nn.RMSNorm modules, each with its own
    eps (attention.py:34-35): with k_eps != eps the oracle matches the
    reference chain built with those two modules, and differs from the
    chain that uses q's eps for k."""
    B, T, Hq, Hkv, D, P = 2, 3, 4, 2, 128, 8
    cache_lens = [5, 0]
    page_lists = [[3], [1]]
    g = torch.Generator().manual_seed(43)
    q = (torch.randn(B, T, Hq, D, generator=g) * 0.05).to(torch.bfloat16)
    k = (torch.randn(B, T, Hkv, D, generator=g) * 0.05).to(torch.bfloat16)
    v = torch.randn(B, T, Hkv, D, generator=g).to(torch.bfloat16)
    q_w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    k_w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    cos_np, sin_np = R.rope_tables(D, 1_000_000, 64)
    cos, sin = torch.from_numpy(cos_np), torch.from_numpy(sin_np)
    pool0 = torch.randn(Hkv, 4 * P, D, generator=g).to(torch.bfloat16)
    tk, tv = pool0.clone(), pool0.clone()
    q_ref = _reference_chain(q, k, v, q_w, k_w, cos, sin, tk, tv, page_lists, cache_lens, P,
                             q_eps=1e-6, k_eps=1e-2)
    ok_k, ok_v = R.torch_bf16_to_bits(pool0).copy(), R.torch_bf16_to_bits(pool0).copy()
    q_ours = R.qknorm_rope_append(
        R.torch_bf16_to_bits(q.reshape(B * T, Hq, D)), R.torch_bf16_to_bits(k.reshape(B * T, Hkv, D)),
        R.torch_bf16_to_bits(v.reshape(B * T, Hkv, D)), R.torch_bf16_to_bits(q_w),
        R.torch_bf16_to_bits(k_w), 1e-6, cos_np, sin_np, ok_k, ok_v, page_lists, cache_lens,
        [T] * B, P, k_eps=1e-2)
    assert np.array_equal(q_ours, R.torch_bf16_to_bits(q_ref.transpose(1, 2).reshape(B * T, Hq, D)))
    assert np.array_equal(ok_k, R.torch_bf16_to_bits(tk))
    mk, mv = pool0.clone(), pool0.clone()
    _reference_chain(q, k, v, q_w, k_w, cos, sin, mk, mv, page_lists, cache_lens, P,
                     q_eps=1e-6, k_eps=1e-6)
    assert not np.array_equal(ok_k, R.torch_bf16_to_bits(mk))
