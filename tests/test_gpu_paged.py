"""GPU parity of the HIP path against the oracle.

* KV append and page gather/scatter: bit-exact.
* Fused q/k RMSNorm + RoPE: bit-exact (rotated q and the appended K rows).
* Attention output (bf16): max-abs <= 2e-2, mean-abs <= 2e-3 and
  error-RMS / output-RMS <= 1e-2 against the float64 oracle.

Covers the five workloads at full size, the reference's own paged-attention
test scenario (tests/test_paged_cache.py:58-112: histories 130 and 200,
query length 2, imported through import_cache), the GroupedQueryAttention
module, split-count invariance, ragged lengths around slice and page
boundaries, copy-on-write of shared pages and a 256-token page size.
"""

import math

import numpy as np
import pytest
import torch

from gpu_util import EPS, assert_attention_close, bits, gpu_step, layer_bits, oracle_step, say
from oracle import paged_ref as R

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from hayate_amd import Cache, PagedKVBatch, PagedKVCacheManager
    from hayate_amd.attention import GroupedQueryAttention
    from hayate_amd.constants import MIN_KV_PAGE_SIZE
    from hayate_amd.rope import compute_rope_params
    from hayate_amd.workloads import ORDER, make_workload
else:  # collected on CPU only to be deselected
    ORDER = []

DEV = "cuda"


@pytest.mark.parametrize("name", ["decode_b1", "decode_b32", "prefill_4x512", "mixed_tick",
                                  "decode_32k"])
def test_workload_parity(name):
    say(f"[workload {name}]")
    w = make_workload(name, device=DEV)
    pre_k, pre_v = layer_bits(w.manager)
    q_rot, out = gpu_step(w)
    post_k, post_v = layer_bits(w.manager)
    pk, pv, q_exp, o_exp = oracle_step(w, pre_k, pre_v)
    assert np.array_equal(bits(q_rot), q_exp), "rotated q differs"
    assert np.array_equal(post_v, pv), "V pool differs (append must be a bit copy)"
    assert np.array_equal(post_k, pk), "K pool differs (norm + rope + append)"
    assert_attention_close(bits(out), o_exp, name)


def test_reference_paged_test_scenario():
    """test_paged_cache.py:58-112 at head_dim 128: histories 130 and 200
    imported through import_cache, query length 2, write_layer then
    attend_layer on the uniform (B, H, T, D) layout."""
    say("[reference scenario]")
    torch.manual_seed(23)
    hkv, hq, d = 2, 4, 128
    m = PagedKVCacheManager(num_layers=1, num_kv_heads=hkv, head_dim=d, max_cache_tokens=1024,
                            page_size=128, max_requests=2, dtype=torch.bfloat16, device=DEV)
    m.k_cache.normal_()
    m.v_cache.normal_()
    handles, hist_k, hist_v = [], [], []
    for length in (130, 200):
        k = torch.randn(1, hkv, length, d, device=DEV, dtype=torch.bfloat16)
        v = torch.randn_like(k)
        handles.append(m.allocate_for_request(Cache.from_tensors(k, v)))
        hist_k.append(k)
        hist_v.append(v)
    state = m.begin_batch(handles, 2)
    q = torch.randn(2, hq, 2, d, device=DEV, dtype=torch.bfloat16)
    new_k = torch.randn(2, hkv, 2, d, device=DEV, dtype=torch.bfloat16)
    new_v = torch.randn_like(new_k)
    state.write_layer(0, new_k, new_v)
    out = state.attend_layer(q, 0)
    torch.cuda.synchronize()
    m.commit_batch(handles, 2)
    # the pages hold history + new rows exactly (gather is a bit copy)
    for row, h in enumerate(handles):
        snap = m.snapshot(h)
        expect_k = torch.cat((hist_k[row], new_k[row : row + 1]), dim=2)
        expect_v = torch.cat((hist_v[row], new_v[row : row + 1]), dim=2)
        assert torch.equal(snap.k.view(torch.int16), expect_k.view(torch.int16))
        assert torch.equal(snap.v.view(torch.int16), expect_v.view(torch.int16))
    pk, pv = layer_bits(m)
    q_packed = bits(q.transpose(1, 2).reshape(4, hq, d))
    expect = R.paged_attention(q_packed, pk, pv, [h.pages for h in handles], [130, 200], [2, 2],
                               128)
    got = bits(out.transpose(1, 2).reshape(4, hq, d))
    assert_attention_close(got, expect, "reference scenario")
    # and the reference test's own check: SDPA on the logical K/V, rtol/atol 3e-2
    for row, old in enumerate((130, 200)):
        keys = torch.cat((hist_k[row][0], new_k[row]), dim=1).float()[None]
        vals = torch.cat((hist_v[row][0], new_v[row]), dim=1).float()[None]
        allowed = torch.arange(old + 2, device=DEV)[None, :] <= (old + torch.arange(2, device=DEV))[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(
            q[row : row + 1].float(), keys, vals, attn_mask=allowed[None, None], enable_gqa=True)
        torch.testing.assert_close(out[row : row + 1].float(), ref, rtol=3e-2, atol=3e-2)


def test_attention_module_paged_forward():
    """GroupedQueryAttention (attention.py:17-122 interface) in paged mode
    against projections + oracle + o_proj."""
    say("[module forward]")
    torch.manual_seed(5)
    d_in, hq, hkv, d, T = 256, 32, 8, 128, 3
    mod = GroupedQueryAttention(d_in, hq, hkv, d, dtype=torch.bfloat16).to(DEV)
    with torch.no_grad():
        mod.q_norm.weight.copy_(1 + 0.1 * torch.randn(d))
        mod.k_norm.weight.copy_(1 + 0.1 * torch.randn(d))
    cos, sin = compute_rope_params(d, 1_000_000, 40_960, device=DEV)
    m = PagedKVCacheManager(2, hkv, d, 4096, 128, 4, torch.bfloat16, DEV, num_q_heads=hq)
    m.k_cache.normal_()
    m.v_cache.normal_()
    handles = []
    for c in (0, 77, 300):
        h = m.allocate()
        m.reserve(h, c)
        h.length = c
        handles.append(h)
    pre_k, pre_v = layer_bits(m, 1)
    batch = m.begin_batch(handles, T)
    x = torch.randn(3, T, d_in, device=DEV, dtype=torch.bfloat16)
    with torch.inference_mode():
        y, nk, nv = mod(x, cos, sin, None, None, None, paged_cache=batch, layer_idx=1)
        qp, kp, vp = mod.project_qkv(x)
    torch.cuda.synchronize()
    assert nk is None and nv is None
    pk, pv = pre_k.copy(), pre_v.copy()
    pages = [list(h.pages) for h in handles]
    q_rot = R.qknorm_rope_append(bits(qp.reshape(3 * T, hq, d)), bits(kp.reshape(3 * T, hkv, d)),
                                 bits(vp.reshape(3 * T, hkv, d)), bits(mod.q_norm.weight),
                                 bits(mod.k_norm.weight), EPS, cos.cpu().numpy(),
                                 sin.cpu().numpy(), pk, pv, pages, [0, 77, 300], [T] * 3, 128)
    post_k, post_v = layer_bits(m, 1)
    assert np.array_equal(post_k, pk) and np.array_equal(post_v, pv)
    ctx = R.paged_attention(q_rot, pk, pv, pages, [0, 77, 300], [T] * 3, 128)
    ctx_t = torch.from_numpy(ctx.astype(np.float32)).to(DEV).to(torch.bfloat16).reshape(3, T, hq * d)
    with torch.inference_mode():
        y_ref = mod.o_proj(ctx_t)
    err = (y.float() - y_ref.float()).abs()
    say(f"  module max_abs={err.max().item():.3e}")
    assert err.max().item() < 5e-2 * max(1.0, y_ref.float().abs().max().item())


@pytest.mark.parametrize("split", [64, 512, 0])
def test_decode_split_count_does_not_change_results(split):
    say(f"[split {split}]")
    w = make_workload("decode_b32", device=DEV, tokens_per_split=split)
    pre_k, pre_v = layer_bits(w.manager)
    _, out = gpu_step(w)
    _, _, _, o_exp = oracle_step(w, pre_k, pre_v)
    assert_attention_close(bits(out), o_exp, f"split {split}")


def _ragged(cache_lens, q_lens, page_size=128, pool_tokens=32768, seed=0):
    say(f"[ragged page={page_size} c={cache_lens} q={q_lens}]")
    hq, hkv, d = 32, 8, 128
    g = torch.Generator().manual_seed(seed)
    m = PagedKVCacheManager(1, hkv, d, pool_tokens, page_size, len(q_lens), torch.bfloat16, DEV,
                            num_q_heads=hq)
    m.k_cache.normal_()
    m.v_cache.normal_()
    perm = torch.randperm(m.num_pages, generator=g).tolist()
    handles, cur = [], 0
    for c, q in zip(cache_lens, q_lens):
        h = m.allocate()
        n = math.ceil((c + q) / page_size)
        m.claim_pages(h, perm[cur : cur + n])
        cur += n
        h.length = c
        handles.append(h)
    n_tok = sum(q_lens)
    q = torch.randn(n_tok, hq, d, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(n_tok, hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(n_tok, hkv, d, generator=g).to(torch.bfloat16).to(DEV)
    pre_k, pre_v = layer_bits(m)
    if page_size >= MIN_KV_PAGE_SIZE:
        batch = m.begin_tick(handles, q_lens)
    else:
        # begin_tick keeps the reference's smallest page (128 tokens); the
        # C ABI takes any power of two >= 32, so the batch is built directly
        # over the pages the handles already hold
        batch = PagedKVBatch(m, list(q_lens), list(cache_lens), [list(h.pages) for h in handles],
                             varlen=True, num_q_heads=hq, tokens_per_split=m.tokens_per_split)
    batch.write_layer(0, k, v)
    out = batch.attend_layer(q, 0)
    torch.cuda.synchronize()
    pk, pv = pre_k.copy(), pre_v.copy()
    pages = [list(h.pages) for h in handles]
    R.kv_append(pk, pv, bits(k), bits(v), pages, cache_lens, q_lens, page_size)
    post_k, post_v = layer_bits(m)
    assert np.array_equal(post_k, pk) and np.array_equal(post_v, pv)
    expect = R.paged_attention(bits(q), pk, pv, pages, cache_lens, q_lens, page_size)
    assert_attention_close(bits(out), expect, "ragged")


def test_decode_lengths_around_slice_and_page_edges():
    ctx = [1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 4095, 4096, 4097]
    _ragged([c - 1 for c in ctx], [1] * len(ctx))


def test_prefill_unaligned_offsets_and_short_chunks():
    _ragged([0, 95, 1000, 128, 3], [2, 33, 100, 512, 61])


def test_mixed_tick_small():
    _ragged([0, 700, 5, 1023, 64], [300, 1, 1, 40, 1])


def test_prefill_deep_prefix_splits():
    """One chunk over a 20,000-token prefix plus a shallow chunk: the deep
    one's key range is split across workgroups (merged by the merge
    launch), the shallow one runs whole."""
    from hayate_amd import _native

    p = _native.plan_tick(np.array([300, 40]), np.array([20_300, 100]), 32, 8, 128, 256, 0)
    assert len(p.prefill_merge) > 0
    assert all(int(r[5]) == -1 for r in p.prefill if int(r[0]) == 1)
    _ragged([20_000, 60], [300, 40], pool_tokens=22_000)


def test_page_size_256():
    _ragged([300, 0, 1000], [1, 70, 1], page_size=256)


@pytest.mark.parametrize("page_size", [32, 64])
def test_small_pages_through_the_c_abi(page_size):
    """Pages of 32 and 64 tokens (the kernels' smallest: a 32-token slice or
    key block must lie in one page): decode contexts around slice and page
    edges, unaligned prefill chunks, and a chunk over a prefix deep enough
    for the planner to split its key range."""
    ctx = [1, 31, 32, 33, 63, 64, 65, 129, 1000]
    _ragged([c - 1 for c in ctx] + [0, 95, 6000], [1] * len(ctx) + [61, 130, 300],
            page_size=page_size, pool_tokens=16384)


def test_more_than_a_thousand_sequences():
    """1,100 sequences: a ten-step sequence search per token in the append
    kernels, decode chunks that hold many pieces. Plain and fused decode,
    then a mixed tick with prefill chunks."""
    n = 1100
    cache_lens = [(7 * i) % 300 for i in range(n)]
    _ragged(cache_lens, [1] * n, pool_tokens=(n + 4) * 384)
    lengths = (cache_lens, [1] * n)
    w_a = make_workload("decode_b32", device=DEV, lengths=lengths)
    w_b = make_workload("decode_b32", device=DEV, lengths=lengths)
    pre_k, pre_v = layer_bits(w_a.manager)
    q_f, out_f = _fused_vs_two_calls(w_a, w_b)
    _, _, q_exp, o_exp = oracle_step(w_a, pre_k, pre_v)
    assert np.array_equal(bits(q_f), q_exp)
    assert_attention_close(bits(out_f), o_exp, "fused 1100")
    q_lens = [1] * n
    for i in (3, 500, 1099):
        q_lens[i] = 70
    _ragged(cache_lens, q_lens, pool_tokens=(n + 4) * 384)


def test_copy_on_write_keeps_shared_pages_intact():
    say("[copy on write]")
    hq, hkv, d = 32, 8, 128
    m = PagedKVCacheManager(1, hkv, d, 4096, 128, 3, torch.bfloat16, DEV, num_q_heads=hq)
    m.k_cache.normal_()
    m.v_cache.normal_()
    parent = m.allocate()
    m.reserve(parent, 256)
    parent.length = 256
    child = m.fork(parent, 256)
    m.truncate(child, 200)  # next append lands in the shared second page
    shared_page = parent.pages[1]
    before = bits(m.k_cache[0, 0, :, shared_page * 128 : (shared_page + 1) * 128]).copy()
    batch = m.begin_batch([child], 1)
    assert child.pages[1] != shared_page and m.page_refcount(shared_page) == 1
    k = torch.randn(1, hkv, 1, d, device=DEV, dtype=torch.bfloat16)
    batch.write_layer(0, k, k)
    torch.cuda.synchronize()
    after = bits(m.k_cache[0, 0, :, shared_page * 128 : (shared_page + 1) * 128])
    assert np.array_equal(before, after)
    new_page = child.pages[1]
    copy = bits(m.k_cache[0, 0, :, new_page * 128 : (new_page + 1) * 128])
    assert np.array_equal(copy[:, :72], before[:, :72])
    assert np.array_equal(copy[:, 72], bits(k[0, :, 0]))


def test_gather_scatter_round_trip_bit_exact():
    say("[gather/scatter]")
    m = PagedKVCacheManager(3, 8, 128, 8192, 128, 2, torch.bfloat16, DEV)
    m.k_cache.normal_()
    m.v_cache.normal_()
    src_k = torch.randn(3, 8, 700, 128, device=DEV, dtype=torch.bfloat16)
    src_v = torch.randn_like(src_k)
    h = m.allocate_for_request(Cache.from_tensors(src_k, src_v))
    snap = m.snapshot(h, 650)
    torch.cuda.synchronize()
    assert torch.equal(snap.k.view(torch.int16), src_k[:, :, :650].view(torch.int16))
    assert torch.equal(snap.v.view(torch.int16), src_v[:, :, :650].view(torch.int16))
    # against the oracle's gather over the same pool
    pool = bits(m.k_cache[:, 0])
    assert np.array_equal(bits(snap.k), R.page_gather(pool, h.pages, 650, 128))


def test_graph_replay_matches_eager():
    """One mixed tick (append + decode + prefill + merges) captured in a HIP
    graph: every replay, with eager work and synchronisations between
    replays, reproduces the eager step bit for bit."""
    say("[graph replay mixed_tick]")
    w = make_workload("mixed_tick", device=DEV, num_layers=1)
    batch = w.begin()
    batch.plan(w.q.shape[1])

    def step():
        q_rot = batch.norm_rope_write_layer(0, w.q, w.k, w.v, w.q_norm_w, w.k_norm_w, EPS,
                                            w.cos, w.sin)
        return q_rot, batch.attend_layer(q_rot, 0)

    q_eager, out_eager = step()
    torch.cuda.synchronize()
    q_eager, out_eager = bits(q_eager), bits(out_eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        q_g, out_g = step()
    scratch = torch.randn(1 << 20, device=DEV)
    for rep in range(3):
        q_g.zero_()
        out_g.zero_()
        scratch.mul_(1.5).sum().item()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(q_g), q_eager), f"replay {rep}: rotated q differs"
        assert np.array_equal(bits(out_g), out_eager), f"replay {rep}: attention differs"


def _fused_vs_two_calls(w_a, w_b, layer=0):
    """decode_layer on w_a's pool, norm_rope_write_layer + attend_layer on
    w_b's identical pool: rotated q, pool and attention output must match
    bit for bit."""
    ba = w_a.begin()
    q_f, out_f = ba.decode_layer(layer, w_a.q, w_a.k, w_a.v, w_a.q_norm_w, w_a.k_norm_w, EPS,
                                 w_a.cos, w_a.sin)
    bb = w_b.begin()
    q_s = bb.norm_rope_write_layer(layer, w_b.q, w_b.k, w_b.v, w_b.q_norm_w, w_b.k_norm_w, EPS,
                                   w_b.cos, w_b.sin)
    out_s = bb.attend_layer(q_s, layer)
    torch.cuda.synchronize()
    assert np.array_equal(bits(q_f), bits(q_s)), "rotated q differs"
    ka, va = layer_bits(w_a.manager, layer)
    kb, vb = layer_bits(w_b.manager, layer)
    assert np.array_equal(ka, kb), "K pool differs"
    assert np.array_equal(va, vb), "V pool differs"
    assert np.array_equal(bits(out_f), bits(out_s)), "attention differs"
    return q_f, out_f


@pytest.mark.parametrize("name", ["decode_b1", "decode_b32", "decode_32k"])
def test_fused_decode_append_matches_two_calls_and_oracle(name):
    say(f"[fused decode {name}]")
    w_a = make_workload(name, device=DEV)
    pre_k, pre_v = layer_bits(w_a.manager)
    w_b = make_workload(name, device=DEV)
    q_f, out_f = _fused_vs_two_calls(w_a, w_b)
    post_k, post_v = layer_bits(w_a.manager)
    pk, pv, q_exp, o_exp = oracle_step(w_a, pre_k, pre_v)
    assert np.array_equal(bits(q_f), q_exp)
    assert np.array_equal(post_k, pk) and np.array_equal(post_v, pv)
    assert_attention_close(bits(out_f), o_exp, f"fused {name}")


def test_fused_decode_append_ragged_and_many_short_sequences():
    """Contexts around slice and page edges, and 100 one-to-three-token
    contexts (chunks of many pieces, several new rows per chunk)."""
    for cache_lens in ([0, 30, 31, 32, 127, 128, 129, 255, 256, 1000, 4095],
                       [i % 3 for i in range(100)]):
        say(f"[fused ragged {cache_lens[:6]}...]")
        lengths = (cache_lens, [1] * len(cache_lens))
        w_a = make_workload("decode_b32", device=DEV, lengths=lengths)
        w_b = make_workload("decode_b32", device=DEV, lengths=lengths)
        pre_k, pre_v = layer_bits(w_a.manager)
        q_f, out_f = _fused_vs_two_calls(w_a, w_b)
        _, _, q_exp, o_exp = oracle_step(w_a, pre_k, pre_v)
        assert np.array_equal(bits(q_f), q_exp)
        assert_attention_close(bits(out_f), o_exp, "fused ragged")


def test_fused_decode_append_wide_dynamic_range_rows():
    """q and k rows whose magnitudes spread log-uniformly over 1e-6 .. 1e2
    (squares over 2^53 apart, so the fp64 sums of squares round): the two
    append layouts still accumulate in one order, so the fused decode and
    the two-call path agree bit for bit; different q and k epsilons reach
    their own norms."""
    say("[fused decode, wide-range rows, q eps != k eps]")
    g = torch.Generator().manual_seed(77)

    def wide(shape):
        mag = torch.pow(10.0, torch.empty(shape).uniform_(-6, 2, generator=g))
        sign = torch.where(torch.rand(shape, generator=g) < 0.5, -1.0, 1.0)
        return (mag * sign).to(torch.bfloat16).to(DEV)

    w_a = make_workload("decode_b32", device=DEV)
    w_b = make_workload("decode_b32", device=DEV)
    q, k = wide(tuple(w_a.q.shape)), wide(tuple(w_a.k.shape))
    for w in (w_a, w_b):
        w.q, w.k = q, k
    pre_k, pre_v = layer_bits(w_a.manager)
    ba = w_a.begin()
    q_f, out_f = ba.decode_layer(0, w_a.q, w_a.k, w_a.v, w_a.q_norm_w, w_a.k_norm_w, 1e-6,
                                 w_a.cos, w_a.sin, k_eps=1e-3)
    bb = w_b.begin()
    q_s = bb.norm_rope_write_layer(0, w_b.q, w_b.k, w_b.v, w_b.q_norm_w, w_b.k_norm_w, 1e-6,
                                   w_b.cos, w_b.sin, k_eps=1e-3)
    out_s = bb.attend_layer(q_s, 0)
    torch.cuda.synchronize()
    assert np.array_equal(bits(q_f), bits(q_s)), "rotated q differs"
    ka, va = layer_bits(w_a.manager)
    kb, vb = layer_bits(w_b.manager)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb), "pools differ"
    assert np.array_equal(bits(out_f), bits(out_s)), "attention differs"
    # the k rows were normed with k_eps: the oracle with eps 1e-3 on k only
    pk, pv = pre_k.copy(), pre_v.copy()
    cos, sin = w_a.cos.cpu().numpy(), w_a.sin.cpu().numpy()
    R.qknorm_rope_append(bits(q), bits(k), bits(w_a.v), bits(w_a.q_norm_w), bits(w_a.k_norm_w),
                         1e-6, cos, sin, pk, pv, w_a.page_lists, w_a.cache_lens, w_a.q_lens,
                         w_a.manager.page_size, k_eps=1e-3)
    diff = np.count_nonzero(ka != pk)
    say(f"  K rows vs oracle with k_eps: {diff} differing bf16 values")
    assert diff == 0


def test_fused_decode_graph_replay_matches_eager():
    say("[graph replay decode_layer]")
    w = make_workload("decode_b32", device=DEV, num_layers=1)
    batch = w.begin()
    batch.plan(w.q.shape[1])

    def step():
        return batch.decode_layer(0, w.q, w.k, w.v, w.q_norm_w, w.k_norm_w, EPS, w.cos, w.sin)

    q_e, out_e = step()
    torch.cuda.synchronize()
    q_e, out_e = bits(q_e), bits(out_e)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        q_g, out_g = step()
    for rep in range(3):
        q_g.zero_()
        out_g.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(q_g), q_e), f"replay {rep}: rotated q differs"
        assert np.array_equal(bits(out_g), out_e), f"replay {rep}: attention differs"


def _custom_workload(hq, hkv, cache_lens, q_lens, page_size=128, seed=5):
    """A Workload of any head geometry (not the Qwen3-4B one): random pool,
    pages placed by a seeded permutation, raw q/k/v, norm weights, rope."""
    from hayate_amd.workloads import SPECS, Workload

    d = 128
    g = torch.Generator().manual_seed(seed)
    need = [math.ceil((c + q) / page_size) for c, q in zip(cache_lens, q_lens)]
    n_pages = sum(need) + 4
    m = PagedKVCacheManager(1, hkv, d, n_pages * page_size, page_size, len(q_lens),
                            torch.bfloat16, DEV, num_q_heads=hq)
    m.k_cache.copy_(torch.randn(m.k_cache.shape, generator=g).to(torch.bfloat16))
    m.v_cache.copy_(torch.randn(m.v_cache.shape, generator=g).to(torch.bfloat16))
    perm = torch.randperm(m.num_pages, generator=g).tolist()
    handles, cur = [], 0
    for c, n in zip(cache_lens, need):
        h = m.allocate()
        m.claim_pages(h, perm[cur : cur + n])
        cur += n
        h.length = c
        handles.append(h)
    n_tok = sum(q_lens)
    cos, sin = compute_rope_params(d, 1e6, max(c + q for c, q in zip(cache_lens, q_lens)) + 1,
                                   device=DEV)
    return Workload(
        spec=SPECS["decode_b1"], manager=m, handles=handles, q_lens=list(q_lens),
        cache_lens=list(cache_lens), page_lists=[list(h.pages) for h in handles],
        q=torch.randn(n_tok, hq, d, generator=g).to(torch.bfloat16).to(DEV),
        k=torch.randn(n_tok, hkv, d, generator=g).to(torch.bfloat16).to(DEV),
        v=torch.randn(n_tok, hkv, d, generator=g).to(torch.bfloat16).to(DEV),
        q_norm_w=(1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(DEV),
        k_norm_w=(1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(DEV),
        cos=cos, sin=sin,
    )


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (64, 8), (64, 4)])
def test_other_gqa_groups_mixed_and_fused_decode(hq, hkv):
    """GQA groups 1, 2, 8 and 16: a mixed tick (two prefill chunks, three
    decode tokens) through the append + attention calls, and a decode tick
    through the fused call, against the oracle."""
    say(f"[gqa hq={hq} hkv={hkv}]")
    cache_lens, q_lens = [0, 300, 5, 700, 2000], [200, 130, 1, 1, 1]
    w = _custom_workload(hq, hkv, cache_lens, q_lens)
    pre_k, pre_v = layer_bits(w.manager)
    q_rot, out = gpu_step(w)
    post_k, post_v = layer_bits(w.manager)
    pk, pv, q_exp, o_exp = oracle_step(w, pre_k, pre_v)
    assert np.array_equal(bits(q_rot), q_exp)
    assert np.array_equal(post_k, pk) and np.array_equal(post_v, pv)
    assert_attention_close(bits(out), o_exp, f"mixed G={hq // hkv}")

    cache_lens = [0, 31, 32, 129, 1000, 2047, 3, 64]
    w_a = _custom_workload(hq, hkv, cache_lens, [1] * len(cache_lens), seed=6)
    w_b = _custom_workload(hq, hkv, cache_lens, [1] * len(cache_lens), seed=6)
    pre_k, pre_v = layer_bits(w_a.manager)
    q_f, out_f = _fused_vs_two_calls(w_a, w_b)
    _, _, q_exp, o_exp = oracle_step(w_a, pre_k, pre_v)
    assert np.array_equal(bits(q_f), q_exp)
    assert_attention_close(bits(out_f), o_exp, f"fused G={hq // hkv}")


def test_append_partial_head_groups():
    """12 q heads and 6 kv heads over 4,092 tokens (256 blocks of 16, enough
    for the append launch to take groups of 8 heads per block): the last q
    group holds 4 heads and the k and v groups 6; rotated q and both pools
    bit-exact against the oracle."""
    say("[append hq=12 hkv=6, 4,092 tokens]")
    cache_lens, q_lens = [0, 100, 4000, 33, 77, 5000], [2000, 1500, 500, 90, 1, 1]
    w = _custom_workload(12, 6, cache_lens, q_lens, seed=11)
    pre_k, pre_v = layer_bits(w.manager)
    batch = w.begin()
    q_rot = batch.norm_rope_write_layer(0, w.q, w.k, w.v, w.q_norm_w, w.k_norm_w, EPS,
                                        w.cos, w.sin)
    torch.cuda.synchronize()
    post_k, post_v = layer_bits(w.manager)
    pk, pv = pre_k.copy(), pre_v.copy()
    q_exp = R.qknorm_rope_append(bits(w.q), bits(w.k), bits(w.v), bits(w.q_norm_w),
                                 bits(w.k_norm_w), EPS, w.cos.cpu().numpy(),
                                 w.sin.cpu().numpy(), pk, pv, w.page_lists, w.cache_lens,
                                 w.q_lens, w.manager.page_size)
    assert np.array_equal(bits(q_rot), q_exp), "rotated q differs"
    assert np.array_equal(post_k, pk), "K pool differs"
    assert np.array_equal(post_v, pv), "V pool differs"


@pytest.mark.parametrize("seed", range(6))
def test_random_mixed_ticks(seed):
    """Seeded random ticks (Qwen3-4B heads): 3-12 sequences, each a decode
    token or a prefill chunk of 2-300 tokens over 0-2,500 cached tokens, so
    the planner's decode cuts and prefill key splits land at arbitrary
    positions; pools and rotated q bit-exact, attention within tolerance."""
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.integers(3, 13))
    q_lens = [1 if rng.random() < 0.5 else int(rng.integers(2, 301)) for _ in range(n)]
    cache_lens = [int(rng.integers(0, 2501)) for _ in range(n)]
    say(f"[random tick seed={seed} q={q_lens} cache={cache_lens}]")
    w = _custom_workload(32, 8, cache_lens, q_lens, seed=seed)
    pre_k, pre_v = layer_bits(w.manager)
    q_rot, out = gpu_step(w)
    post_k, post_v = layer_bits(w.manager)
    pk, pv, q_exp, o_exp = oracle_step(w, pre_k, pre_v)
    assert np.array_equal(bits(q_rot), q_exp), "rotated q differs"
    assert np.array_equal(post_k, pk) and np.array_equal(post_v, pv), "pools differ"
    assert_attention_close(bits(out), o_exp, f"random tick {seed}")


@pytest.mark.parametrize("seed", range(4))
def test_random_ticks_deep_prefixes_pages_and_groups(seed):
    """Seeded random ticks over deeper prefixes (0-8,000 cached tokens, so
    the planner cuts long prefill tiles into full parts plus a short
    remainder), pages of 128 or 256 tokens (begin_tick keeps the reference's
    128-token minimum; smaller pages go through the C ABI in
    test_small_pages_through_the_c_abi) and GQA groups 1-16; pools and
    rotated q bit-exact, attention within tolerance."""
    rng = np.random.default_rng(2000 + seed)
    hq, hkv = [(32, 8), (64, 8), (16, 8), (8, 8), (64, 4)][int(rng.integers(0, 5))]
    page_size = [128, 256][int(rng.integers(0, 2))]
    n = int(rng.integers(2, 7))
    q_lens = [1 if rng.random() < 0.4 else int(rng.integers(2, 513)) for _ in range(n)]
    cache_lens = [int(rng.integers(0, 8001)) for _ in range(n)]
    say(f"[random deep tick seed={seed} hq={hq} hkv={hkv} page={page_size} q={q_lens} "
        f"cache={cache_lens}]")
    w = _custom_workload(hq, hkv, cache_lens, q_lens, page_size=page_size, seed=seed)
    pre_k, pre_v = layer_bits(w.manager)
    q_rot, out = gpu_step(w)
    post_k, post_v = layer_bits(w.manager)
    pk, pv, q_exp, o_exp = oracle_step(w, pre_k, pre_v)
    assert np.array_equal(bits(q_rot), q_exp), "rotated q differs"
    assert np.array_equal(post_k, pk) and np.array_equal(post_v, pv), "pools differ"
    assert_attention_close(bits(out), o_exp, f"random deep tick {seed}")


def test_maximum_context_last_rope_row():
    """Qwen3's longest context: rope tables of 40,960 rows (the reference
    model's max_position_embeddings) and tokens at positions up to 40,959,
    the tables' last row. A mixed tick (a decode token at position 40,959, a
    64-token chunk ending there, a short decode) through the append +
    attention calls, and a decode tick through the fused call against the
    two calls; pools and rotated q bit-exact, attention within tolerance."""
    say("[maximum context 40,960]")
    cache_lens, q_lens = [40_959, 40_896, 10], [1, 64, 1]
    w = _custom_workload(32, 8, cache_lens, q_lens, seed=21)
    w.cos, w.sin = compute_rope_params(128, 1_000_000, 40_960, device=DEV)
    pre_k, pre_v = layer_bits(w.manager)
    q_rot, out = gpu_step(w)
    post_k, post_v = layer_bits(w.manager)
    pk, pv, q_exp, o_exp = oracle_step(w, pre_k, pre_v)
    assert np.array_equal(bits(q_rot), q_exp), "rotated q differs"
    assert np.array_equal(post_k, pk) and np.array_equal(post_v, pv), "pools differ"
    assert_attention_close(bits(out), o_exp, "maximum context, mixed tick")

    cache_lens = [40_959, 10, 20_000]
    w_a = _custom_workload(32, 8, cache_lens, [1] * 3, seed=22)
    w_b = _custom_workload(32, 8, cache_lens, [1] * 3, seed=22)
    for wk in (w_a, w_b):
        wk.cos, wk.sin = compute_rope_params(128, 1_000_000, 40_960, device=DEV)
    pre_k, pre_v = layer_bits(w_a.manager)
    q_f, out_f = _fused_vs_two_calls(w_a, w_b)
    _, _, q_exp, o_exp = oracle_step(w_a, pre_k, pre_v)
    assert np.array_equal(bits(q_f), q_exp), "fused: rotated q differs"
    assert_attention_close(bits(out_f), o_exp, "maximum context, fused decode")


def test_few_key_rows_exact_base():
    """Rows that see 1-4 keys (the first tokens of a chunk at offset 0) put
    most weight on one key, so an error in that key's probability shows in
    the output. The prefill kernel subtracts the exact fp32 row max, so the
    largest probability is exactly 1 in bf16 as in the fp32 row sum. On
    these seeded inputs the rows' max-abs error is 0.0082 (a base rounded
    to bf16 gave 0.0156); the bound sits between the two."""
    say("[few-key rows, chunk at offset 0]")
    g = torch.Generator().manual_seed(21)
    m = PagedKVCacheManager(1, 8, 128, 8192, 128, 2, torch.bfloat16, DEV, num_q_heads=32)
    m.k_cache.copy_(torch.randn(m.k_cache.shape, generator=g).to(torch.bfloat16))
    m.v_cache.copy_(torch.randn(m.v_cache.shape, generator=g).to(torch.bfloat16))
    handles = []
    for c in (0, 130):
        h = m.allocate()
        m.reserve(h, c)
        h.length = c
        handles.append(h)
    q_lens = [64, 40]
    q = torch.randn(sum(q_lens), 32, 128, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(sum(q_lens), 8, 128, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(sum(q_lens), 8, 128, generator=g).to(torch.bfloat16).to(DEV)
    pre_k = R.torch_bf16_to_bits(m.k_cache[0, 0])
    pre_v = R.torch_bf16_to_bits(m.v_cache[0, 0])
    batch = m.begin_tick(handles, q_lens)
    batch.write_layer(0, k, v)
    out = batch.attend_layer(q, 0)
    torch.cuda.synchronize()
    pages = [list(h.pages) for h in handles]
    R.kv_append(pre_k, pre_v, bits(k), bits(v), pages, [0, 130], q_lens, 128)
    exp = R.paged_attention(bits(q), pre_k, pre_v, pages, [0, 130], q_lens, 128)
    got = R.bf16_to_f32(bits(out)).astype(np.float64).reshape(exp.shape)
    rows = slice(0, 4)  # tokens 0-3 of the first sequence: 1-4 keys
    e = exp[rows]
    err = np.abs(got[rows] - e)
    say(f"  max_abs {err.max():.4f}")
    assert err.max() <= 0.011, err.max()


def test_static_tick_batch_replays_one_shape_at_other_lengths():
    """A mixed tick shape (two prompt chunks, three decode tokens) captured
    once over a StaticTickBatch (tick_graph.py: fixed metadata buffers,
    decode chunk and prefill item lists padded with empty records) and
    replayed at two sets of cached lengths whose plans differ (other
    prefill item, split and decode chunk counts): each replay, after an
    in-place refresh, equals an eager begin_tick batch at the same lengths
    bit for bit (rotated q, pools, attention), and the second matches the
    oracle."""
    from hayate_amd.tick_graph import StaticTickBatch

    say("[static tick batch: one capture, two plans]")
    q_lens = [256, 320, 1, 1, 1]
    lens_a = [0, 1024, 100, 300, 37]
    lens_b = [256, 3500, 1500, 2001, 38]
    w = _custom_workload(32, 8, lens_b, q_lens, seed=11)
    m, hs = w.manager, w.handles
    pre = (m.k_cache.clone(), m.v_cache.clone())

    def set_lengths(lens):
        for h, c in zip(hs, lens):
            h.length = c
        m.k_cache.copy_(pre[0])
        m.v_cache.copy_(pre[1])

    def step(batch):
        q_rot = batch.norm_rope_write_layer(0, w.q, w.k, w.v, w.q_norm_w, w.k_norm_w, EPS,
                                            w.cos, w.sin)
        return q_rot, batch.attend_layer(q_rot, 0)

    plans = []
    expected = []
    for lens in (lens_a, lens_b):
        set_lengths(lens)
        eager = PagedKVBatch(m, q_lens, list(lens), [list(h.pages) for h in hs], varlen=True,
                             num_q_heads=32)
        plans.append(eager.plan(32).host)
        q_e, o_e = step(eager)
        torch.cuda.synchronize()
        expected.append((bits(q_e), bits(o_e), layer_bits(m)))
    say(f"  prefill items {[len(p.prefill) for p in plans]}, "
        f"slots {[p.n_prefill_slots for p in plans]}, chunks {[p.n_chunks for p in plans]}")
    assert len(plans[0].prefill) != len(plans[1].prefill)
    assert plans[0].n_chunks != plans[1].n_chunks

    slots = max(p.n_prefill_slots for p in plans) + 4
    static = StaticTickBatch(m, q_lens, 32, max_tokens=max(c + q for c, q in zip(lens_b, q_lens)),
                             prefill_slots=slots)
    set_lengths(lens_a)
    assert static.refresh(hs)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(static)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        q_g, o_g = step(static)
    for rep, (lens, (q_e, o_e, pools_e)) in enumerate(zip((lens_a, lens_b, lens_a),
                                                         expected + expected[:1])):
        set_lengths(lens)
        assert static.refresh(hs)
        q_g.zero_()
        o_g.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(q_g), q_e), f"replay {rep}: rotated q differs"
        assert np.array_equal(bits(o_g), o_e), f"replay {rep}: attention differs"
        k_b, v_b = layer_bits(m)
        assert np.array_equal(k_b, pools_e[0]) and np.array_equal(v_b, pools_e[1]), \
            f"replay {rep}: pools differ"
    # the second length set against the oracle
    set_lengths(lens_b)
    pre_k, pre_v = layer_bits(m)
    w.cache_lens = list(lens_b)
    pk, pv, q_exp, o_exp = oracle_step(w, pre_k, pre_v)
    q_e, o_e, pools_e = expected[1]
    assert np.array_equal(q_e, q_exp) and np.array_equal(pools_e[0], pk)
    assert_attention_close(o_e, o_exp, "static tick, second lengths")


def test_large_logits_scaled_in_fp32():
    """Scores 16 times the unit-norm case (both q/k norm weights x 4, so a
    row's scaled scores spread over tens of exp2 units and the softmax is
    peaky), on a tick with two prompt chunks and three decode tokens. The
    kernels scale scores in fp32 as the reference does; a query pre-scaled
    and rounded to bf16 before the product (what the prefill kernel once
    did) measured max-abs 0.14 and relative RMS 5.7e-3 here. Tolerance for
    this case: relative RMS 5e-3, max-abs 4e-2 (outputs reach ~4 in
    magnitude, where one bf16 step is 1.6e-2)."""
    say("[large logits]")
    for seed in (1, 2):
        w = _custom_workload(32, 8, [0, 700, 1500, 300, 2000], [256, 200, 1, 1, 1], seed=seed)
        w.q_norm_w = (w.q_norm_w.float() * 4).to(torch.bfloat16)
        w.k_norm_w = (w.k_norm_w.float() * 4).to(torch.bfloat16)
        pre_k, pre_v = layer_bits(w.manager)
        q_rot, out = gpu_step(w)
        post_k, post_v = layer_bits(w.manager)
        pk, pv, q_exp, o_exp = oracle_step(w, pre_k, pre_v)
        assert np.array_equal(bits(q_rot), q_exp) and np.array_equal(post_k, pk)
        st = R.compare(bits(out), o_exp)
        say(f"  seed {seed}: max_abs={st['max_abs']:.3e} rel_rms={st['rel_rms']:.3e}")
        assert st["finite"] and st["rel_rms"] <= 5e-3 and st["max_abs"] <= 4e-2, st


def test_static_tick_batch_refuses_a_plan_past_its_slots():
    """A StaticTickBatch sized for fewer prefill partial slots than a tick's
    plan needs leaves its buffers alone, returns False and reports the
    slots needed; a batch built with that many serves the tick, and its
    (uncaptured) calls equal an eager batch's bit for bit."""
    from hayate_amd.tick_graph import StaticTickBatch

    say("[static tick batch: slot capacity]")
    q_lens = [256, 64]
    lens = [6000, 3000]  # deep prefixes: the planner splits the first chunk's tiles
    w = _custom_workload(32, 8, lens, q_lens, seed=12)
    m, hs = w.manager, w.handles
    eager = PagedKVBatch(m, q_lens, list(lens), [list(h.pages) for h in hs], varlen=True,
                         num_q_heads=32)
    need = eager.plan(32).host.n_prefill_slots
    assert need > 0
    max_tokens = max(c + q for c, q in zip(lens, q_lens))
    small = StaticTickBatch(m, q_lens, 32, max_tokens=max_tokens, prefill_slots=need - 1)
    assert not small.refresh(hs) and small.prefill_slots_needed == need
    big = StaticTickBatch(m, q_lens, 32, max_tokens=max_tokens, prefill_slots=need)
    assert big.refresh(hs)
    pre = (m.k_cache.clone(), m.v_cache.clone())
    outs = []
    for batch in (eager, big):
        m.k_cache.copy_(pre[0])
        m.v_cache.copy_(pre[1])
        q_rot = batch.norm_rope_write_layer(0, w.q, w.k, w.v, w.q_norm_w, w.k_norm_w, EPS,
                                            w.cos, w.sin)
        out = batch.attend_layer(q_rot, 0)
        torch.cuda.synchronize()
        outs.append((bits(q_rot), bits(out), layer_bits(m)))
    (qa, oa, (ka, va)), (qb, ob, (kb, vb)) = outs
    assert np.array_equal(qa, qb) and np.array_equal(oa, ob)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
