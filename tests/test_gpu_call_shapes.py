"""GPU parity of the call shapes the reference Engine makes after the drop-in.

The reference's tick (hayate/engine/engine.py:209-224) builds one batch with
``begin_batch(handles, T)``, runs every layer's GroupedQueryAttention.forward
on it (attention.py:55-76: projections, q/k norm, rope, write_layer,
attend_layer) and commits with ``commit_batch``. Prefill groups have equal T
(engine.py:257-261); a decode tick is ``begin_batch(handles, 1)``
(engine.py:278-289). These tests run exactly those shapes through the HIP
path and check them against the oracle:

* the module at T == 1 on a uniform batch (the fused decode_layer on
  (B, 1, H, D) strides) at the batch-32 decode lengths;
* write_layer + attend_layer at T == 1 on the uniform (B, H, 1, D) layout
  (the plain decode kernel), and write_layer on a packed varlen tick;
* the module on a uniform 512-token prefill;
* the module's varlen branch (one packed begin_tick mixing prefill chunks
  and decode tokens, and an all-decode varlen tick);
* a multi-tick loop with two layers sharing each batch: a 512-token prefill,
  commit, decode ticks that cross a page boundary, a mixed varlen tick.

o_proj is the identity (d_in = num_heads * head_dim), so the module's output
is the attention context bit for bit; it is held to the attention
tolerances (max-abs 2e-2, mean-abs 2e-3, relative RMS 1e-2). Pools and
rotated keys are compared bit for bit after every layer of every tick.
"""

import math

import numpy as np
import pytest
import torch

from gpu_util import EPS, assert_attention_close, bits, layer_bits, say
from oracle import paged_ref as R

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from hayate_amd import PagedKVCacheManager
    from hayate_amd.attention import GroupedQueryAttention
    from hayate_amd.rope import compute_rope_params

DEV = "cuda"
HQ, HKV, D, P = 32, 8, 128, 128
D_IN = HQ * D


def make_module(seed):
    """GroupedQueryAttention with Qwen3-4B heads, random projections, norm
    weights 1 + 0.1 N(0, 1) and an identity o_proj."""
    g = torch.Generator().manual_seed(seed)
    mod = GroupedQueryAttention(D_IN, HQ, HKV, D, dtype=torch.bfloat16).to(DEV)
    with torch.no_grad():
        for lin in (mod.q_proj, mod.k_proj, mod.v_proj):
            w = torch.randn(lin.weight.shape, generator=g) / math.sqrt(D_IN)
            lin.weight.copy_(w.to(torch.bfloat16))
        mod.q_norm.weight.copy_((1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16))
        mod.k_norm.weight.copy_((1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16))
        mod.o_proj.weight.copy_(torch.eye(D_IN, dtype=torch.bfloat16))
    return mod


class Tables:
    def __init__(self):
        self.cos, self.sin = compute_rope_params(D, 1_000_000, 40_960, device=DEV)
        self.cos_np = self.cos.cpu().numpy()
        self.sin_np = self.sin.cpu().numpy()


def make_manager(num_layers, pool_tokens, max_requests, seed):
    m = PagedKVCacheManager(num_layers, HKV, D, pool_tokens, P, max_requests, torch.bfloat16,
                            DEV, num_q_heads=HQ)
    g = torch.Generator(device=DEV).manual_seed(seed)
    m.k_cache.normal_(generator=g)
    m.v_cache.normal_(generator=g)
    return m


class OraclePools:
    """Host copy of every layer's pools, advanced by the oracle."""

    def __init__(self, m):
        self.k = [layer_bits(m, l)[0] for l in range(m.num_layers)]
        self.v = [layer_bits(m, l)[1] for l in range(m.num_layers)]

    def check(self, m, what):
        for l in range(m.num_layers):
            gk, gv = layer_bits(m, l)
            assert np.array_equal(gk, self.k[l]), f"{what}: K pool of layer {l} differs"
            assert np.array_equal(gv, self.v[l]), f"{what}: V pool of layer {l} differs"


def expected_layer(mod, x, pools, layer, tables, page_lists, cache_lens, q_lens):
    """Projections of x by the module's own fused q/k/v GEMM, then the oracle's
    norm + rope + append (advancing the host pools) and attention.
    Returns the (N, HQ, D) context."""
    with torch.inference_mode():
        q, k, v = mod.project_qkv(x)
    n = sum(q_lens)
    q_rot = R.qknorm_rope_append(
        bits(q).reshape(n, HQ, D), bits(k).reshape(n, HKV, D), bits(v).reshape(n, HKV, D),
        bits(mod.q_norm.weight), bits(mod.k_norm.weight), EPS, tables.cos_np, tables.sin_np,
        pools.k[layer], pools.v[layer], page_lists, cache_lens, q_lens, P)
    return R.paged_attention(q_rot, pools.k[layer], pools.v[layer], page_lists, cache_lens,
                             q_lens, P)


def run_module(mod, x, batch, layer, tables):
    with torch.inference_mode():
        y, nk, nv = mod(x, tables.cos, tables.sin, None, None, None, paged_cache=batch,
                        layer_idx=layer)
    torch.cuda.synchronize()
    assert nk is None and nv is None
    return y


def place(m, cache_lens, seed):
    """Handles holding `cache_lens` tokens on seeded random pages."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(m.num_pages, generator=g).tolist()
    handles, cur = [], 0
    for c in cache_lens:
        h = m.allocate()
        n = math.ceil(c / P)
        m.claim_pages(h, perm[cur : cur + n])
        cur += n
        h.length = c
        handles.append(h)
    return handles


def pool_for(cache_lens, q=1):
    """Pool tokens for these requests after appending q tokens each."""
    return (sum(math.ceil((c + q) / P) for c in cache_lens) + 8) * P


def decode_b32_lengths():
    g = torch.Generator().manual_seed(1002)
    return [c - 1 for c in torch.randint(256, 4097, (32,), generator=g).tolist()]


def test_module_decode_tick_through_begin_batch():
    """begin_batch(handles, 1) + GroupedQueryAttention.forward at T == 1: the
    reference Engine's decode forward (engine.py:218, attention.py:55-76)."""
    say("[module decode T=1, batch 32]")
    tables = Tables()
    cache_lens = decode_b32_lengths()
    m = make_manager(2, pool_for(cache_lens), 32, 3)
    handles = place(m, cache_lens, 4)
    pools = OraclePools(m)
    mod = make_module(5)
    batch = m.begin_batch(handles, 1)
    page_lists = [list(h.pages) for h in handles]
    x = torch.randn(32, 1, D_IN, generator=torch.Generator().manual_seed(6)).to(
        torch.bfloat16).to(DEV)
    y = run_module(mod, x, batch, 1, tables)
    ctx = expected_layer(mod, x, pools, 1, tables, page_lists, cache_lens, [1] * 32)
    pools.check(m, "decode T=1")
    assert y.shape == (32, 1, D_IN)
    assert_attention_close(bits(y).reshape(32, HQ, D), ctx, "module decode T=1")
    m.commit_batch(handles, 1)
    assert [h.length for h in handles] == [c + 1 for c in cache_lens]


def test_uniform_write_and_attend_at_t1():
    """write_layer + attend_layer on the uniform (B, H, 1, D) layout: the
    plain decode kernel with bhtd strides."""
    say("[uniform write_layer + attend_layer T=1]")
    cache_lens = decode_b32_lengths()
    m = make_manager(1, pool_for(cache_lens), 32, 7)
    handles = place(m, cache_lens, 8)
    pools = OraclePools(m)
    batch = m.begin_batch(handles, 1)
    page_lists = [list(h.pages) for h in handles]
    g = torch.Generator().manual_seed(9)
    k = torch.randn(32, HKV, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(32, HKV, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    q = torch.randn(32, HQ, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    batch.write_layer(0, k, v)
    out = batch.attend_layer(q, 0)
    torch.cuda.synchronize()
    assert out.shape == (32, HQ, 1, D)
    R.kv_append(pools.k[0], pools.v[0], bits(k.transpose(1, 2).reshape(32, HKV, D)),
                bits(v.transpose(1, 2).reshape(32, HKV, D)), page_lists, cache_lens, [1] * 32,
                P)
    pools.check(m, "uniform T=1")
    expect = R.paged_attention(bits(q.transpose(1, 2).reshape(32, HQ, D)), pools.k[0],
                               pools.v[0], page_lists, cache_lens, [1] * 32, P)
    assert_attention_close(bits(out.transpose(1, 2)).reshape(32, HQ, D), expect,
                           "uniform attend T=1")


def test_write_layer_packed_varlen_tick():
    """write_layer on a packed (N, Hkv, D) varlen tick, whose rows are
    addressed by token index alone (the append loads them before it looks
    the token's sequence up), with 8 kv heads and with 12, whose second
    8-head group is partly empty: pools bit-exact against the oracle."""
    cache_lens = [0, 130, 511, 1000, 77]
    q_lens = [300, 1, 1, 64, 129]
    for hkv in (HKV, 12):
        say(f"[write_layer packed varlen tick, {hkv} kv heads]")
        pool = (sum(math.ceil((c + q) / P) for c, q in zip(cache_lens, q_lens)) + 8) * P
        m = PagedKVCacheManager(1, hkv, D, pool, P, len(cache_lens), torch.bfloat16, DEV,
                                num_q_heads=hkv)
        g = torch.Generator(device=DEV).manual_seed(20)
        m.k_cache.normal_(generator=g)
        m.v_cache.normal_(generator=g)
        handles = place(m, cache_lens, 21)
        pools = OraclePools(m)
        batch = m.begin_tick(handles, q_lens)
        page_lists = [list(h.pages) for h in handles]
        n = sum(q_lens)
        gh = torch.Generator().manual_seed(22)
        k = torch.randn(n, hkv, D, generator=gh).to(torch.bfloat16).to(DEV)
        v = torch.randn(n, hkv, D, generator=gh).to(torch.bfloat16).to(DEV)
        batch.write_layer(0, k, v)
        torch.cuda.synchronize()
        R.kv_append(pools.k[0], pools.v[0], bits(k), bits(v), page_lists, cache_lens, q_lens, P)
        pools.check(m, f"packed write_layer, {hkv} kv heads")


def test_module_uniform_prefill_512():
    """begin_batch(handles, 512) + the module: one equal-length prefill group
    as prefill_batch forms it (engine.py:257-261), cached offsets 0 and 777."""
    say("[module uniform prefill T=512]")
    tables = Tables()
    cache_lens = [0, 777]
    m = make_manager(1, 16_384, 2, 10)
    handles = place(m, cache_lens, 11)
    pools = OraclePools(m)
    mod = make_module(12)
    batch = m.begin_batch(handles, 512)
    page_lists = [list(h.pages) for h in handles]
    x = torch.randn(2, 512, D_IN, generator=torch.Generator().manual_seed(13)).to(
        torch.bfloat16).to(DEV)
    y = run_module(mod, x, batch, 0, tables)
    ctx = expected_layer(mod, x, pools, 0, tables, page_lists, cache_lens, [512, 512])
    pools.check(m, "prefill T=512")
    assert_attention_close(bits(y).reshape(1024, HQ, D), ctx, "module prefill T=512")


def test_module_varlen_branch():
    """begin_tick + the module's varlen branch (x of shape (1, N, d_in)):
    a mixed tick (prefill chunks and decode tokens in one packed batch) and
    an all-decode varlen tick (the fused decode launch)."""
    say("[module varlen mixed + all-decode]")
    tables = Tables()
    cache_lens = [0, 1500, 300, 4000, 129, 64]
    q_lens = [200, 1, 512, 1, 70, 1]
    m = make_manager(1, 32_768, 6, 14)
    handles = place(m, cache_lens, 15)
    pools = OraclePools(m)
    mod = make_module(16)
    batch = m.begin_tick(handles, q_lens)
    page_lists = [list(h.pages) for h in handles]
    n = sum(q_lens)
    g = torch.Generator().manual_seed(17)
    x = torch.randn(1, n, D_IN, generator=g).to(torch.bfloat16).to(DEV)
    y = run_module(mod, x, batch, 0, tables)
    ctx = expected_layer(mod, x, pools, 0, tables, page_lists, cache_lens, q_lens)
    pools.check(m, "varlen mixed")
    assert_attention_close(bits(y).reshape(n, HQ, D), ctx, "module varlen mixed")
    m.commit_tick(handles, q_lens)

    cache_lens = [h.length for h in handles]
    batch = m.begin_tick(handles, [1] * 6)
    page_lists = [list(h.pages) for h in handles]
    x = torch.randn(1, 6, D_IN, generator=g).to(torch.bfloat16).to(DEV)
    y = run_module(mod, x, batch, 0, tables)
    ctx = expected_layer(mod, x, pools, 0, tables, page_lists, cache_lens, [1] * 6)
    pools.check(m, "varlen decode")
    assert_attention_close(bits(y).reshape(6, HQ, D), ctx, "module varlen decode")


def test_multi_tick_loop_two_layers():
    """Several ticks with two layers sharing each batch, as the engine's
    layer loop does (qwen.py:137-150): a 512-token prefill of two requests,
    decode ticks whose first append opens a new page, then a varlen tick
    adding a third request's 300-token chunk to the two decodes. Every layer
    of every tick: pools bit-exact, context within tolerance."""
    say("[multi-tick, 2 layers]")
    tables = Tables()
    m = make_manager(2, 8192, 3, 18)
    mods = [make_module(19), make_module(20)]
    pools = OraclePools(m)
    a, b = m.allocate(), m.allocate()
    g = torch.Generator().manual_seed(21)

    def tick(handles, q_lens, uniform):
        cache_lens = [h.length for h in handles]
        if uniform:
            batch = m.begin_batch(handles, q_lens[0])
        else:
            batch = m.begin_tick(handles, q_lens)
        page_lists = [list(h.pages) for h in handles]
        n = sum(q_lens)
        for layer in range(2):
            if uniform:
                x = torch.randn(len(handles), q_lens[0], D_IN, generator=g)
            else:
                x = torch.randn(1, n, D_IN, generator=g)
            x = x.to(torch.bfloat16).to(DEV)
            y = run_module(mods[layer], x, batch, layer, tables)
            ctx = expected_layer(mods[layer], x, pools, layer, tables, page_lists, cache_lens,
                                 q_lens)
            what = f"tick c={cache_lens} q={q_lens} layer {layer}"
            pools.check(m, what)
            assert_attention_close(bits(y).reshape(n, HQ, D), ctx, what)
        if uniform:
            m.commit_batch(handles, q_lens[0])
        else:
            m.commit_tick(handles, q_lens)

    tick([a, b], [512, 512], uniform=True)
    assert a.length == b.length == 512 and len(a.pages) == 4
    for step in range(3):
        tick([a, b], [1, 1], uniform=True)
        assert len(a.pages) == 5  # token 512 opened the fifth page
    c = m.allocate()
    tick([a, b, c], [1, 1, 300], uniform=False)
    assert (a.length, b.length, c.length) == (516, 516, 300)
    tick([a, b, c], [1, 1, 1], uniform=False)
