"""GPU parity of the ops either side of the attention path.

* Batched sampling (hayate_amd/sampler.py) on device logits at Qwen3's
  vocabulary (151,936) and batch 32, with a seeded device generator, against
  the reference's per-row semantics (hayate/engine/sampler.py:39-65): greedy
  is argmax (first index among ties); top-k keeps exactly the tokens whose
  score is >= the k-th largest; top-p keeps the shortest descending prefix
  whose mass exceeds p plus the crossing token; temperature divides the
  logits; rows with different settings in one batch do not interact; the
  draws follow softmax(logits / T) over the kept set. The kept sets are
  planted: each row's logits put a few tokens at chosen values over a
  background whose total mass would dominate if a filter let it through.
* The fused q/k/v projection (one GEMM over [W_q; W_k; W_v]) against the
  reference's three projections (attention.py:58-60) in bf16 at Qwen3-4B
  width for 1, 32 and 512 tokens.
* The module on a mixed varlen tick with the oracle fed from the three
  separate projections, not from the module's own fused GEMM.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gpu_util import EPS, assert_attention_close, bits, layer_bits, say
from oracle import paged_ref as R

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from hayate_amd import PagedKVCacheManager
    from hayate_amd.attention import GroupedQueryAttention
    from hayate_amd.rope import compute_rope_params
    from hayate_amd.sampler import sample_batch

DEV = "cuda"
VOCAB = 151_936
B = 32


# ----------------------------------------------------------------- sampling
class PlantedRows:
    """Logits (B, VOCAB) bf16 on the device, one sampling setting per row,
    and the set of token ids each row may return (None: any)."""

    def __init__(self, seed):
        self.g = torch.Generator().manual_seed(seed)
        self.logits = torch.empty(B, VOCAB)
        self.temperature, self.top_k, self.top_p = [], [], []
        self.support = []
        self.freq = {}  # row -> (token ids, expected probabilities)

    def _positions(self, n):
        return torch.randperm(VOCAB, generator=self.g)[:n].tolist()

    def plant_greedy(self, row, ties):
        x = torch.randn(VOCAB, generator=self.g)
        if ties:  # two tokens share the maximum: argmax is the first of them
            pos = sorted(self._positions(2))
            x[pos] = x.max() + 1.0
        self.logits[row] = x
        self._set(row, 0.0, None, None, None)

    def plant_top_k(self, row, k, temperature, tie=False, extra=5):
        """k + extra planted tokens 3.0, 2.75, ... over a background near -6
        (at T = 1 the background holds ~150x the planted mass); with tie,
        one more token equals the k-th value and must be kept too."""
        x = -6.0 + 0.5 * torch.randn(VOCAB, generator=self.g)
        pos = self._positions(k + extra + 1)
        vals = [3.0 - 0.25 * j for j in range(k + extra)]
        for p, v in zip(pos, vals):
            x[p] = v
        keep = pos[:k]
        if tie:
            x[pos[-1]] = vals[k - 1]
            keep = keep + [pos[-1]]
        self.logits[row] = x
        self._set(row, temperature, k, None, set(keep))
        return pos, vals

    def plant_top_p(self, row, probs, p, top_k=None, temperature=1.0):
        """Planted tokens with logits log(probs) (descending), background at
        -40 (mass ~1e-12); the kept set is the shortest prefix whose mass
        exceeds p, the crossing token included."""
        assert all(a > b for a, b in zip(probs, probs[1:]))
        x = torch.full((VOCAB,), -40.0)
        pos = self._positions(len(probs))
        for q, v in zip(pos, probs):
            x[q] = math.log(v)
        self.logits[row] = x
        # expected set: over the tokens top-k leaves, at temperature T
        cand = probs[: top_k] if top_k else probs
        w = [v ** (1.0 / temperature) for v in cand]
        w = [v / sum(w) for v in w]
        n, mass = 0, 0.0
        while True:
            mass += w[n]
            n += 1
            if mass > p or n == len(w):
                break
        # keep the design away from a rounding decision
        if p < 1:
            assert min(abs(sum(w[:j]) - p) for j in range(1, len(w) + 1)) > 5e-3
        self._set(row, temperature, top_k, p, set(pos[:n]))
        return pos[:n], w[:n]

    def _set(self, row, t, k, p, support):
        self.temperature.append(t)
        self.top_k.append(k)
        self.top_p.append(p)
        self.support.append(support)


def build_rows():
    rows = PlantedRows(123)
    for r in range(4):
        rows.plant_greedy(r, ties=r >= 2)
    for r, (k, t, tie) in enumerate([(1, 0.7, False), (2, 1.0, False), (3, 1.3, False),
                                     (5, 1.0, True), (8, 0.5, True), (8, 2.0, False),
                                     (13, 1.0, False), (20, 1.0, False)]):
        rows.plant_top_k(4 + r, k, t, tie=tie)
    probs = [0.3, 0.2, 0.15, 0.12, 0.1, 0.08, 0.05 - 1e-9]
    for r, p in enumerate([0.25, 0.45, 0.62, 0.8, 0.9, 0.97, 0.99, 1.0]):
        rows.plant_top_p(12 + r, probs, p)
    # top-k then top-p at temperature 2 (the CPU test's case, planted)
    for r, (k, p) in enumerate([(3, 0.5), (4, 0.6), (5, 0.9), (2, 0.99)]):
        rows.plant_top_p(20 + r, probs, p, top_k=k, temperature=2.0)
    # eight identical rows for the frequency check: top-k 4 at T = 1.5
    pos = torch.randperm(VOCAB, generator=rows.g)[:6].tolist()
    vals = [2.0, 1.5, 1.0, 0.5, 0.4, 0.3]
    x = -8.0 + 0.5 * torch.randn(VOCAB, generator=rows.g)
    for p, v in zip(pos, vals):
        x[p] = v
    w = [math.exp(v / 1.5) for v in vals[:4]]
    expect = [v / sum(w) for v in w]
    for r in range(24, 32):
        rows.logits[r] = x
        rows._set(r, 1.5, 4, None, set(pos[:4]))
        rows.freq[r] = (pos[:4], expect)
    rows.logits = rows.logits.to(torch.bfloat16).to(DEV)
    return rows


def test_greedy_sampling_is_argmax_on_device_logits():
    """A batch of 32 greedy rows at vocab 151,936 in bf16 (the engine's
    logits dtype), with planted ties in half of them: the sampler returns
    the first maximal index of every row, as the reference's per-row
    argmax does, equal to numpy's on the host copy."""
    say("[sampler: greedy at vocab 151936]")
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, VOCAB, generator=g)
    for r in range(0, B, 2):
        pos = sorted(torch.randperm(VOCAB, generator=g)[:3].tolist())
        x[r, pos] = x[r].max() + 0.5
    logits = x.to(torch.bfloat16).to(DEV)
    out = sample_batch(logits, [0.0] * B, [None] * B, [None] * B)
    host = logits.float().cpu().numpy()
    assert out.shape == (B, 1) and out.dtype == torch.long
    assert out.flatten().tolist() == np.argmax(host, axis=1).tolist()
    per_row = [int(torch.argmax(logits[r])) for r in range(B)]
    assert out.flatten().tolist() == per_row


def test_sampling_supports_and_frequencies_on_device():
    """One batch mixing greedy, top-k (with ties at the k-th), top-p (the
    crossing token kept), top-k + top-p at temperature 2 and a frequency
    block, drawn 300 times with a seeded device generator: every draw lies
    in its row's planted kept set, every kept token with at least 3 %
    probability appears, and the frequency rows follow softmax(logits / T)
    over the top 4 within five standard errors."""
    say("[sampler: planted supports at vocab 151936, batch 32]")
    rows = build_rows()
    gen = torch.Generator(device=DEV).manual_seed(2024)
    calls = 300
    draws = torch.empty(calls, B, dtype=torch.long, device=DEV)
    for i in range(calls):
        draws[i] = sample_batch(rows.logits, rows.temperature, rows.top_k, rows.top_p,
                                gen).flatten()
    draws = draws.cpu().numpy()
    host = rows.logits.float().cpu().numpy()
    for r in range(B):
        seen = set(draws[:, r].tolist())
        if rows.temperature[r] == 0:
            assert seen == {int(np.argmax(host[r]))}, r
            continue
        support = rows.support[r]
        assert seen <= support, (r, sorted(seen - support)[:5])
        # every kept token with >= 3 % probability shows up in 300 draws
        # (a miss has probability below 1e-4)
        ids, q = kept_probs(rows, r)
        frequent = {i for i, v in zip(ids, q) if v >= 0.03}
        assert frequent <= seen, (r, sorted(frequent - seen))
    counts = np.zeros(4)
    for r, (pos, expect) in rows.freq.items():
        for j, p in enumerate(pos):
            counts[j] += np.count_nonzero(draws[:, r] == p)
    n = calls * len(rows.freq)
    assert counts.sum() == n
    for c, q in zip(counts, expect):
        se = math.sqrt(q * (1 - q) / n)
        say(f"  frequency {c / n:.4f} expected {q:.4f} (se {se:.4f})")
        assert abs(c / n - q) <= 5 * se


def kept_probs(rows, r):
    """(kept token ids, their probabilities): softmax of the row's own
    logits / T (host copy, float64) over its planted kept set."""
    x = rows.logits[r].float().cpu().double()
    ids = sorted(rows.support[r], key=lambda i: -float(x[i]))
    s = torch.tensor([float(x[i]) for i in ids], dtype=torch.float64) / rows.temperature[r]
    return ids, torch.softmax(s, dim=0).tolist()


def test_sampling_rows_do_not_interact():
    """The same planted row drawn alone and inside the mixed batch: its
    supports are the same, and changing every other row's settings (all
    greedy, then all top-k 1) leaves it inside the same set."""
    say("[sampler: row independence]")
    rows = build_rows()
    r = 14  # top-p 0.62: three kept tokens
    gen = torch.Generator(device=DEV).manual_seed(5)
    alone = set()
    for _ in range(200):
        alone |= set(sample_batch(rows.logits[r : r + 1], [1.0], [None], [0.62], gen)
                     .flatten().tolist())
    assert alone == rows.support[r]
    for t_other, k_other in ((0.0, None), (1.0, 1)):
        temps = [t_other] * B
        ks = [k_other] * B
        ps = [None] * B
        temps[r], ks[r], ps[r] = 1.0, None, 0.62
        seen = set()
        for _ in range(200):
            out = sample_batch(rows.logits, temps, ks, ps, gen).flatten().tolist()
            seen.add(out[r])
        assert seen == rows.support[r]


# --------------------------------------------------------------- projection
D_IN, HQ, HKV, D = 2560, 32, 8, 128


def qwen_module(seed):
    g = torch.Generator().manual_seed(seed)
    mod = GroupedQueryAttention(D_IN, HQ, HKV, D, dtype=torch.bfloat16).to(DEV)
    with torch.no_grad():
        for lin in (mod.q_proj, mod.k_proj, mod.v_proj, mod.o_proj):
            lin.weight.copy_((torch.randn(lin.weight.shape, generator=g)
                              / math.sqrt(lin.weight.shape[1])).to(torch.bfloat16))
        mod.q_norm.weight.copy_((1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16))
        mod.k_norm.weight.copy_((1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16))
    return mod


def ulps_bits(a, b):
    """Distance in bf16 units in the last place between two arrays of bf16
    bit patterns (mapped to a monotone integer line)."""
    ia = a.astype(np.int32)
    ib = b.astype(np.int32)
    ia = np.where(ia & 0x8000, 0x8000 - ia, ia)
    ib = np.where(ib & 0x8000, 0x8000 - ib, ib)
    return np.abs(ia - ib)



# hipBLASLt may pick a different kernel for the fused GEMM's wider N than
# for each projection alone, which changes the fp32 accumulation order: a
# few outputs then round to a neighbouring bf16 value. Measured on MI355X
# at 32 tokens: 25 of 131,072 q values, 12 of 32,768 k and 10 of 32,768 v
# values differ (bit-exact at 1 token), each by one rounding step of the
# value, or by up to 2 ulps for values near zero, where the 2,560-term
# sums cancel. The bound: at most 0.1 % of the values differ, each by at
# most one bf16 step of the larger of the two values or 1/128 of the
# output's RMS, whichever is larger. A wrong split, stride or weight order
# moves nearly every value by about the RMS.
MAX_FRACTION = 1e-3


def diff_stats(a_bits, b_bits):
    """(fraction of differing values, largest |a - b| over its allowance,
    max ulp): the allowance is one bf16 step (2^(e - 7) for a value in
    [2^e, 2^(e+1))) of max(|a|, |b|), at least RMS(b) / 128."""
    a = R.bf16_to_f32(a_bits).astype(np.float64)
    b = R.bf16_to_f32(b_bits).astype(np.float64)
    rms = math.sqrt(float(np.mean(b * b)))
    big = np.maximum(np.abs(a), np.abs(b))
    step = np.exp2(np.floor(np.log2(np.maximum(big, 1e-30))) - 7)
    allowance = np.maximum(step, rms / 128)
    return (np.count_nonzero(a_bits != b_bits) / a_bits.size,
            float(np.max(np.abs(a - b) / allowance)), int(ulps_bits(a_bits, b_bits).max()))


@pytest.mark.parametrize("tokens", [1, 32, 512])
def test_fused_qkv_projection_equals_three_projections(tokens):
    """project_qkv (one GEMM over the concatenated weight) against
    q_proj(x), k_proj(x), v_proj(x) computed separately in bf16, as the
    reference does (attention.py:58-60), at Qwen3-4B width (d_in 2560,
    4096 + 1024 + 1024 outputs), within the bound above."""
    say(f"[project_qkv vs three projections, {tokens} tokens]")
    mod = qwen_module(31)
    x = torch.randn(1, tokens, D_IN, generator=torch.Generator().manual_seed(tokens)).to(
        torch.bfloat16).to(DEV)
    with torch.inference_mode():
        q, k, v = mod.project_qkv(x)
        q3 = F.linear(x, mod.q_proj.weight).view(1, tokens, HQ, D)
        k3 = F.linear(x, mod.k_proj.weight).view(1, tokens, HKV, D)
        v3 = F.linear(x, mod.v_proj.weight).view(1, tokens, HKV, D)
    torch.cuda.synchronize()
    stats = []
    for name, a, b in (("q", q, q3), ("k", k, k3), ("v", v, v3)):
        frac, over, ulp = diff_stats(bits(a), bits(b))
        say(f"  {name}: {frac:.2e} of values differ, max |diff| / allowance {over:.3f}, "
            f"max {ulp} ulp")
        stats.append((name, frac, over))
    for name, frac, over in stats:
        assert frac <= MAX_FRACTION and over <= 1.0, (name, frac, over)


def test_module_against_oracle_fed_by_three_projections():
    """The module on a mixed varlen tick (prefill chunks and decode tokens)
    at Qwen3-4B width, checked against the oracle whose q, k and v come
    from the reference's three separate projections (attention.py:58-60),
    not from the module's fused GEMM: the context (read at o_proj's input)
    within the attention tolerances, the appended K/V rows within the
    projection bound above, every other pool value untouched."""
    say("[module vs oracle fed by q_proj/k_proj/v_proj]")
    mod = qwen_module(32)
    cos, sin = compute_rope_params(D, 1_000_000, 40_960, device=DEV)
    cache_lens = [0, 700, 129, 3000]
    q_lens = [300, 1, 64, 1]
    m = PagedKVCacheManager(1, HKV, D, 16_384, 128, 4, torch.bfloat16, DEV, num_q_heads=HQ)
    g = torch.Generator(device=DEV).manual_seed(33)
    m.k_cache.normal_(generator=g)
    m.v_cache.normal_(generator=g)
    perm = torch.randperm(m.num_pages, generator=torch.Generator().manual_seed(34)).tolist()
    handles, cur = [], 0
    for c in cache_lens:
        h = m.allocate()
        need = math.ceil(c / 128)
        m.claim_pages(h, perm[cur : cur + need])
        cur += need
        h.length = c
        handles.append(h)
    pre_k, pre_v = layer_bits(m)
    batch = m.begin_tick(handles, q_lens)
    page_lists = [list(h.pages) for h in handles]
    n = sum(q_lens)
    x = torch.randn(1, n, D_IN, generator=torch.Generator().manual_seed(35)).to(
        torch.bfloat16).to(DEV)
    # the module's o_proj is random here, so the check reads the context
    # through a hook on o_proj's input
    ctx = {}
    hook = mod.o_proj.register_forward_pre_hook(lambda _m, a: ctx.setdefault("x", a[0].clone()))
    with torch.inference_mode():
        mod(x, cos, sin, None, None, None, paged_cache=batch, layer_idx=0)
        q3 = F.linear(x, mod.q_proj.weight)[0].view(n, HQ, D)
        k3 = F.linear(x, mod.k_proj.weight)[0].view(n, HKV, D)
        v3 = F.linear(x, mod.v_proj.weight)[0].view(n, HKV, D)
    hook.remove()
    torch.cuda.synchronize()
    pk, pv = pre_k.copy(), pre_v.copy()
    q_rot = R.qknorm_rope_append(bits(q3), bits(k3), bits(v3), bits(mod.q_norm.weight),
                                 bits(mod.k_norm.weight), EPS, cos.cpu().numpy(),
                                 sin.cpu().numpy(), pk, pv, page_lists, cache_lens, q_lens, 128)
    # the appended rows carry the projection's rounding differences; every
    # other pool value is untouched
    post_k, post_v = layer_bits(m)
    rows = np.zeros(post_k.shape[:2], dtype=bool)  # (kv head, pool token) rows appended
    for c, ql, pl in zip(cache_lens, q_lens, page_lists):
        rows[:, R.physical_positions(pl, c + ql, 128)[c:]] = True
    for name, got, want in (("K", post_k, pk), ("V", post_v, pv)):
        assert np.array_equal(got[~rows], want[~rows]), f"{name}: untouched rows changed"
        frac, over, ulp = diff_stats(got[rows], want[rows])
        say(f"  {name} rows appended: {frac:.2e} of values differ, max |diff| / allowance "
            f"{over:.3f}, max {ulp} ulp")
        # a normed k row can move by one rounding step in several values
        # when one input value moves: at most 1 % of the values, two steps
        assert frac <= 1e-2 and over <= 2.0, name
    expect = R.paged_attention(q_rot, pk, pv, page_lists, cache_lens, q_lens, 128)
    assert_attention_close(bits(ctx["x"]).reshape(n, HQ, D), expect, "module, three projections")
