"""The engine (hayate_amd/engine.py) on the GPU, checked layer by layer.

A small Qwen3-shaped model (Qwen3-4B attention heads: 32 q / 8 kv, head_dim
128; hidden 4096, 3 layers, vocab 512, random weights) runs real scheduler
ticks: prompt chunks of up to 512 tokens and decode tokens in one varlen
batch per tick, greedy sampling, commit, release. Layer 1's o_proj is the
identity, so its attention module returns the context itself; on every tick
a hook records that layer's input, its pool before and after the layer and
its output, and the test replays the layer through the oracle (fused q/k/v
projection by the module, then norm + rope + append + attention): pools bit
for bit, context within the attention tolerances.

The prefix-cache test checks that a hit shares the prompt's pages (no
gather, no scatter: refcounts instead), that the first append into the
shared partial page copies it, and that the request attends correctly.
"""

import numpy as np
import pytest
import torch

from gpu_util import EPS, assert_attention_close, bits, say
from oracle import paged_ref as R

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from hayate_amd.engine import Engine, Request
    from hayate_amd.model import Qwen3Config

    CFG = Qwen3Config(vocab_size=512, hidden_size=4096, num_layers=3, num_heads=32,
                      num_kv_groups=8, head_dim=128, intermediate_size=1024)

CHECK = 1
HQ, HKV, D = 32, 8, 128


def make_engine(**kw):
    eng = Engine(config=CFG, seed=3, max_cache_tokens=16_384, max_batch_size=8,
                 stop_token_ids=set(), **kw)
    with torch.no_grad():
        eng.model.layers[CHECK].self_attn.o_proj.weight.copy_(
            torch.eye(HQ * D, dtype=torch.bfloat16))
    g = torch.Generator(device=eng.device).manual_seed(4)
    eng.paged_cache.k_cache.normal_(generator=g)
    eng.paged_cache.v_cache.normal_(generator=g)
    return eng


class LayerProbe:
    """Records (x, batch, pools before, pools after, output) of one
    layer's attention module on every forward."""

    def __init__(self, eng):
        self.eng = eng
        self.records = []
        attn = eng.model.layers[CHECK].self_attn
        self._pre = attn.register_forward_pre_hook(self.before)
        self._post = attn.register_forward_hook(self.after)

    def pools(self):
        torch.cuda.synchronize()
        m = self.eng.paged_cache
        return bits(m.k_cache[CHECK, 0]), bits(m.v_cache[CHECK, 0])

    def before(self, mod, args):
        batch = args[7]
        pages = [[int(p) for p in row if p >= 0] for row in batch._table_np]
        self.records.append({"x": args[0].detach().clone(), "pre": self.pools(),
                             "q_lens": list(batch.q_lens),
                             "cache_lens": list(batch.cache_lens_host), "pages": pages})

    def after(self, mod, args, out):
        rec = self.records[-1]
        rec["post"] = self.pools()
        rec["y"] = out[0].detach().clone()

    def check_all(self, tables):
        mod = self.eng.model.layers[CHECK].self_attn
        for i, rec in enumerate(self.records):
            pk, pv = rec["pre"][0].copy(), rec["pre"][1].copy()
            with torch.inference_mode():
                q, k, v = mod.project_qkv(rec["x"])
            n = sum(rec["q_lens"])
            q_rot = R.qknorm_rope_append(
                bits(q).reshape(n, HQ, D), bits(k).reshape(n, HKV, D),
                bits(v).reshape(n, HKV, D), bits(mod.q_norm.weight), bits(mod.k_norm.weight),
                EPS, tables[0], tables[1], pk, pv, rec["pages"], rec["cache_lens"],
                rec["q_lens"], 128)
            ctx = R.paged_attention(q_rot, pk, pv, rec["pages"], rec["cache_lens"],
                                    rec["q_lens"], 128)
            what = f"forward {i} q_lens={rec['q_lens']} cache={rec['cache_lens']}"
            assert np.array_equal(rec["post"][0], pk), f"{what}: K pool"
            assert np.array_equal(rec["post"][1], pv), f"{what}: V pool"
            assert_attention_close(bits(rec["y"]).reshape(n, HQ, D), ctx, what)
        self.records.clear()


def tables_of(eng):
    return eng.model.cos.cpu().numpy(), eng.model.sin.cpu().numpy()


def prompt(seed, n):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, CFG.vocab_size, (n,), generator=g).tolist()


def test_engine_ticks_match_the_oracle_layer_by_layer():
    say("[engine: 3 requests, chunked prefill + decode, layer 1 vs oracle]")
    eng = make_engine()
    probe = LayerProbe(eng)
    tables = tables_of(eng)
    reqs = []
    for i, n in enumerate((700, 300, 50)):
        r = Request(id=i, prompt_tokens=prompt(10 + i, n), max_tokens=4)
        eng.add_request(r)
        reqs.append(r)
    shapes = []
    while eng.generate():
        shapes.append((eng.last_tick.prefill_tokens, eng.last_tick.decode_tokens))
        probe.check_all(tables)
    say(f"  ticks (prefill, decode tokens): {shapes}")
    # tick 1: chunks 512 + 300 + 50; tick 2: A's last 188 + two decodes; ...
    assert shapes[0] == (862, 0) and shapes[1] == (188, 2)
    assert len(shapes) >= 4 and all(p == 0 for p, _ in shapes[2:])
    for r in reqs:
        assert r.is_completed and len(r.tokens) == 4
        assert r.paged_cache is None  # released after completion
    assert eng.paged_cache.free_page_count == eng.paged_cache.num_pages


def test_prefix_cache_hit_shares_pages():
    say("[engine: prefix-cache hit shares pages]")
    eng = make_engine(enable_prefix_cache=True, prefix_cache_max_tokens=4096)
    probe = LayerProbe(eng)
    tables = tables_of(eng)
    tokens = prompt(20, 300)
    first = Request(id=0, prompt_tokens=list(tokens), max_tokens=3)
    eng.add_request(first)
    eng.generate()  # prefill: the prompt's pages go to the prefix cache
    probe.check_all(tables)
    assert not first.is_prefill and len(eng.prefix_cache) == 1
    owner_pages = list(first.paged_cache.pages)
    m = eng.paged_cache
    assert [m.page_refcount(p) for p in owner_pages] == [2, 2, 2]

    def forbidden(*a, **k):
        raise AssertionError("a prefix hit must not gather or scatter")

    m.import_cache = forbidden
    m._gather = forbidden
    second = Request(id=1, prompt_tokens=list(tokens), max_tokens=3)
    eng.add_request(second)  # hit: 299 tokens (max_prefix_len = len - 1)
    assert second.kv_cache.length == 299
    eng.generate()  # first decodes; second prefills one token at position 299
    probe.check_all(tables)
    pages = second.paged_cache.pages
    assert pages[:2] == owner_pages[:2], "full prompt pages are shared"
    assert pages[2] != owner_pages[2], "the partial page was copied on write"
    assert m.page_refcount(owner_pages[0]) == 3  # first, the cache entry, second
    # the copied page holds the prompt's keys (the shared tokens 256..298)
    k = m.k_cache[:, 0]
    assert torch.equal(k[:, :, pages[2] * 128 : pages[2] * 128 + 43].view(torch.int16),
                       k[:, :, owner_pages[2] * 128 : owner_pages[2] * 128 + 43]
                       .view(torch.int16))
    while eng.generate():
        probe.check_all(tables)
    assert first.is_completed and second.is_completed
    eng.clear_prefix_cache()
    assert m.free_page_count == m.num_pages


def test_prefill_batch_and_decode_batch_match_generate():
    """The reference's call shapes (engine.py:226-289: prefill_batch until
    every prompt is done, then decode_batch) give the tokens the scheduler
    path gives; two requests of equal length keep every tick's shape the
    same on both paths, so the tokens must agree exactly."""
    say("[engine: prefill_batch / decode_batch against generate]")
    prompts = [prompt(30, 700), prompt(31, 700)]
    eng = make_engine()
    ra = [Request(id=i, prompt_tokens=list(p), max_tokens=4) for i, p in enumerate(prompts)]
    for r in ra:
        eng.add_request(r)
    while eng.generate():
        pass
    eng = make_engine()
    rb = [Request(id=i, prompt_tokens=list(p), max_tokens=4) for i, p in enumerate(prompts)]
    for r in rb:
        eng._prepare_request(r)
    pending = list(rb)
    while pending:
        eng.prefill_batch(pending)
        pending = [r for r in pending if r.is_prefill]
    with pytest.raises(ValueError):
        eng.prefill_batch(rb)  # prompts done
    while not all(r.is_completed for r in rb):
        eng.decode_batch([r for r in rb if not r.is_completed])
    assert [r.tokens for r in ra] == [r.tokens for r in rb]
    assert all(len(r.tokens) == 4 for r in rb)


def test_benchmark_reports_prefill_and_decode():
    """hayate_amd.benchmark (the reference's benchmarks/cli.py method) on a
    small run: both phases timed, every page returned afterwards."""
    from hayate_amd import benchmark

    say("[engine: benchmark.run]")
    eng = make_engine()
    rows = benchmark.run(eng, batch_size=2, context_tokens=200, decode_steps=3, repetitions=1)
    assert [r["phase"] for r in rows] == ["prefill", "decode"]
    assert rows[0]["tokens_per_second"] > 0 and rows[1]["tokens_per_second"] > 0
    assert rows[1]["latency_ms_per_step"] > 0
    say(f"  {rows}")
    assert eng.paged_cache.free_page_count == eng.paged_cache.num_pages


def test_compiled_engine_replays_decode_graphs_like_eager():
    """Engine(compile=True) replays decode ticks from captured HIP graphs
    (tick_graph.py). Over ticks that cross page boundaries, with the
    batch shrinking as requests finish (3, then 2, then 1 sequences: one
    capture per batch size; the one prompt tick's shape occurs once and
    runs eagerly), the greedy tokens equal the eager engine's."""
    say("[engine: decode graphs against eager]")
    lengths, max_tokens = (120, 250, 40), (12, 30, 8)
    prompts = [prompt(40 + i, n) for i, n in enumerate(lengths)]

    def run(compiled):
        eng = make_engine(compile=compiled)
        reqs = [Request(id=i, prompt_tokens=list(p), max_tokens=m)
                for i, (p, m) in enumerate(zip(prompts, max_tokens))]
        for r in reqs:
            eng.add_request(r)
        while eng.generate():
            pass
        return eng, [r.tokens for r in reqs]

    eager, t_eager = run(False)
    graphs, t_graph = run(True)
    assert eager.tick_graphs is None
    runner = graphs.tick_graphs
    say(f"  captures {runner.captures}, replays {runner.replays}")
    # one capture per batch size, although the plan's chunk count changes
    # every 64 tokens of total context at these lengths
    assert runner.captures == 3 and runner.replays >= 25
    assert t_graph == t_eager
    assert graphs.paged_cache.free_page_count == graphs.paged_cache.num_pages


def test_compiled_engine_with_prefix_cache_and_admission_matches_eager():
    """A longer run: 10 requests through a batch limit of 4 (admission
    over time, so prefill chunks, mixed ticks and decode ticks of sizes 1-4
    alternate), half of them repeating an earlier prompt (prefix-cache hits
    whose shared partial page is copied on the first append, inside decode
    ticks replayed from graphs). Tokens equal the eager engine's; every
    page comes back."""
    say("[engine: decode graphs + prefix cache + admission]")
    base = [prompt(60 + i, n) for i, n in enumerate((300, 130, 520, 90, 260))]
    prompts = base + [list(p) for p in base]
    max_tokens = [3 + (i * 7) % 9 for i in range(len(prompts))]

    def run(compiled):
        eng = make_engine(compile=compiled, enable_prefix_cache=True,
                          prefix_cache_max_tokens=4096)
        eng.scheduler.max_batch_size = 4
        reqs, hits = [], 0
        for i, (p, m) in enumerate(zip(prompts, max_tokens)):
            if i == len(base):
                # the repeats arrive once the originals' prompts are cached
                while any(r.is_prefill for r in reqs):
                    eng.generate()
            r = Request(id=i, prompt_tokens=list(p), max_tokens=m)
            eng.add_request(r)
            hits += r.kv_cache is not None
            reqs.append(r)
        while eng.generate():
            pass
        eng.clear_prefix_cache()
        assert eng.paged_cache.free_page_count == eng.paged_cache.num_pages
        return eng, [r.tokens for r in reqs], hits

    _, t_eager, hits_eager = run(False)
    eng, t_graph, hits_graph = run(True)
    say(f"  prefix hits {hits_graph}, captures {eng.tick_graphs.captures}, "
        f"replays {eng.tick_graphs.replays} ({eng.tick_graphs.prompt_replays} with prompt chunks)")
    assert hits_eager == hits_graph >= 3
    assert eng.tick_graphs.replays > 0
    assert t_graph == t_eager


def test_compiled_engine_replays_prompt_and_mixed_ticks_like_eager():
    """Ticks with prompt chunks replayed from graphs: three prompts of
    1,300, 1,300 and 700 tokens in 256-token chunks give the shapes
    (256, 256, 256) twice, (256, 256, 188), then (256, 256, 1) twice (the
    third request decodes while the others prefill) and decode ticks. A
    prompt shape is captured on its second occurrence, at a larger cached
    length than the first, so its plan differs (more split query tiles;
    the padded item lists carry other real counts). The greedy tokens
    equal the eager engine's, and so do both pools bit for bit at the end:
    every layer's appended K/V rows of every tick, replayed or not."""
    say("[engine: prompt and mixed ticks from graphs against eager]")
    lengths, max_tokens = (1300, 1300, 700), (6, 5, 9)
    prompts = [prompt(70 + i, n) for i, n in enumerate(lengths)]

    def run(compiled):
        eng = make_engine(compile=compiled, prefill_chunk_size=256)
        reqs = [Request(id=i, prompt_tokens=list(p), max_tokens=m)
                for i, (p, m) in enumerate(zip(prompts, max_tokens))]
        for r in reqs:
            eng.add_request(r)
        sizes = []
        while eng.generate():
            sizes.append((eng.last_tick.prefill_tokens, eng.last_tick.decode_tokens))
        torch.cuda.synchronize()
        return eng, [r.tokens for r in reqs], sizes

    eager, t_eager, s_eager = run(False)
    eng, t_graph, s_graph = run(True)
    runner = eng.tick_graphs
    say(f"  ticks (prefill, decode tokens): {s_graph}")
    say(f"  captures {runner.captures}, replays {runner.replays}, "
        f"with prompt chunks {runner.prompt_replays}")
    assert s_graph == s_eager
    assert s_graph[:5] == [(768, 0), (768, 0), (700, 0), (512, 1), (512, 1)]
    assert t_graph == t_eager
    assert runner.prompt_replays >= 2
    for name in ("k_cache", "v_cache"):
        a = getattr(eager.paged_cache, name).view(torch.int16)
        b = getattr(eng.paged_cache, name).view(torch.int16)
        assert torch.equal(a, b), f"{name} differs between the eager and the replayed engine"
    assert eng.paged_cache.free_page_count == eng.paged_cache.num_pages
