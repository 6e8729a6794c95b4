"""Prompt-prefill and token-decode timing of the engine.

Counterpart of the reference's benchmarks/cli.py (:98-190), with the same
measurements on this engine:

* prefill: every request's prompt chunks until each has sampled its first
  token, timed between two device synchronisations (cli.py:98-126);
* decode: ``decode_steps`` decode ticks over requests whose prompts were
  prefilled outside the timer (cli.py:128-142);
* one warm-up of each phase, then the median of ``repetitions`` runs; prompt
  tokens per second, decode tokens per second and per-step latency, peak
  allocated device memory (cli.py:145-190).

Prompts are deterministic token sequences of exactly ``context_tokens``
tokens (rotated per request, as cli.py:47-58 does with its seed text): the
tokenizer's encoding of a fixed sentence when the engine has a tokenizer,
seeded random ids otherwise. Stop tokens are disabled while measuring so
every request produces its full token count.

Run as ``python -m hayate_amd.benchmark [--model DIR] --batch-size B
--context-tokens N --decode-steps S [--compile]``; without --model the
engine uses synthetic Qwen3-4B weights; --compile replays ticks from
captured HIP graphs (the reference's CLI flag of the same name compiles
with torch.compile).
"""

from __future__ import annotations

import argparse
import gc
import json
import statistics
import time
from contextlib import contextmanager
from pathlib import Path
from typing import Callable, List, Optional

import torch

from .constants import DEFAULT_KV_CACHE_TOKENS, DEFAULT_KV_PAGE_SIZE, MAX_BATCH_SIZE
from .engine import Engine, Request

SEED_TEXT = "Paged attention keeps every request's keys and values in fixed-size pages. "


def prompt_tokens(engine: Engine, length: int, offset: int, seed: int = 0) -> List[int]:
    """A repeatable prompt of exactly `length` tokens, rotated by `offset`."""
    if engine.tokenizer is not None:
        base = engine.tokenizer.encode(SEED_TEXT, add_special_tokens=False)
        if not base:
            raise RuntimeError("the benchmark's seed text produced no tokens")
    else:
        g = torch.Generator().manual_seed(seed)
        vocab = engine.model.embed_tokens.weight.shape[0]
        base = torch.randint(0, vocab, (61,), generator=g).tolist()
    shift = offset % len(base)
    base = base[shift:] + base[:shift]
    return (base * (length // len(base) + 1))[:length]


def make_requests(engine: Engine, batch_size: int, context_tokens: int,
                  output_tokens: int) -> List[Request]:
    """Benchmark requests, prepared as add_request would prepare them."""
    requests = [Request(id=i, prompt_tokens=prompt_tokens(engine, context_tokens, i),
                        max_tokens=output_tokens) for i in range(batch_size)]
    for r in requests:
        engine._prepare_request(r)
    return requests


@contextmanager
def fixed_generation(engine: Engine):
    """No stop tokens while measuring: every request runs its full length."""
    saved = engine.sampler.stop_token_ids
    engine.sampler.stop_token_ids = set()
    try:
        yield
    finally:
        engine.sampler.stop_token_ids = saved


def release(engine: Engine, requests: List[Request]) -> None:
    """Drop the benchmark's requests and their pages."""
    engine.scheduler.current_batch.clear()
    while not engine.scheduler.pool.empty():
        engine.scheduler.pool.get()
    for r in requests:
        engine.release_request_cache(r)
    gc.collect()


def measure(operation: Callable[[], None]) -> tuple[float, float]:
    """Seconds between two device synchronisations around `operation`, and
    the peak allocated device memory in GB."""
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    start = time.perf_counter()
    operation()
    torch.cuda.synchronize()
    return time.perf_counter() - start, torch.cuda.max_memory_allocated() / 1e9


def prefill_all(engine: Engine, requests: List[Request]) -> None:
    """Prompt chunks until every request has sampled its first token."""
    pending = list(requests)
    while pending:
        engine.prefill_batch(pending)
        pending = [r for r in pending if r.is_prefill]


def prefill_once(engine: Engine, batch_size: int, context_tokens: int) -> tuple[float, float]:
    requests = make_requests(engine, batch_size, context_tokens, 1)
    result = measure(lambda: prefill_all(engine, requests))
    release(engine, requests)
    return result


def decode_once(engine: Engine, batch_size: int, context_tokens: int,
                decode_steps: int) -> tuple[float, float]:
    requests = make_requests(engine, batch_size, context_tokens, decode_steps + 1)
    prefill_all(engine, requests)

    def decode():
        for _ in range(decode_steps):
            engine.decode_batch(requests)

    result = measure(decode)
    release(engine, requests)
    return result


def _median(samples):
    return (statistics.median(s[0] for s in samples), statistics.median(s[1] for s in samples))


def run(engine: Engine, batch_size: int = 1, context_tokens: int = 512, decode_steps: int = 64,
        repetitions: int = 3) -> List[dict]:
    """Warm-up, then the median prefill and decode measurements (cli.py:145-190)."""
    if batch_size > min(engine.scheduler.max_batch_size, engine.paged_cache.max_requests):
        raise ValueError("batch size exceeds the engine's batch limit")
    if context_tokens + decode_steps > engine.max_position_embeddings:
        raise ValueError(f"context and decode steps exceed the "
                         f"{engine.max_position_embeddings}-token window")
    with fixed_generation(engine):
        prefill_once(engine, batch_size, context_tokens)
        prefill_s, prefill_gb = _median(
            [prefill_once(engine, batch_size, context_tokens) for _ in range(repetitions)])
        decode_once(engine, batch_size, context_tokens, decode_steps)
        decode_s, decode_gb = _median(
            [decode_once(engine, batch_size, context_tokens, decode_steps)
             for _ in range(repetitions)])
    return [
        {"phase": "prefill", "latency_ms": prefill_s * 1e3,
         "tokens_per_second": batch_size * context_tokens / prefill_s,
         "peak_vram_gb": prefill_gb},
        {"phase": "decode", "latency_ms_per_step": decode_s * 1e3 / decode_steps,
         "tokens_per_second": batch_size * decode_steps / decode_s,
         "peak_vram_gb": decode_gb},
    ]


def _positive(value: str) -> int:
    n = int(value)
    if n < 1:
        raise argparse.ArgumentTypeError("expected a positive integer")
    return n


def main(argv: Optional[List[str]] = None) -> List[dict]:
    ap = argparse.ArgumentParser(description="Prefill and decode timing of the engine.")
    ap.add_argument("--model", default=None,
                    help="local model directory (safetensors + tokenizer); synthetic if omitted")
    ap.add_argument("--batch-size", type=_positive, default=1)
    ap.add_argument("--context-tokens", type=_positive, default=512)
    ap.add_argument("--decode-steps", type=_positive, default=64)
    ap.add_argument("--repetitions", type=_positive, default=3)
    ap.add_argument("--compile", action="store_true",
                    help="replay ticks from captured HIP graphs")
    ap.add_argument("--compile-mode", default="default")
    ap.add_argument("--max-cache-tokens", type=_positive, default=None,
                    help="pool size (default: enough for the batch, at least the engine's)")
    ap.add_argument("--json", type=Path, default=None)
    args = ap.parse_args(argv)
    need = args.batch_size * (args.context_tokens + args.decode_steps + DEFAULT_KV_PAGE_SIZE)
    engine = Engine(args.model, args.compile, args.compile_mode,
                    max_batch_size=max(args.batch_size, MAX_BATCH_SIZE),
                    max_cache_tokens=args.max_cache_tokens or max(need, DEFAULT_KV_CACHE_TOKENS))
    rows = run(engine, args.batch_size, args.context_tokens, args.decode_steps, args.repetitions)
    text = json.dumps(rows, indent=2)
    print(text)
    if args.json is not None:
        args.json.write_text(text + "\n")
    return rows


if __name__ == "__main__":
    main()
