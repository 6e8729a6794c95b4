"""Continuous-batching engine over the paged-attention path.

The counterpart of the reference's hayate/engine/engine.py:26-348 (with
request.py, scheduler.py and constants.py), on one MI355X:

* same request lifecycle: ``add_request`` validates and tokenizes
  (engine.py:131-181), looks up a reusable prompt prefix, the scheduler
  admits up to ``max_batch_size`` requests per tick (scheduler.py:22-28),
  prompts advance in chunks of ``prefill_chunk_size`` tokens with a cached
  prefix cut back to ``len(prompt) - 1`` (engine.py:236-255), completed
  requests release their pages (engine.py:200-207, 293-298);
* one model forward per tick: the reference runs one forward per group of
  equal-length prefill chunks and then a separate decode forward
  (engine.py:257-261, 303-312); here every prefill chunk and every decode
  token of the tick go into one varlen batch (``begin_tick``), so a tick is
  one pass over the 36 layers and one sampling call;
* the prefix cache shares pool pages instead of copying (PagedPrefix,
  prefix_cache.py), and the pool makes room by evicting cold prefix entries
  when a tick would not fit;
* weights come from a local safetensors directory (no download) or are
  synthetic (random, for benchmarks and tests).

Tokenization needs a tokenizer (a local transformers tokenizer directory);
without one, requests carry ``prompt_tokens`` and responses stay token ids.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass, field
from queue import Queue
from typing import List, Optional, Union

import torch

from .constants import (
    COMPILE_MODES,
    DEFAULT_KV_CACHE_TOKENS,
    DEFAULT_KV_PAGE_SIZE,
    DEFAULT_PREFILL_CHUNK_SIZE,
    MAX_BATCH_SIZE,
)
from .model import Qwen3Config, Qwen3Model, init_synthetic_weights, load_local_weights
from .paged_cache import PagedCacheHandle, PagedKVCacheManager, PagedPrefix
from .prefix_cache import PrefixCache
from .sampler import Sampler
from .tick_graph import TickGraphRunner

DEFAULT_PREFIX_CACHE_MAX_TOKENS = 4096  # constants.py:27


@dataclass
class Request:
    """One prompt, its generated tokens and its progress (request.py:7-34)."""

    id: int = 0
    prompt: str = ""
    max_tokens: int = 100
    prompt_tokens: List[int] = field(default_factory=list)
    tokens: List[int] = field(default_factory=list)
    kv_cache: object = None
    paged_cache: Optional[PagedCacheHandle] = None
    is_completed: bool = False
    is_prefill: bool = True
    response: Optional[str] = None
    temperature: float = 0.0
    top_k: Optional[int] = None
    top_p: Optional[float] = None


class Scheduler:
    """Waiting queue plus the active batch (scheduler.py:8-28)."""

    def __init__(self, max_batch_size: int = MAX_BATCH_SIZE):
        self.pool: Queue = Queue()
        self.current_batch: List[Request] = []
        self.request_id = 0
        self.max_batch_size = max_batch_size

    def add(self, request: Request) -> None:
        self.pool.put(request)

    def tick(self) -> List[Request]:
        self.current_batch = [r for r in self.current_batch if not r.is_completed]
        while not self.pool.empty() and len(self.current_batch) < self.max_batch_size:
            self.current_batch.append(self.pool.get())
        return self.current_batch


@dataclass
class TickStats:
    """What the last tick ran: sequences, query tokens, prefill/decode split."""

    num_seqs: int = 0
    num_tokens: int = 0
    prefill_tokens: int = 0
    decode_tokens: int = 0


class Engine:
    """Loads (or synthesises) the model and runs scheduler ticks."""

    def __init__(
        self,
        model_dir: Optional[str] = None,
        compile: bool = False,
        compile_mode: str = "default",
        enable_prefix_cache: bool = False,
        prefix_cache_max_tokens: int = DEFAULT_PREFIX_CACHE_MAX_TOKENS,
        prefill_chunk_size: int = DEFAULT_PREFILL_CHUNK_SIZE,
        max_cache_tokens: int = DEFAULT_KV_CACHE_TOKENS,
        kv_page_size: int = DEFAULT_KV_PAGE_SIZE,
        *,
        config: Optional[Qwen3Config] = None,
        seed: int = 0,
        max_batch_size: int = MAX_BATCH_SIZE,
        tokenizer=None,
        stop_token_ids: Optional[set[int]] = None,
        device: str = "cuda",
    ):
        """Positional arguments follow the reference's Engine (engine.py:29-39).
        compile=True replays ticks from captured HIP graphs (tick_graph.py):
        decode ticks from their first occurrence, ticks with prompt chunks
        from the second occurrence of their shape on — except in
        "max-autotune-no-cudagraphs" mode, which by its name asks for no
        graphs; there is no torch.compile on this path."""
        if not torch.cuda.is_available():
            raise RuntimeError("the engine needs a HIP GPU")
        if compile_mode not in COMPILE_MODES:
            raise ValueError(
                f"unknown compile mode '{compile_mode}'. Valid options: {COMPILE_MODES}"
            )
        for name, value in (("prefill_chunk_size", prefill_chunk_size),
                            ("max_cache_tokens", max_cache_tokens),
                            ("max_batch_size", max_batch_size)):
            if isinstance(value, bool) or not isinstance(value, int) or value < 1:
                raise ValueError(f"{name} must be a positive integer")
        if (isinstance(kv_page_size, bool) or not isinstance(kv_page_size, int)
                or kv_page_size < 1 or kv_page_size & (kv_page_size - 1)):
            raise ValueError("kv_page_size must be a positive power of two")
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.prefill_chunk_size = prefill_chunk_size
        with torch.device(self.device):
            self.model = Qwen3Model(config)
        if model_dir is not None:
            load_local_weights(self.model, model_dir)
        else:
            init_synthetic_weights(self.model, seed)
        self.model.eval()
        self.model.initialize_rope(self.device)
        self.num_layers = self.model.num_layers
        self.max_position_embeddings = self.model.max_position_embeddings
        if tokenizer is None and model_dir is not None:
            tokenizer = _local_tokenizer(model_dir)
        self.tokenizer = tokenizer
        if stop_token_ids is None:
            stop_token_ids = _stop_token_ids(model_dir, tokenizer)
        self.scheduler = Scheduler(max_batch_size)
        # one trie level of the prefix index per KV page
        self.prefix_cache = (PrefixCache(prefix_cache_max_tokens, block_tokens=kv_page_size)
                             if enable_prefix_cache else None)
        self.sampler = Sampler(tokenizer, stop_token_ids,
                               torch.Generator(device=self.device).manual_seed(seed))
        self.paged_cache = PagedKVCacheManager(
            num_layers=self.num_layers, num_kv_heads=self.model.num_kv_groups,
            head_dim=self.model.head_dim, max_cache_tokens=max_cache_tokens,
            page_size=kv_page_size, max_requests=max_batch_size,
            dtype=self.model.embed_tokens.weight.dtype, device=self.device,
            num_q_heads=self.model.num_heads,
        )
        self.last_tick = TickStats()
        self.tick_graphs = (
            TickGraphRunner(self.model, self.paged_cache, self.max_position_embeddings)
            if compile and compile_mode != "max-autotune-no-cudagraphs" else None
        )

    # ------------------------------------------------------------ requests
    def add_request(self, request: Request) -> None:
        self._prepare_request(request)
        self.scheduler.add(request)

    def _prepare_request(self, request: Request) -> None:
        """Tokenize, check limits and attach a reusable prefix (engine.py:136-164)."""
        self.sampler.validate_parameters(request.temperature, request.top_k, request.top_p)
        if not request.prompt_tokens:
            if self.tokenizer is None:
                raise ValueError("no tokenizer: give the request's prompt_tokens")
            request.prompt_tokens = self.tokenizer.encode(request.prompt)
        self._validate_request_lengths(request)
        if request.kv_cache is not None and request.kv_cache.length > 0:
            return
        request.kv_cache = None
        if self.prefix_cache is None:
            return
        max_prefix_len = max(len(request.prompt_tokens) - 1, 0)
        match = self.prefix_cache.get(request.prompt_tokens, max_prefix_len=max_prefix_len)
        if match.cache is None or match.length == 0:
            return
        request.kv_cache = match.cache

    def _validate_request_lengths(self, request: Request) -> None:
        if request.max_tokens < 1:
            raise ValueError("max_tokens must be at least 1")
        if not request.prompt_tokens:
            raise ValueError("prompt must tokenize to at least one token")
        required = len(request.prompt_tokens) + request.max_tokens - 1
        if required > self.max_position_embeddings:
            raise ValueError(
                "request exceeds model context window: "
                f"prompt tokens ({len(request.prompt_tokens)}) + generated-token positions "
                f"({request.max_tokens - 1}) = {required}, "
                f"max supported positions = {self.max_position_embeddings}"
            )

    def clear_prefix_cache(self) -> None:
        if self.prefix_cache is not None:
            self.prefix_cache.clear()

    def release_request_cache(self, request: Request) -> None:
        """Return a request's pages and drop any prefix it still holds."""
        if request.paged_cache is not None:
            self.paged_cache.release(request.paged_cache)
            request.paged_cache = None
        if request.kv_cache is not None:
            request.kv_cache.reset()
            request.kv_cache = None

    def _store_prompt_prefix(self, request: Request) -> None:
        """Share the processed prompt's pages with the prefix cache
        (engine.py:188-198, without the gather and the clone)."""
        if self.prefix_cache is None or request.paged_cache is None:
            return
        if request.paged_cache.length < len(request.prompt_tokens):
            return
        shared = self.paged_cache.share(request.paged_cache, len(request.prompt_tokens))
        self.prefix_cache.put(request.prompt_tokens, shared)
        shared.reset()

    # ---------------------------------------------------------------- ticks
    def _begin_tick(self, handles, q_lens):
        """begin_tick, evicting cold prefix entries while the pool is full."""
        while True:
            try:
                return self.paged_cache.begin_tick(handles, q_lens)
            except MemoryError:
                if self.prefix_cache is None or not self.prefix_cache.evict_lru():
                    raise

    def _reserve_tick(self, handles, q_lens) -> None:
        """reserve_tick, evicting cold prefix entries while the pool is full."""
        while True:
            try:
                self.paged_cache.reserve_tick(handles, q_lens)
                return
            except MemoryError:
                if self.prefix_cache is None or not self.prefix_cache.evict_lru():
                    raise

    def _attach(self, request: Request) -> None:
        """Give a new request its pages: a shared prefix (no copy), an
        imported Cache, or none (engine.py:237-243)."""
        prefix = request.kv_cache
        while True:
            try:
                request.paged_cache = self.paged_cache.allocate_for_request(prefix)
                break
            except MemoryError:
                if self.prefix_cache is None or not self.prefix_cache.evict_lru():
                    raise
        if prefix is not None:
            prefix.reset()
        request.kv_cache = None

    def step(self, batch: List[Request]) -> None:
        """One forward pass: a prompt chunk for every request in prefill and
        one token for every request in decode, as a single varlen batch;
        then sampling for the requests whose prompt is done or that decode."""
        handles, q_lens, tokens, samplers = [], [], [], []
        for row, r in enumerate(batch):
            if r.is_prefill:
                if r.paged_cache is None:
                    self._attach(r)
                max_prefix_len = len(r.prompt_tokens) - 1
                pos = r.paged_cache.length
                if pos > max_prefix_len:
                    self.paged_cache.truncate(r.paged_cache, max_prefix_len)
                    pos = max_prefix_len
                end = min(pos + self.prefill_chunk_size, len(r.prompt_tokens))
                chunk = r.prompt_tokens[pos:end]
                if end == len(r.prompt_tokens):
                    samplers.append(row)
            else:
                chunk = [r.tokens[-1]]
                samplers.append(row)
            handles.append(r.paged_cache)
            q_lens.append(len(chunk))
            tokens.extend(chunk)
        logits = None
        if self.tick_graphs is not None:
            self._reserve_tick(handles, q_lens)
            logits = self.tick_graphs.run(handles, q_lens, tokens)
        if logits is None:
            paged = self._begin_tick(handles, q_lens)
            ids = torch.tensor(tokens, dtype=torch.long, device=self.device).unsqueeze(0)
            with torch.inference_mode():
                logits, _, _ = self.model(ids, paged_cache=paged)
        self.paged_cache.commit_tick(handles, q_lens)
        n_prefill = sum(q for q, r in zip(q_lens, batch) if r.is_prefill)
        self.last_tick = TickStats(len(batch), len(tokens), n_prefill, len(tokens) - n_prefill)
        if not samplers:
            return
        reqs = [batch[i] for i in samplers]
        rows = torch.tensor(samplers, dtype=torch.long, device=self.device)
        next_tokens = self.sampler.sample(logits[:, -1, :].index_select(0, rows), reqs)
        for r, tok in zip(reqs, next_tokens.flatten().tolist()):
            self.sampler.finalize(r, tok)
            if r.is_prefill:
                r.is_prefill = False
                self._store_prompt_prefix(r)

    def prefill_batch(self, requests: List[Request]) -> None:
        """One prompt chunk per request, sampling the requests whose prompt is
        done (engine.py:226-276). The reference runs one forward per group of
        equal-length chunks; here all chunks go into one varlen tick."""
        for r in requests:
            if not r.prompt_tokens:
                if self.tokenizer is None:
                    raise ValueError("no tokenizer: give the request's prompt_tokens")
                r.prompt_tokens = self.tokenizer.encode(r.prompt)
            if not r.prompt_tokens:
                raise ValueError("prompt must tokenize to at least one token")
            if not r.is_prefill:
                raise ValueError("prefill_batch needs requests whose prompt is not done")
        if requests:
            self.step(requests)

    def decode_batch(self, requests: List[Request]) -> None:
        """One token for every request from its latest token (engine.py:278-289)."""
        if any(r.is_prefill for r in requests):
            raise ValueError("decode_batch needs requests whose prompt is done")
        if requests:
            self.step(requests)

    def generate(self) -> bool:
        """One scheduler tick; False once no request is active (engine.py:291-314)."""
        previous = list(self.scheduler.current_batch)
        batch = self.scheduler.tick()
        active = {id(r) for r in batch}
        for r in previous:
            if r.is_completed and id(r) not in active:
                self.release_request_cache(r)
        if not batch:
            return False
        self.step(batch)
        return True

    def generate_text(
        self,
        prompts: Union[str, List[str], List[int], List[List[int]]],
        max_tokens: int = 100,
        temperature: float = 0.0,
        top_k: Optional[int] = None,
        top_p: Optional[float] = None,
    ):
        """Run prompts (text, or token-id lists) to completion (engine.py:316-348)."""
        if isinstance(prompts, str) or (prompts and isinstance(prompts[0], int)):
            prompts = [prompts]
        requests = []
        for prompt in prompts:
            req = Request(id=self.scheduler.request_id, max_tokens=max_tokens,
                          temperature=temperature, top_k=top_k, top_p=top_p)
            if isinstance(prompt, str):
                req.prompt = prompt
            else:
                req.prompt_tokens = list(prompt)
            self.scheduler.request_id += 1
            self.add_request(req)
            requests.append(req)
        while self.generate():
            pass
        return requests[0] if len(requests) == 1 else requests


def _stop_token_ids(model_dir: Optional[str], tokenizer) -> set[int]:
    """End-of-generation ids: the checkpoint's generation_config.json
    eos_token_id (an id or a list) and the tokenizer's eos id
    (engine.py:112-129)."""
    ids: set[int] = set()
    if model_dir is not None:
        path = os.path.join(model_dir, "generation_config.json")
        try:
            with open(path) as f:
                eos = json.load(f).get("eos_token_id")
            if isinstance(eos, int):
                ids.add(eos)
            elif eos is not None:
                ids.update(int(t) for t in eos)
        except (OSError, ValueError, TypeError):
            pass  # the tokenizer's id below still applies
    if tokenizer is not None and tokenizer.eos_token_id is not None:
        ids.add(int(tokenizer.eos_token_id))
    return ids


def _local_tokenizer(model_dir: str):
    """A transformers tokenizer from the checkpoint directory, if it has one."""
    if not any(os.path.exists(os.path.join(model_dir, f))
               for f in ("tokenizer.json", "tokenizer_config.json")):
        return None
    from transformers import AutoTokenizer

    return AutoTokenizer.from_pretrained(model_dir, use_fast=True, local_files_only=True)
