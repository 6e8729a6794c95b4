"""Token sampling on the GPU for a whole batch at once.

Semantics of the reference's hayate/engine/sampler.py:
* ``validate_parameters`` (:15-37): same checks and messages;
* per row (``_sample_row``, :39-65): temperature 0 is argmax; otherwise the
  scores are logits / temperature, top-k keeps every score >= the k-th
  largest, top-p keeps the shortest prefix of the descending-sorted
  distribution whose mass exceeds p together with the token that crosses
  it, and one token is drawn from the softmax of what is left;
* ``finalize`` (:87-93): append, stop on a stop token or the length limit.

The reference loops over rows in Python, one small kernel chain per row
(:67-85). Here every row of the batch goes through one sort and a handful of
batched ops, with per-row temperature / k / p as tensors, so a tick costs
the same few launches whatever the batch size.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch


def validate_parameters(temperature, top_k, top_p) -> None:
    """Reject invalid temperature, top-k or nucleus settings (sampler.py:15-37)."""
    if (
        isinstance(temperature, bool)
        or not isinstance(temperature, (int, float))
        or not math.isfinite(temperature)
        or temperature < 0
    ):
        raise ValueError("temperature must be a finite number greater than or equal to 0")
    if top_k is not None and (isinstance(top_k, bool) or not isinstance(top_k, int) or top_k < 1):
        raise ValueError("top_k must be a positive integer or None")
    if top_p is not None and (
        isinstance(top_p, bool)
        or not isinstance(top_p, (int, float))
        or not math.isfinite(top_p)
        or not 0 < top_p <= 1
    ):
        raise ValueError("top_p must be greater than 0 and at most 1, or None")


def sample_batch(logits: torch.Tensor, temperature: Sequence[float],
                 top_k: Sequence[Optional[int]], top_p: Sequence[Optional[float]],
                 generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """One token id per row of logits (n, vocab) -> int64 (n, 1)."""
    n, vocab = logits.shape
    dev = logits.device
    greedy_rows = [i for i, t in enumerate(temperature) if t == 0]
    out = torch.argmax(logits, dim=-1, keepdim=True)
    if len(greedy_rows) == n:
        return out
    rows = [i for i in range(n) if temperature[i] != 0]
    idx = torch.tensor(rows, device=dev, dtype=torch.long)
    temp = torch.tensor([float(temperature[i]) for i in rows], device=dev).unsqueeze(1)
    scores = logits.index_select(0, idx).float() / temp
    sorted_scores, sorted_idx = torch.sort(scores, dim=-1, descending=True)
    # top-k: keep scores >= the k-th largest (ties kept, as masked_fill(< threshold))
    ks = [min(top_k[i], vocab) if top_k[i] is not None else vocab for i in rows]
    kth = sorted_scores.gather(1, torch.tensor(ks, device=dev).unsqueeze(1) - 1)
    keep = scores >= kth
    sorted_scores = sorted_scores.masked_fill(sorted_scores < kth, -torch.inf)
    # top-p over the top-k survivors: remove a token once the mass before it
    # exceeds p (the crossing token stays, so the set is never empty)
    ps = torch.tensor([float(top_p[i]) if top_p[i] is not None else 1.0 for i in rows],
                      device=dev).unsqueeze(1)
    use_p = ps < 1
    probs = torch.softmax(sorted_scores, dim=-1)
    remove_sorted = torch.cumsum(probs, dim=-1) > ps
    remove_sorted = torch.cat(
        [torch.zeros_like(remove_sorted[:, :1]), remove_sorted[:, :-1]], dim=1) & use_p
    remove = torch.zeros_like(remove_sorted).scatter(1, sorted_idx, remove_sorted)
    scores = scores.masked_fill(~keep | remove, -torch.inf)
    drawn = torch.multinomial(torch.softmax(scores, dim=-1), 1, generator=generator)
    out.index_copy_(0, idx, drawn)
    return out


class Sampler:
    """Samples the next token of each request (sampler.py:8-93)."""

    def __init__(self, tokenizer=None, stop_token_ids: Optional[set[int]] = None,
                 generator: Optional[torch.Generator] = None):
        self.tokenizer = tokenizer
        self.stop_token_ids = set(stop_token_ids or ())
        self.generator = generator

    validate_parameters = staticmethod(validate_parameters)

    def sample(self, logits: torch.Tensor, requests=None) -> torch.Tensor:
        if requests is None:
            return torch.argmax(logits, dim=-1, keepdim=True)
        if logits.ndim != 2 or logits.shape[0] != len(requests):
            raise ValueError("sampling logits must have one vocabulary row per request")
        for r in requests:
            validate_parameters(r.temperature, r.top_k, r.top_p)
        return sample_batch(logits, [r.temperature for r in requests],
                            [r.top_k for r in requests], [r.top_p for r in requests],
                            self.generator)

    def finalize(self, request, tok: int) -> None:
        request.tokens.append(tok)
        if tok in self.stop_token_ids or len(request.tokens) >= request.max_tokens:
            request.is_completed = True
            if self.tokenizer is not None:
                request.response = self.tokenizer.decode(request.tokens,
                                                         skip_special_tokens=True)
