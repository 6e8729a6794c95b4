"""Batched sampler (hayate_amd/sampler.py) against the reference's per-row
semantics (hayate/engine/sampler.py:15-93), on the CPU, by closed-form
cases: greedy is argmax; top-k keeps exactly the k largest scores (ties at
the k-th kept); top-p keeps the shortest descending prefix whose mass
exceeds p plus the crossing token; temperature scales the scores; rows with
different settings in one batch do not interact."""

import math
from types import SimpleNamespace

import pytest
import torch

from hayate_amd.sampler import Sampler, sample_batch, validate_parameters


def draws(logits, t, k, p, n=4000, seed=0):
    """Token frequencies of n draws from one row."""
    g = torch.Generator().manual_seed(seed)
    rows = logits.unsqueeze(0).expand(n, -1).contiguous()
    out = sample_batch(rows, [t] * n, [k] * n, [p] * n, g).flatten()
    return torch.bincount(out, minlength=logits.numel()).float() / n


def test_greedy_is_argmax_per_row():
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(6, 50, generator=g)
    out = sample_batch(logits, [0.0] * 6, [None] * 6, [None] * 6)
    assert torch.equal(out.flatten(), logits.argmax(dim=-1))
    assert out.shape == (6, 1) and out.dtype == torch.long


def test_top_k_keeps_exactly_the_k_largest():
    logits = torch.tensor([0.0, 3.0, 1.0, 2.9, -1.0, 2.8])
    f = draws(logits, 1.0, 2, None)
    assert set(torch.nonzero(f).flatten().tolist()) == {1, 3}
    # relative frequency follows exp of the kept scores
    assert f[1] / f[3] == pytest.approx(math.exp(0.1), rel=0.15)
    # top_k = 1 is greedy whatever the temperature
    assert torch.nonzero(draws(logits, 5.0, 1, None)).flatten().tolist() == [1]


def test_top_k_keeps_ties_at_the_threshold():
    logits = torch.tensor([1.0, 2.0, 2.0, 0.0])
    f = draws(logits, 1.0, 1, None)  # threshold 2.0: both tied tokens stay
    assert set(torch.nonzero(f).flatten().tolist()) == {1, 2}


def test_top_p_keeps_the_crossing_token():
    probs = torch.tensor([0.5, 0.3, 0.2])
    logits = probs.log()
    # mass before token 1 is 0.5 <= 0.6 and token 1 crosses: {0, 1}
    assert set(torch.nonzero(draws(logits, 1.0, None, 0.6)).flatten().tolist()) == {0, 1}
    # p = 0.5: cumsum > 0.5 first at token 1, which is kept: {0, 1}
    assert set(torch.nonzero(draws(logits, 1.0, None, 0.5)).flatten().tolist()) == {0, 1}
    # p = 0.4: token 0 alone already exceeds p
    assert torch.nonzero(draws(logits, 1.0, None, 0.4)).flatten().tolist() == [0]
    # p = 1 keeps everything, in proportion
    f = draws(logits, 1.0, None, 1.0, n=20000)
    assert f.tolist() == pytest.approx(probs.tolist(), abs=0.02)


def test_top_k_then_top_p_and_temperature():
    logits = torch.tensor([2.0, 1.0, 0.5, 0.0, -3.0])
    # top-k 3 leaves tokens 0-2; at temperature 2 their weights are
    # exp(1), exp(0.5), exp(0.25); top-p 0.7 then keeps tokens 0 and 1
    w = torch.tensor([1.0, 0.5, 0.25]).exp()
    w = w / w.sum()
    assert w[0] < 0.7 < w[0] + w[1]
    f = draws(logits, 2.0, 3, 0.7, n=20000)
    assert set(torch.nonzero(f).flatten().tolist()) == {0, 1}
    assert (f[0] / f[1]).item() == pytest.approx(math.exp(0.5), rel=0.1)


def test_mixed_rows_in_one_batch():
    logits = torch.tensor([[0.0, 1.0, 5.0], [4.0, 0.0, 0.0], [0.0, 9.0, 0.0]])
    g = torch.Generator().manual_seed(3)
    out = sample_batch(logits, [0.0, 1.0, 0.7], [None, 1, None], [None, None, 0.5], g)
    assert out.flatten().tolist() == [2, 0, 1]


def test_validation_and_finalize():
    validate_parameters(0.0, None, None)
    for bad in ((-1.0, None, None), (float("nan"), None, None), (True, None, None),
                (1.0, 0, None), (1.0, 2.5, None), (1.0, None, 0.0), (1.0, None, 1.5)):
        with pytest.raises(ValueError):
            validate_parameters(*bad)
    s = Sampler(stop_token_ids={7})
    r = SimpleNamespace(tokens=[], max_tokens=3, is_completed=False, response=None)
    s.finalize(r, 1)
    assert not r.is_completed
    s.finalize(r, 7)
    assert r.is_completed and r.tokens == [1, 7]
    with pytest.raises(ValueError):
        s.sample(torch.zeros(2, 4), [SimpleNamespace(temperature=0.0, top_k=None, top_p=None)])
