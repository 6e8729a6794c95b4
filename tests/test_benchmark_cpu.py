"""Host helpers of hayate_amd.benchmark, on the CPU: the checks the
reference's tests/test_benchmark.py makes of its benchmark CLI (positive
sizes, exact-length repeatable prompts, the median of paired samples),
applied to this engine's counterpart."""

import argparse
from types import SimpleNamespace

import pytest
import torch

from hayate_amd import benchmark


def test_positive_sizes():
    assert benchmark._positive("4") == 4
    with pytest.raises(argparse.ArgumentTypeError):
        benchmark._positive("0")


def _engine(tokenizer=None, vocab=100):
    model = SimpleNamespace(embed_tokens=SimpleNamespace(weight=torch.empty(vocab, 1)))
    return SimpleNamespace(tokenizer=tokenizer, model=model)


def test_prompts_have_the_exact_length_and_rotate_per_request():
    class Tokenizer:
        def encode(self, text, add_special_tokens=False):
            return [1, 2, 3]

    eng = _engine(Tokenizer())
    assert benchmark.prompt_tokens(eng, 5, 1) == [2, 3, 1, 2, 3]
    assert benchmark.prompt_tokens(eng, 2, 0) == [1, 2]
    assert benchmark.prompt_tokens(eng, 7, 3) == [1, 2, 3, 1, 2, 3, 1]  # rotation wraps


def test_prompts_without_a_tokenizer_are_seeded_ids_in_the_vocabulary():
    eng = _engine(vocab=50)
    a = benchmark.prompt_tokens(eng, 300, 0)
    assert len(a) == 300 and all(0 <= t < 50 for t in a)
    assert a == benchmark.prompt_tokens(eng, 300, 0)  # repeatable
    b = benchmark.prompt_tokens(eng, 300, 1)
    assert b[:60] == a[1:61]  # request i is the same sequence rotated by i


def test_median_of_paired_samples():
    assert benchmark._median([(1.0, 4.0), (3.0, 2.0)]) == (2.0, 3.0)
    assert benchmark._median([(5.0, 1.0)]) == (5.0, 1.0)
