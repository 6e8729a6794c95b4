"""The CPU baseline (oracle/flex_ref.py: the reference's paged write +
compiled FlexAttention over the physical-page BlockMask) computes the same
attention as the oracle: a small uniform batch with histories on scattered
pages, one prefill-shaped query block, on the CPU (one Inductor compile)."""

import math

import numpy as np
import torch

from oracle import flex_ref as F
from oracle import paged_ref as R


def test_flex_baseline_matches_the_oracle():
    g = torch.Generator().manual_seed(8)
    P, cap, T = 128, 4096, 3
    cache_lens = [130, 300]
    perm = torch.randperm(cap // P, generator=g).tolist()
    pages, cur = [], 0
    for c in cache_lens:
        n = math.ceil((c + T) / P)
        pages.append(perm[cur : cur + n])
        cur += n
    kp = torch.randn(1, 8, cap, 128, generator=g).to(torch.bfloat16)
    vp = torch.randn(1, 8, cap, 128, generator=g).to(torch.bfloat16)
    q = torch.randn(2, 32, T, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(2, 8, T, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 8, T, 128, generator=g).to(torch.bfloat16)
    pk, pv = R.torch_bf16_to_bits(kp[0]).copy(), R.torch_bf16_to_bits(vp[0]).copy()
    batch = F.FlexPagedBatch(pages, cache_lens, T, P, cap)
    batch.write_layer(kp, vp, k, v)
    out = batch.attend_layer(q, kp, vp)
    R.kv_append(pk, pv, R.torch_bf16_to_bits(k.transpose(1, 2).reshape(2 * T, 8, 128)),
                R.torch_bf16_to_bits(v.transpose(1, 2).reshape(2 * T, 8, 128)), pages,
                cache_lens, [T, T], P)
    assert np.array_equal(R.torch_bf16_to_bits(kp[0]), pk)
    expect = R.paged_attention(R.torch_bf16_to_bits(q.transpose(1, 2).reshape(2 * T, 32, 128)),
                               pk, pv, pages, cache_lens, [T, T], P)
    stats = R.compare(R.torch_bf16_to_bits(out.transpose(1, 2).reshape(2 * T, 32, 128)), expect)
    assert stats["finite"] and stats["max_abs"] <= R.MAX_ABS_TOL, stats
    assert stats["rel_rms"] <= R.REL_RMS_TOL, stats
