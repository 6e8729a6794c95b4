"""Helpers shared by the GPU parity tests: run one attention step of a
workload through the HIP path and the same step through the oracle."""

from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import paged_ref as R

EPS = 1e-6


def bits(t: torch.Tensor) -> np.ndarray:
    return R.torch_bf16_to_bits(t)


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def layer_bits(manager, layer=0):
    return bits(manager.k_cache[layer, 0]), bits(manager.v_cache[layer, 0])


def gpu_step(w, layer=0):
    """Fused norm + rope + append, then attention; returns (q_rot, out)."""
    batch = w.begin()
    q_rot = batch.norm_rope_write_layer(layer, w.q, w.k, w.v, w.q_norm_w, w.k_norm_w,
                                        EPS, w.cos, w.sin)
    out = batch.attend_layer(q_rot, layer)
    torch.cuda.synchronize()
    return q_rot, out


def oracle_step(w, pre_k, pre_v):
    """The same step on the CPU; returns (pool_k, pool_v, q_rot bits, out)."""
    pk, pv = pre_k.copy(), pre_v.copy()
    cos = w.cos.cpu().numpy()
    sin = w.sin.cpu().numpy()
    q_rot = R.qknorm_rope_append(bits(w.q), bits(w.k), bits(w.v), bits(w.q_norm_w),
                                 bits(w.k_norm_w), EPS, cos, sin, pk, pv, w.page_lists,
                                 w.cache_lens, w.q_lens, w.manager.page_size)
    out = R.paged_attention(q_rot, pk, pv, w.page_lists, w.cache_lens, w.q_lens,
                            w.manager.page_size)
    return pk, pv, q_rot, out


def assert_attention_close(actual_bits, expected, what=""):
    stats = R.compare(actual_bits, expected)
    say(f"  {what} max_abs={stats['max_abs']:.3e} mean_abs={stats['mean_abs']:.3e} "
        f"rel_rms={stats['rel_rms']:.3e}")
    assert stats["finite"], what
    assert stats["max_abs"] <= R.MAX_ABS_TOL, (what, stats)
    assert stats["mean_abs"] <= R.MEAN_ABS_TOL, (what, stats)
    assert stats["rel_rms"] <= R.REL_RMS_TOL, (what, stats)
    return stats
