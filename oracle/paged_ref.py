"""CPU restatement of the reference's paged-attention path.

TEST INFRASTRUCTURE ONLY. This module is the checker: only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and
only to compute expected values or a reported CPU timing. The product path
(hayate-exp_amd/hayate_amd) never imports it.

bf16 tensors are numpy uint16 bit patterns; float work is numpy (float64 by
default for attention, so the oracle is more accurate than any bf16 kernel).
Each function cites the reference file:line it restates (paths relative to
the reference repository root).

Pinning (tests/test_oracle.py): every function here is checked against a
torch library routine, the reference's own torch op chain, a brute-force
loop or a closed form (see the test module docstring); none is "parity
unpinned". The reference holds no golden vectors or fixtures for this path,
so there is no tests/golden/ directory.
"""

from __future__ import annotations

import numpy as np
import torch

# ---------------------------------------------------------------------------
# bf16 bit conversions
# ---------------------------------------------------------------------------


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns to float32."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (the rounding of torch's
    bf16 conversion that the reference's `.to(bfloat16)` casts use, e.g.
    rope.py:47). NaN maps to the quiet NaN 0x7fc0; torch's CPU and GPU
    conversions emit other NaN payloads, so NaNs are compared as NaNs."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded = np.where(nan, np.uint16(0x7FC0), rounded)
    return rounded.astype(np.uint16)


def torch_bf16_to_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def bits_to_torch_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(
        torch.bfloat16
    )


# ---------------------------------------------------------------------------
# Page-table index math and bit copies
# ---------------------------------------------------------------------------


def physical_positions(pages, length: int, page_size: int) -> np.ndarray:
    """Physical token of logical positions 0..length-1 of one request:
    pages[t // P] * P + t % P (paged_cache.py:306-315)."""
    if length == 0:
        return np.zeros(0, dtype=np.int64)
    t = np.arange(length, dtype=np.int64)
    pages = np.asarray(pages, dtype=np.int64)
    return pages[t // page_size] * page_size + t % page_size


def append_positions(page_lists, cache_lens, q_lens, page_size: int) -> np.ndarray:
    """Physical token for every new token, packed in sequence order:
    positions cache_len_b + i, i < q_len_b (paged_cache.py:49-56, written for
    per-sequence query lengths)."""
    out = []
    for pages, c, q in zip(page_lists, cache_lens, q_lens):
        t = np.arange(c, c + q, dtype=np.int64)
        pages = np.asarray(pages, dtype=np.int64)
        out.append(pages[t // page_size] * page_size + t % page_size)
    return np.concatenate(out) if out else np.zeros(0, dtype=np.int64)


def kv_append(pool_k, pool_v, k_new, v_new, page_lists, cache_lens, q_lens, page_size):
    """pool[h, phys, :] = new[tok, h, :] for one layer, in place
    (paged_cache.py:44-60). pool_*: uint16 (Hkv, capacity, D); new: uint16
    packed (N, Hkv, D)."""
    pos = append_positions(page_lists, cache_lens, q_lens, page_size)
    pool_k[:, pos, :] = np.transpose(k_new, (1, 0, 2))
    pool_v[:, pos, :] = np.transpose(v_new, (1, 0, 2))


def page_gather(pool, pages, length: int, page_size: int) -> np.ndarray:
    """Compact copy of the first `length` positions of every layer/head:
    pool (L, Hkv, capacity, D) -> (L, Hkv, length, D)
    (snapshot, paged_cache.py:180-190)."""
    return pool[:, :, physical_positions(pages, length, page_size), :].copy()


def page_scatter(pool, pages, src, page_size: int) -> None:
    """Inverse of page_gather, in place (import_cache, paged_cache.py:153-166)."""
    length = src.shape[2]
    pool[:, :, physical_positions(pages, length, page_size), :] = src


# ---------------------------------------------------------------------------
# q/k RMSNorm and RoPE
# ---------------------------------------------------------------------------


def rms_norm(x_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    """nn.RMSNorm(head_dim, eps) on bf16 rows (attention.py:34-35, 62-63):
    fp32 upcast, mean of squares, rsqrt(mean + eps) as an IEEE 1/sqrt,
    multiply by it, multiply by the weight, one rounding to bf16
    (torch/_decomp/decompositions.py `_fused_rms_norm`).

    The mean is the correctly rounded one: squares of bf16 values are exact
    in float32 and their sum is exact in float64, so summing in float64 and
    rounding once fixes the result independently of summation order (torch's
    CPU kernel gives the same bits; the test checks it)."""
    x = bf16_to_f32(x_bits)
    w = bf16_to_f32(w_bits)
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    ms = ss.astype(np.float32) / np.float32(x.shape[-1])
    r = (np.float32(1.0) / np.sqrt(ms + np.float32(eps))).astype(np.float32)
    y = (x * r).astype(np.float32) * w
    return f32_to_bf16(y.astype(np.float32))


def rope_tables(head_dim: int, theta: float, context_length: int):
    """fp32 cos/sin tables (rope.py:4-28), built with the same torch ops so
    that entries are bit-identical to the tables the engine builds."""
    exps = torch.arange(0, head_dim, 2, dtype=torch.float32)[: head_dim // 2].float()
    inv_freq = 1.0 / (theta ** (exps / head_dim))
    pos = torch.arange(context_length, dtype=torch.float32)
    ang = pos.unsqueeze(1) * inv_freq.unsqueeze(0)
    ang = torch.cat([ang, ang], dim=1)
    return torch.cos(ang).numpy(), torch.sin(ang).numpy()


def apply_rope(x_bits: np.ndarray, cos: np.ndarray, sin: np.ndarray, positions) -> np.ndarray:
    """NeoX rotate-half on bf16 rows (rope.py:31-47): with x1, x2 the halves,
    y = bf16(fl(x * cos[pos]) + fl(cat(-x2, x1) * sin[pos])) in fp32.
    x_bits (..., H, D) with positions broadcast over the head axis."""
    x = bf16_to_f32(x_bits)
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    c = cos[np.asarray(positions)][..., None, :]
    s = sin[np.asarray(positions)][..., None, :]
    a = (x * c).astype(np.float32)
    b = (rot * s).astype(np.float32)
    return f32_to_bf16((a + b).astype(np.float32))


def qknorm_rope_append(q, k, v, q_w, k_w, eps, cos, sin, pool_k, pool_v, page_lists,
                       cache_lens, q_lens, page_size, k_eps=None):
    """attention.py:62-75 on packed tokens: q/k RMSNorm, RoPE at positions
    cache_len + i, append of k and v. Returns the rotated q (bf16 bits).
    `eps` is q_norm's epsilon, `k_eps` k_norm's (default: the same)."""
    positions = np.concatenate(
        [np.arange(c, c + n, dtype=np.int64) for c, n in zip(cache_lens, q_lens)]
    )
    qn = rms_norm(q, q_w, eps) if q_w is not None else q
    kn = rms_norm(k, k_w, eps if k_eps is None else k_eps) if k_w is not None else k
    if cos is not None:
        qn = apply_rope(qn, cos, sin, positions)
        kn = apply_rope(kn, cos, sin, positions)
    kv_append(pool_k, pool_v, kn, v, page_lists, cache_lens, q_lens, page_size)
    return qn


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------


def paged_attention(q_bits, pool_k, pool_v, page_lists, cache_lens, q_lens, page_size,
                    scale=None, dtype=np.float64) -> np.ndarray:
    """Causal GQA attention over pages (paged_cache.py:62-71, mask 266-271):
    query i of sequence b (logical position c_b + i) attends to logical keys
    k <= c_b + i gathered through its page list; query head h reads kv head
    h // (Hq / Hkv) (enable_gqa). q_bits packed (N, Hq, D) bf16 bits; pools
    (Hkv, capacity, D) bf16 bits. Returns (N, Hq, D) in `dtype`."""
    n_tok, hq, d = q_bits.shape
    hkv = pool_k.shape[0]
    group = hq // hkv
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    q = bf16_to_f32(q_bits).astype(dtype)
    out = np.zeros((n_tok, hq, d), dtype=dtype)
    start = 0
    for pages, c, ql in zip(page_lists, cache_lens, q_lens):
        kv = c + ql
        pos = physical_positions(pages, kv, page_size)
        qi = np.arange(ql)
        allowed = np.arange(kv)[None, :] <= (c + qi)[:, None]  # (ql, kv)
        for g in range(hkv):
            kg = bf16_to_f32(pool_k[g, pos, :]).astype(dtype)
            vg = bf16_to_f32(pool_v[g, pos, :]).astype(dtype)
            qg = q[start : start + ql, g * group : (g + 1) * group, :].reshape(ql * group, d)
            s = (qg @ kg.T).reshape(ql, group, kv) * dtype(scale)
            s = np.where(allowed[:, None, :], s, -np.inf)
            s = s - s.max(axis=-1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=-1, keepdims=True)
            o = p.reshape(ql * group, kv) @ vg
            out[start : start + ql, g * group : (g + 1) * group, :] = o.reshape(ql, group, d)
        start += ql
    return out


def compare(actual_bits: np.ndarray, expected: np.ndarray) -> dict:
    """Error statistics of bf16 output bits against a float reference."""
    a = bf16_to_f32(actual_bits).astype(np.float64)
    e = np.asarray(expected, dtype=np.float64)
    diff = np.abs(a - e)
    rms_e = float(np.sqrt(np.mean(e * e))) if e.size else 0.0
    return {
        "max_abs": float(diff.max()) if diff.size else 0.0,
        "mean_abs": float(diff.mean()) if diff.size else 0.0,
        "rel_rms": float(np.sqrt(np.mean(diff * diff)) / rms_e) if rms_e > 0 else 0.0,
        "finite": bool(np.isfinite(a).all()),
    }


# Tolerances of the attention output (bf16 result vs this oracle).
MAX_ABS_TOL = 2e-2
MEAN_ABS_TOL = 2e-3
REL_RMS_TOL = 1e-2
