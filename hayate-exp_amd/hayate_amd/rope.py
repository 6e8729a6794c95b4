"""Rotary-embedding tables (the reference's hayate/model/rope.py:4-28).

The HIP kernels never evaluate sin/cos: they read these fp32 tables, built by
torch on the model's device exactly as the reference builds them
(qwen.py:60-67), so a rotated value depends only on the table entries.
"""

from __future__ import annotations

import torch


def compute_rope_params(
    head_dim: int,
    theta_base: int = 10_000,
    context_length: int = 4096,
    dtype: torch.dtype = torch.float32,
    device: torch.device | str | None = None,
):
    """Return fp32 (context_length, head_dim) cosine and sine tables.

    Feature pair j rotates at inv_freq[j] = theta_base ** (-2j / head_dim);
    both halves of the head share the angles (NeoX rotate-half layout).
    """
    if head_dim % 2:
        raise ValueError("head_dim must be even")
    exponents = torch.arange(0, head_dim, 2, dtype=dtype, device=device)
    inv_freq = 1.0 / (theta_base ** (exponents[: head_dim // 2].float() / head_dim))
    positions = torch.arange(context_length, dtype=dtype, device=device)
    angles = positions.unsqueeze(1) * inv_freq.unsqueeze(0)
    angles = torch.cat([angles, angles], dim=1)
    return torch.cos(angles), torch.sin(angles)
