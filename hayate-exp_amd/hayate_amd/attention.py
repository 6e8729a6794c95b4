"""Grouped-query attention module for the paged path.

Same constructor, parameters and forward signature as the reference's
hayate/model/attention.py:17-122. In paged mode (the only mode Engine uses,
engine.py:218-223):

* the three projections (attention.py:58-60) run as one GEMM against the
  concatenated q/k/v weight, and q, k and v are strided views of its output
  that the fused append kernel reads in place (no split copies);
* q/k RMSNorm, RoPE and the paged K/V append (attention.py:62-75) are one
  HIP launch, and paged attention another (a decode tick does both in one
  launch plus the merge);
* the kernels write the context as (B, T, Hq, D), so the reshape before
  o_proj (attention.py:118-120) is a view.

The non-paged branch (contiguous history / varlen flash, attention.py:78-117)
is not part of this library and raises.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F


class GroupedQueryAttention(nn.Module):
    def __init__(self, d_in, num_heads, num_kv_groups, head_dim, dtype=None):
        super().__init__()
        if num_heads % num_kv_groups:
            raise ValueError("num_heads must be divisible by num_kv_groups")
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.num_kv_groups = num_kv_groups
        self.q_proj = nn.Linear(d_in, num_heads * head_dim, bias=False, dtype=dtype)
        self.k_proj = nn.Linear(d_in, num_kv_groups * head_dim, bias=False, dtype=dtype)
        self.v_proj = nn.Linear(d_in, num_kv_groups * head_dim, bias=False, dtype=dtype)
        self.o_proj = nn.Linear(num_heads * head_dim, d_in, bias=False, dtype=dtype)
        self.q_norm = nn.RMSNorm(head_dim, eps=1e-6, dtype=dtype)
        self.k_norm = nn.RMSNorm(head_dim, eps=1e-6, dtype=dtype)
        self._qkv_key = None
        self._qkv_weight = None

    def fused_qkv_weight(self) -> torch.Tensor:
        """cat(q_proj.weight, k_proj.weight, v_proj.weight) along the output
        dim, rebuilt whenever one of them is replaced or modified in place
        (checkpoint loading copies into the parameters)."""
        ws = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight)
        key = tuple((w.data_ptr(), w._version, w.device, w.dtype) for w in ws)
        if key != self._qkv_key:
            with torch.no_grad():
                self._qkv_weight = torch.cat([w.detach() for w in ws], dim=0)
            self._qkv_key = key
        return self._qkv_weight

    def project_qkv(self, x):
        """x (B, T, d_in) -> q (B, T, Hq, D), k, v (B, T, Hkv, D): strided views
        of one GEMM output (row stride (Hq + 2 Hkv) * D)."""
        B, T, _ = x.shape
        hq = self.num_heads * self.head_dim
        hkv = self.num_kv_groups * self.head_dim
        y = F.linear(x, self.fused_qkv_weight())
        q = y[..., :hq].view(B, T, self.num_heads, self.head_dim)
        k = y[..., hq : hq + hkv].view(B, T, self.num_kv_groups, self.head_dim)
        v = y[..., hq + hkv :].view(B, T, self.num_kv_groups, self.head_dim)
        return q, k, v

    def forward(
        self,
        x,
        cos,
        sin,
        position_ids,
        prev_k,
        prev_v,
        varlen_metadata=None,
        paged_cache=None,
        layer_idx=None,
    ):
        """x (B, T, d_in) -> (o_proj(context), None, None).

        Positions are the batch's cache_lens + token index, which is what the
        reference's position_ids hold in paged mode (qwen.py:89-109).
        """
        if paged_cache is None:
            raise NotImplementedError(
                "only the paged attention path is provided (pass paged_cache)"
            )
        B, T, _ = x.shape
        q, k, v = self.project_qkv(x)
        q_norm_w = self.q_norm.weight
        k_norm_w = self.k_norm.weight
        eps = self.q_norm.eps if self.q_norm.eps is not None else torch.finfo(torch.float32).eps
        if paged_cache.varlen:
            # Varlen ticks carry packed tokens: x is (1, N, d_in).
            if B != 1:
                raise ValueError("a varlen tick expects x of shape (1, tokens, d_in)")
            if all(ql == 1 for ql in paged_cache.q_lens):
                # a decode tick: norm, rope, append and attention in one launch
                _, context = paged_cache.decode_layer(
                    layer_idx, q[0], k[0], v[0], q_norm_w, k_norm_w, eps, cos, sin
                )
            else:
                q_rot = paged_cache.norm_rope_write_layer(
                    layer_idx, q[0], k[0], v[0], q_norm_w, k_norm_w, eps, cos, sin
                )
                context = paged_cache.attend_layer(q_rot, layer_idx)
            context = context.unsqueeze(0)
        elif T == 1:
            _, context = paged_cache.decode_layer(
                layer_idx, q, k, v, q_norm_w, k_norm_w, eps, cos, sin
            )
            context = context.transpose(1, 2)
        else:
            q_rot = paged_cache.norm_rope_write_layer(
                layer_idx, q, k, v, q_norm_w, k_norm_w, eps, cos, sin
            )
            context = paged_cache.attend_layer(q_rot.transpose(1, 2), layer_idx).transpose(1, 2)
        context = context.reshape(B, T, self.num_heads * self.head_dim)
        return self.o_proj(context), None, None
