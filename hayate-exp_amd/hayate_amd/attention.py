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


# Number of fused q/k/v weight buffers built so far (any module).
qkv_rebuilds = 0


def _views_of(f: torch.Tensor, ws) -> bool:
    """True when `ws` are consecutive row blocks of `f`, in order."""
    row = 0
    for w in ws:
        n = w.shape[0]
        if (w.device != f.device or w.dtype != f.dtype or w.shape[1:] != f.shape[1:]
                or w.stride() != f.stride() or w.data_ptr() != f[row : row + n].data_ptr()):
            return False
        row += n
    return row == f.shape[0]


def _norm_eps(norm: nn.RMSNorm, dtype: torch.dtype) -> float:
    """The epsilon nn.RMSNorm applies to inputs of `dtype`."""
    return float(norm.eps) if norm.eps is not None else float(torch.finfo(dtype).eps)


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
        self._qkv_weight = None

    def fused_qkv_weight(self) -> torch.Tensor:
        """The concatenated [W_q; W_k; W_v] (rows along the output dim), held
        once: q_proj.weight, k_proj.weight and v_proj.weight are views of
        it, so checkpoint loads and in-place updates of the parameters write
        straight into the fused buffer and no second copy exists. The
        buffer is (re)built, and the three parameters re-pointed into it,
        the first time and whenever a parameter was replaced rather than
        updated in place (module.to(), assignment); each rebuild advances
        `qkv_rebuilds`, so holders of its address (captured graphs) can
        tell."""
        global qkv_rebuilds
        lins = (self.q_proj, self.k_proj, self.v_proj)
        f = self._qkv_weight
        if f is not None and _views_of(f, [lin.weight for lin in lins]):
            return f
        # a normal tensor even when first called under inference_mode, so the
        # parameters stay trainable and updatable in place
        with torch.inference_mode(False), torch.no_grad():
            f = torch.cat([lin.weight.detach() for lin in lins], dim=0)
        row = 0
        for lin in lins:
            n = lin.weight.shape[0]
            lin.weight = nn.Parameter(f[row : row + n], requires_grad=lin.weight.requires_grad)
            row += n
        self._qkv_weight = f
        qkv_rebuilds += 1
        return f

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
        # each norm keeps its own eps; None means the input dtype's epsilon,
        # as nn.RMSNorm resolves it
        eps = _norm_eps(self.q_norm, q.dtype)
        k_eps = _norm_eps(self.k_norm, k.dtype)
        if paged_cache.varlen:
            # Varlen ticks carry packed tokens: x is (1, N, d_in).
            if B != 1:
                raise ValueError("a varlen tick expects x of shape (1, tokens, d_in)")
            if all(ql == 1 for ql in paged_cache.q_lens):
                # a decode tick: norm, rope, append and attention in one launch
                _, context = paged_cache.decode_layer(
                    layer_idx, q[0], k[0], v[0], q_norm_w, k_norm_w, eps, cos, sin,
                    k_eps=k_eps,
                )
            else:
                q_rot = paged_cache.norm_rope_write_layer(
                    layer_idx, q[0], k[0], v[0], q_norm_w, k_norm_w, eps, cos, sin,
                    k_eps=k_eps,
                )
                context = paged_cache.attend_layer(q_rot, layer_idx)
            context = context.unsqueeze(0)
        elif T == 1:
            _, context = paged_cache.decode_layer(
                layer_idx, q, k, v, q_norm_w, k_norm_w, eps, cos, sin, k_eps=k_eps
            )
            context = context.transpose(1, 2)
        else:
            q_rot = paged_cache.norm_rope_write_layer(
                layer_idx, q, k, v, q_norm_w, k_norm_w, eps, cos, sin, k_eps=k_eps
            )
            context = paged_cache.attend_layer(q_rot.transpose(1, 2), layer_idx).transpose(1, 2)
        context = context.reshape(B, T, self.num_heads * self.head_dim)
        return self.o_proj(context), None, None
