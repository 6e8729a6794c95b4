"""Qwen3 transformer on the paged path.

The module tree and parameter names are those of the reference's
hayate/model/qwen.py:8-58 (embed_tokens, layers.N.{self_attn, mlp,
input_layernorm, post_attention_layernorm}, norm, out_head), block.py:8-58
and linear.py:5-22, so a checkpoint loads through the same name map
(hayate/utils.py:114-144). Only the paged mode (the one Engine uses,
engine.py:218-223) is provided: attention goes through
hayate_amd.attention.GroupedQueryAttention and the HIP kernels; the
projections, norms and the MLP stay torch ops.

The geometry is a Qwen3Config (Qwen3-4B by default, qwen.py:14-31); tests
build smaller models with the same attention heads.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn

from .attention import GroupedQueryAttention
from .rope import compute_rope_params


@dataclass(frozen=True)
class Qwen3Config:
    """Architecture sizes (defaults: Qwen3-4B, qwen.py:14-31)."""

    vocab_size: int = 151_936
    hidden_size: int = 2560
    num_layers: int = 36
    num_heads: int = 32
    num_kv_groups: int = 8
    head_dim: int = 128
    intermediate_size: int = 9728
    rms_norm_eps: float = 1e-6
    rope_theta: int = 1_000_000
    max_position_embeddings: int = 40_960


class FeedForward(nn.Module):
    """SiLU-gated MLP (linear.py:5-22)."""

    def __init__(self, emb_dim: int, hidden_dim: int, dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        self.gate_proj = nn.Linear(emb_dim, hidden_dim, bias=False, dtype=dtype)
        self.up_proj = nn.Linear(emb_dim, hidden_dim, bias=False, dtype=dtype)
        self.down_proj = nn.Linear(hidden_dim, emb_dim, bias=False, dtype=dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))


class TransformerBlock(nn.Module):
    """Pre-norm attention + MLP with residuals (block.py:8-58)."""

    def __init__(self, cfg: Qwen3Config, dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        self.self_attn = GroupedQueryAttention(cfg.hidden_size, cfg.num_heads, cfg.num_kv_groups,
                                               cfg.head_dim, dtype=dtype)
        self.mlp = FeedForward(cfg.hidden_size, cfg.intermediate_size, dtype=dtype)
        self.input_layernorm = nn.RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps, dtype=dtype)
        self.post_attention_layernorm = nn.RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps,
                                                   dtype=dtype)

    def forward(self, x, cos, sin, position_ids, prev_k, prev_v, varlen_metadata=None,
                paged_cache=None, layer_idx=None):
        shortcut = x
        x, new_k, new_v = self.self_attn(self.input_layernorm(x), cos, sin, position_ids, prev_k,
                                         prev_v, varlen_metadata, paged_cache, layer_idx)
        x = x + shortcut
        shortcut = x
        x = self.mlp(self.post_attention_layernorm(x)) + shortcut
        return x, new_k, new_v


class Qwen3Model(nn.Module):
    """Embedding, the transformer blocks and the output head (qwen.py:8-165)."""

    def __init__(self, config: Qwen3Config | None = None, dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        cfg = config or Qwen3Config()
        self.config = cfg
        self.num_layers = cfg.num_layers
        self.num_heads = cfg.num_heads
        self.num_kv_groups = cfg.num_kv_groups
        self.head_dim = cfg.head_dim
        self.max_position_embeddings = cfg.max_position_embeddings
        self.rope_theta = cfg.rope_theta
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size, dtype=dtype)
        self.layers = nn.ModuleList([TransformerBlock(cfg, dtype) for _ in range(cfg.num_layers)])
        self.norm = nn.RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps, dtype=dtype)
        self.out_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False, dtype=dtype)
        self.cos = None
        self.sin = None

    def initialize_rope(self, device: torch.device | str) -> None:
        """fp32 RoPE tables on the weights' device (qwen.py:60-67)."""
        self.cos, self.sin = compute_rope_params(self.head_dim, self.rope_theta,
                                                 self.max_position_embeddings, device=device)

    def forward(self, token_ids, prev_k=None, prev_v=None, cache_lens=None, pad_lengths=None,
                use_varlen=False, paged_cache=None):
        """token_ids (B, T) on a uniform batch (begin_batch) or (1, N) packed
        tokens on a varlen tick (begin_tick). Returns (logits, None, None):
        logits (B, 1, vocab) of each sequence's last token, as qwen.py:162-165
        returns for the uniform case."""
        if paged_cache is None:
            raise NotImplementedError("only the paged path is provided (pass paged_cache)")
        if self.cos is None:
            self.initialize_rope(self.embed_tokens.weight.device)
        x = self.embed_tokens(token_ids)
        for layer_idx, block in enumerate(self.layers):
            x, _, _ = block(x, self.cos, self.sin, None, None, None, None, paged_cache, layer_idx)
        if paged_cache.varlen:
            # each sequence's last packed token
            last = paged_cache.q_start[1:].to(torch.long) - 1
            x = x[0].index_select(0, last).unsqueeze(1)
        else:
            x = x[:, -1:, :]
        return self.out_head(self.norm(x)), None, None


def qwen_weight_map(model: Qwen3Model) -> dict[str, torch.Tensor]:
    """Checkpoint tensor name -> parameter (the names of hayate/utils.py:114-144)."""
    weight_map = {
        "model.embed_tokens.weight": model.embed_tokens.weight,
        "model.norm.weight": model.norm.weight,
        "lm_head.weight": model.out_head.weight,
    }
    for i, block in enumerate(model.layers):
        attn = block.self_attn
        prefix = f"model.layers.{i}."
        weight_map.update({
            prefix + "self_attn.q_proj.weight": attn.q_proj.weight,
            prefix + "self_attn.k_proj.weight": attn.k_proj.weight,
            prefix + "self_attn.v_proj.weight": attn.v_proj.weight,
            prefix + "self_attn.o_proj.weight": attn.o_proj.weight,
            prefix + "self_attn.q_norm.weight": attn.q_norm.weight,
            prefix + "self_attn.k_norm.weight": attn.k_norm.weight,
            prefix + "input_layernorm.weight": block.input_layernorm.weight,
            prefix + "mlp.gate_proj.weight": block.mlp.gate_proj.weight,
            prefix + "mlp.up_proj.weight": block.mlp.up_proj.weight,
            prefix + "mlp.down_proj.weight": block.mlp.down_proj.weight,
            prefix + "post_attention_layernorm.weight": block.post_attention_layernorm.weight,
        })
    return weight_map


def load_local_weights(model: Qwen3Model, model_dir: str) -> None:
    """Copy every model tensor from the safetensors files of a local
    checkpoint directory (no download: the directory must exist). As in the
    reference (utils.py:147-217), lm_head is tied to the embedding when the
    checkpoint has none, and a missing required tensor raises KeyError."""
    import glob
    import os

    from safetensors import safe_open

    files = sorted(glob.glob(os.path.join(model_dir, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no safetensors files in '{model_dir}'")
    weight_map = qwen_weight_map(model)
    required = {n for n in weight_map if n != "lm_head.weight"}
    loaded = set()
    for path in files:
        with safe_open(path, "pt", "cpu") as f:
            for name in f.keys():
                param = weight_map.get(name)
                if param is None:
                    continue
                t = f.get_tensor(name)
                if tuple(t.shape) != tuple(param.shape):
                    raise ValueError(f"Shape mismatch in tensor '{name}': "
                                     f"{tuple(param.shape)} vs {tuple(t.shape)}")
                with torch.no_grad():
                    param.copy_(t.to(dtype=param.dtype, device=param.device))
                loaded.add(name)
    missing = sorted(required - loaded)
    if missing:
        raise KeyError(f"Missing required checkpoint tensors: {', '.join(missing[:5])}")
    if "lm_head.weight" not in loaded:
        model.out_head.weight = model.embed_tokens.weight


def init_synthetic_weights(model: Qwen3Model, seed: int = 0) -> None:
    """Random weights of the right scale (no checkpoint can be fetched):
    linears N(0, 1/fan_in), embeddings N(0, 1), norm weights 1 + 0.1 N(0, 1),
    generated on the model's device."""
    dev = model.embed_tokens.weight.device
    g = torch.Generator(device=dev).manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.copy_(1 + 0.1 * torch.randn(p.shape, generator=g, device=dev))
            elif p.dim() == 2 and "embed" not in name:
                p.copy_(torch.randn(p.shape, generator=g, device=dev) * p.shape[1] ** -0.5)
            else:
                p.copy_(torch.randn(p.shape, generator=g, device=dev))
