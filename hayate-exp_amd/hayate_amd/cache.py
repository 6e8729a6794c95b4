"""Contiguous per-request KV cache (the format of the reference's
hayate/model/cache.py:6-83), used by import_cache and snapshot.

Tensors have shape (layers, kv_heads, tokens, head_dim).
"""

from __future__ import annotations

import torch


class Cache:
    __slots__ = ("k", "v", "_length")

    def __init__(self):
        self.k: torch.Tensor | None = None
        self.v: torch.Tensor | None = None
        self._length = 0

    @classmethod
    def from_tensors(cls, k: torch.Tensor | None, v: torch.Tensor | None) -> "Cache":
        cache = cls()
        cache.k = k
        cache.v = v
        cache._length = 0 if k is None else int(k.shape[2])
        return cache

    @property
    def length(self) -> int:
        return self._length

    @property
    def capacity(self) -> int:
        return 0 if self.k is None else int(self.k.shape[2])

    def slice(self, end: int, clone: bool = False) -> "Cache":
        if end < 0:
            raise ValueError("cache slice end must be non-negative")
        if self.k is None or self.v is None:
            return Cache()
        if end > self.length:
            raise ValueError(f"cache slice end {end} exceeds cache length {self.length}")
        k = self.k[:, :, :end, :]
        v = self.v[:, :, :end, :]
        if clone:
            k = k.contiguous().clone()
            v = v.contiguous().clone()
        return Cache.from_tensors(k, v)

    def reset(self) -> None:
        self.k = None
        self.v = None
        self._length = 0
