"""hayate_amd: MI355X-native paged attention for hayate's Engine.

Host code in PyTorch-ROCm over libhayate_attn.so (hand-written HIP kernels
for gfx950, C ABI in include/hayate_attn.h).
"""

from .cache import Cache
from .paged_cache import PagedCacheHandle, PagedKVBatch, PagedKVCacheManager, PagedPrefix
from .prefix_cache import PrefixCache, PrefixCacheMatch
from .rope import compute_rope_params

__all__ = [
    "Cache",
    "PagedCacheHandle",
    "PagedKVBatch",
    "PagedKVCacheManager",
    "PagedPrefix",
    "PrefixCache",
    "PrefixCacheMatch",
    "compute_rope_params",
]
