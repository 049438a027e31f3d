"""Construction parameters of the radix prefix cache
(sglang_mlx/srt/mem_cache/cache_init_params.py:13-17)."""

from __future__ import annotations

import dataclasses


@dataclasses.dataclass
class CacheInitParams:
    """disable: turn the cache into a no-op; page_size: tokens per tree
    granule (kept for interface compatibility, the tree is token-granular as
    in the reference); eviction_policy: lru, lfu, fifo, mru, filo or
    priority."""

    disable: bool = False
    page_size: int = 1
    eviction_policy: str = "lru"
