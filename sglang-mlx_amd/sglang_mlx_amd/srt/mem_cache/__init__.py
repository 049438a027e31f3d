"""KV memory management around the paged-KV kernels: slot allocator, HBM
pool, per-request cache adapter and the radix prefix cache."""

from .base_prefix_cache import (BasePrefixCache, EvictParams, EvictResult, InsertParams, InsertResult,
                                MatchResult)
from .cache_init_params import CacheInitParams
from .evict_policy import (EvictionStrategy, FIFOStrategy, FILOStrategy, LFUStrategy, LRUStrategy, MRUStrategy,
                           PriorityStrategy)
from .memory_pool import MHATokenPool, PooledKVCache, TokenPoolAllocator
from .radix_cache import RadixCache, TreeNode

__all__ = [
    "BasePrefixCache", "CacheInitParams", "EvictParams", "EvictResult", "EvictionStrategy", "FIFOStrategy",
    "FILOStrategy", "InsertParams", "InsertResult", "LFUStrategy", "LRUStrategy", "MHATokenPool", "MRUStrategy",
    "MatchResult", "PooledKVCache", "PriorityStrategy", "RadixCache", "TokenPoolAllocator", "TreeNode",
]
