"""KV memory management around the paged-KV kernels: slot allocator, HBM
pool, per-request cache adapter, the radix prefix cache, and their
block-granular counterparts for the paged kernels."""

from .base_prefix_cache import (BasePrefixCache, EvictParams, EvictResult, InsertParams, InsertResult,
                                MatchResult)
from .cache_init_params import CacheInitParams
from .evict_policy import (EvictionStrategy, FIFOStrategy, FILOStrategy, LFUStrategy, LRUStrategy, MRUStrategy,
                           PriorityStrategy)
from .memory_pool import MHATokenPool, PooledKVCache, TokenPoolAllocator, decode_batch
from .paged_pool import (BlockAllocator, BlockRadixCache, BlockTable, CascadePlan, build_block_tables,
                         build_cascade_plan, plan_prefix_groups, tail_partitions)
from .radix_cache import RadixCache, TreeNode

__all__ = [
    "BasePrefixCache", "BlockAllocator", "BlockRadixCache", "BlockTable", "build_block_tables", "build_cascade_plan",
    "CascadePlan", "plan_prefix_groups", "tail_partitions", "CacheInitParams", "EvictParams", "EvictResult", "EvictionStrategy", "FIFOStrategy",
    "FILOStrategy", "InsertParams", "InsertResult", "LFUStrategy", "LRUStrategy", "MHATokenPool", "MRUStrategy",
    "MatchResult", "PooledKVCache", "PriorityStrategy", "decode_batch", "RadixCache", "TokenPoolAllocator", "TreeNode",
]
