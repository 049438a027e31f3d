"""Eviction orderings of the radix cache (sglang_mlx/srt/mem_cache/evict_policy.py:19-57).

Each strategy maps a tree node to a sort key; the cache evicts the smallest
key first.
"""

from __future__ import annotations

from abc import ABC, abstractmethod


class EvictionStrategy(ABC):
    @abstractmethod
    def get_priority(self, node): ...


class LRUStrategy(EvictionStrategy):
    """Least recently used first."""

    def get_priority(self, node):
        return node.last_access_time


class LFUStrategy(EvictionStrategy):
    """Fewest hits first, then least recently used."""

    def get_priority(self, node):
        return (node.hit_count, node.last_access_time)


class FIFOStrategy(EvictionStrategy):
    """Oldest node first."""

    def get_priority(self, node):
        return node.creation_time


class MRUStrategy(EvictionStrategy):
    """Most recently used first."""

    def get_priority(self, node):
        return -node.last_access_time


class FILOStrategy(EvictionStrategy):
    """Newest node first."""

    def get_priority(self, node):
        return -node.creation_time


class PriorityStrategy(EvictionStrategy):
    """Lowest request priority first, then least recently used."""

    def get_priority(self, node):
        return (node.priority, node.last_access_time)


STRATEGIES = {
    "lru": LRUStrategy,
    "lfu": LFUStrategy,
    "fifo": FIFOStrategy,
    "mru": MRUStrategy,
    "filo": FILOStrategy,
    "priority": PriorityStrategy,
}
