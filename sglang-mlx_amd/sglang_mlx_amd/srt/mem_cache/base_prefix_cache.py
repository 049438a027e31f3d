"""Interface types of prefix caches
(sglang_mlx/srt/mem_cache/base_prefix_cache.py:16-93).

KV slot indices travel as plain lists of ints, as in the reference.
"""

from __future__ import annotations

import dataclasses
from abc import ABC, abstractmethod
from typing import Any, NamedTuple


class MatchResult(NamedTuple):
    """device_indices: pool slots of the longest cached prefix, in token
    order; last_node: the tree node where that prefix ends."""

    device_indices: list[int]
    last_node: Any


@dataclasses.dataclass
class InsertParams:
    key: list[int]                    # token ids
    value: list[int] | None = None    # pool slots (None: the token ids stand in)
    priority: int = 0


@dataclasses.dataclass
class InsertResult:
    prefix_len: int                   # tokens of the key that were already cached


@dataclasses.dataclass
class EvictParams:
    num_tokens: int


@dataclasses.dataclass
class EvictResult:
    num_tokens_evicted: int = 0


class BasePrefixCache(ABC):
    @abstractmethod
    def reset(self): ...

    @abstractmethod
    def match_prefix(self, key: list[int]) -> MatchResult: ...

    @abstractmethod
    def insert(self, params: InsertParams) -> InsertResult: ...

    @abstractmethod
    def evict(self, params: EvictParams) -> EvictResult: ...

    @abstractmethod
    def inc_lock_ref(self, node: Any): ...

    @abstractmethod
    def dec_lock_ref(self, node: Any): ...

    def evictable_size(self):
        return 0

    def protected_size(self):
        return 0

    def total_size(self):
        raise NotImplementedError()
