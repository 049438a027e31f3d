"""Token-granular radix tree over KV pool slots: the prefix cache of the
reference (sglang_mlx/srt/mem_cache/radix_cache.py:50-391).

Observable behaviour follows the reference:
  * ``match_prefix`` returns the pool slots of the longest cached prefix and
    splits a node that the key matches only partly (:135-148, :238-270);
  * ``insert`` adds the uncached suffix as a new leaf, splitting where the
    key diverges inside a node, and returns the cached prefix length; a
    missing value stands for the token ids themselves (:150-163, :294-338);
  * ``evict`` frees unlocked leaves in strategy order, returns their slots to
    the attached allocator and lets a parent that becomes a childless,
    unlocked leaf join the queue (:165-189);
  * lock references walk from a node to the root and move the node's length
    between the evictable and protected counters (:191-221); the root is
    always locked (:124).

Determinism.  The reference stamps nodes with ``time.monotonic()``; here the
clock is injectable (``clock=`` of the constructor), and every place that
reads it reads it in the same order as the reference, so a logical clock
replays the same ordering deterministically.  Ties between equal eviction
keys are broken by node creation order (the reference leaves them to set
iteration order).
"""

from __future__ import annotations

import heapq
import itertools
import sys
import time
from typing import Callable

from .base_prefix_cache import (BasePrefixCache, EvictParams, EvictResult, InsertParams, InsertResult,
                                MatchResult)
from .cache_init_params import CacheInitParams
from .evict_policy import STRATEGIES

_ids = itertools.count()


class TreeNode:
    """One edge of the tree: ``key`` holds token ids, ``value`` the pool
    slots of those tokens (``None`` once evicted)."""

    def __init__(self, clock: Callable[[], float] = time.monotonic, priority: int = 0, id: int | None = None):
        self.children: dict[int, TreeNode] = {}
        self.parent: TreeNode | None = None
        self.key: list[int] = []
        self.value: list[int] | None = None
        self.lock_ref = 0
        self.last_access_time = clock()
        self.creation_time = clock()
        self.hit_count = 0
        self.priority = priority
        self.id = next(_ids) if id is None else id

    @property
    def evicted(self) -> bool:
        return self.value is None

    def __lt__(self, other: "TreeNode") -> bool:
        return (self.last_access_time, self.id) < (other.last_access_time, other.id)

    def __repr__(self) -> str:
        more = "..." if len(self.key) > 10 else ""
        return f"TreeNode(id={self.id}, key={self.key[:10]}{more}, lock_ref={self.lock_ref})"


def common_prefix_len(a: list[int], b: list[int]) -> int:
    n = min(len(a), len(b))
    i = 0
    while i < n and a[i] == b[i]:
        i += 1
    return i


class RadixCache(BasePrefixCache):
    def __init__(self, params: CacheInitParams | None = None, clock: Callable[[], float] = time.monotonic):
        params = params or CacheInitParams()
        self.disable = params.disable
        self.page_size = params.page_size
        self.eviction_policy = params.eviction_policy.lower()
        if self.eviction_policy not in STRATEGIES:
            raise ValueError(f"Unknown eviction policy: {self.eviction_policy}")
        self.eviction_strategy = STRATEGIES[self.eviction_policy]()
        self.clock = clock
        self.allocator = None
        self.evictable_leaves: set[TreeNode] = set()
        self.reset()

    # ---- public API -------------------------------------------------------

    def reset(self):
        self.root_node = TreeNode(self.clock, priority=-sys.maxsize)
        self.root_node.value = []
        self.root_node.lock_ref = 1
        self.evictable_size_ = 0
        self.protected_size_ = 0
        self.evictable_leaves.clear()

    def set_allocator(self, allocator) -> None:
        """Eviction returns the slots of evicted nodes to ``allocator.free``."""
        self.allocator = allocator

    def match_prefix(self, key: list[int]) -> MatchResult:
        if self.disable or not key:
            return MatchResult(device_indices=[], last_node=self.root_node)
        pieces, node = self._walk_match(key)
        slots: list[int] = []
        for p in pieces:
            slots.extend(p)
        return MatchResult(device_indices=slots, last_node=node)

    def insert(self, params: InsertParams) -> InsertResult:
        if self.disable:
            return InsertResult(prefix_len=0)
        value = list(params.key) if params.value is None else params.value
        return InsertResult(prefix_len=self._walk_insert(params.key, value, params.priority or 0))

    def evict(self, params: EvictParams) -> EvictResult:
        if self.disable:
            return EvictResult()
        prio = self.eviction_strategy.get_priority
        heap = [(prio(n), n.id, n) for n in self.evictable_leaves]
        heapq.heapify(heap)
        freed = 0
        while freed < params.num_tokens and heap:
            _, _, leaf = heapq.heappop(heap)
            if self.allocator is not None:
                self.allocator.free(leaf.value)
            freed += len(leaf.value)
            parent = leaf.parent
            self._remove_leaf(leaf)
            if not parent.children and parent.lock_ref == 0:
                heapq.heappush(heap, (prio(parent), parent.id, parent))
        return EvictResult(num_tokens_evicted=freed)

    def inc_lock_ref(self, node: TreeNode) -> int:
        """Lock ``node`` and its ancestors; returns the change of the
        evictable size (<= 0)."""
        if self.disable:
            return 0
        delta = 0
        while node is not self.root_node:
            if node.lock_ref == 0:
                n = len(node.key)
                self.evictable_size_ -= n
                self.protected_size_ += n
                delta -= n
            node.lock_ref += 1
            self._refresh_leaf(node)
            node = node.parent
        return delta

    def dec_lock_ref(self, node: TreeNode) -> int:
        """Undo one inc_lock_ref; returns the change of the evictable size
        (>= 0)."""
        if self.disable:
            return 0
        delta = 0
        while node is not self.root_node:
            if node.lock_ref == 1:
                n = len(node.key)
                self.evictable_size_ += n
                self.protected_size_ -= n
                delta += n
            node.lock_ref -= 1
            self._refresh_leaf(node)
            node = node.parent
        return delta

    def evictable_size(self):
        return self.evictable_size_

    def protected_size(self):
        return self.protected_size_

    def total_size(self):
        total, todo = 0, [self.root_node]
        while todo:
            n = todo.pop()
            total += len(n.value) if n.value else 0
            todo.extend(c for c in n.children.values() if not c.evicted)
        return total

    def pretty_print(self):
        todo = [(self.root_node, 0)]
        while todo:
            n, indent = todo.pop()
            print(" " * indent, len(n.key), n.key[:10], f"r={n.lock_ref}")
            todo.extend((c, indent + 2) for c in n.children.values())
        print(f"#tokens: {self.total_size()}")

    # ---- internals ----------------------------------------------------------

    def _walk_match(self, key: list[int]):
        now = self.clock()
        node = self.root_node
        node.last_access_time = now
        pieces: list[list[int]] = []
        while key and key[0] in node.children:
            child = node.children[key[0]]
            child.last_access_time = now
            n = common_prefix_len(child.key, key)
            if n < len(child.key):
                head = self._split(child, n)
                pieces.append(head.value)
                return pieces, head
            pieces.append(child.value)
            node = child
            key = key[n:]
        return pieces, node

    def _walk_insert(self, key: list[int], value: list[int], priority: int) -> int:
        now = self.clock()
        node = self.root_node
        node.last_access_time = now
        node.priority = max(node.priority, priority)
        matched = 0
        while key and key[0] in node.children:
            node = node.children[key[0]]
            node.last_access_time = now
            n = common_prefix_len(node.key, key)
            matched += n
            key, value = key[n:], value[n:]
            if n < len(node.key):
                node = self._split(node, n)
            node.priority = max(node.priority, priority)
        if key:
            leaf = TreeNode(self.clock, priority=priority)
            leaf.parent = node
            leaf.key = list(key)
            leaf.value = list(value)
            node.children[key[0]] = leaf
            self.evictable_size_ += len(key)
            self._refresh_leaf(node)
            self._refresh_leaf(leaf)
        return matched

    def _split(self, child: TreeNode, n: int) -> TreeNode:
        """parent -> child[k0..kL) becomes parent -> head[k0..kn) -> child[kn..kL);
        both keep their part of the slots.  Returns head."""
        head = TreeNode(self.clock, priority=child.priority)
        parent = child.parent
        head.parent = parent
        head.lock_ref = child.lock_ref
        head.key, child.key = child.key[:n], child.key[n:]
        head.value, child.value = child.value[:n], child.value[n:]
        head.children = {child.key[0]: child}
        child.parent = head
        parent.children[head.key[0]] = head
        return head

    def _remove_leaf(self, leaf: TreeNode):
        parent = leaf.parent
        removed = parent.children.pop(leaf.key[0], None)
        assert removed is leaf, f"parent does not hold child key {leaf.key[0]}"
        self.evictable_size_ -= len(leaf.key)
        self.evictable_leaves.discard(leaf)
        self._refresh_leaf(parent)

    def _refresh_leaf(self, node: TreeNode):
        """Keep ``evictable_leaves`` = unlocked, live nodes without live children."""
        leaf = (not node.evicted and node.lock_ref == 0
                and all(c.evicted for c in node.children.values()))
        if leaf:
            self.evictable_leaves.add(node)
        else:
            self.evictable_leaves.discard(node)
