"""Block-granular KV bookkeeping for the paged decode kernels.

The reference manages the KV pool one token at a time (TokenPoolAllocator,
sglang_mlx/srt/mem_cache/memory_pool.py:27-68; RadixCache with page_size
unused, radix_cache.py:98).  The paged kernels read the cache through block
tables, so this module keeps the same structures at block granularity:

* BlockAllocator -- the LIFO free stack of TokenPoolAllocator applied to
  block ids 1..num_blocks-1 (block 0 is the padding block and is never
  handed out; a fresh allocator returns descending runs).  Blocks carry a
  reference count so that one block can sit in several block tables and in
  the radix tree at once; ``free`` drops one reference and a block returns
  to the stack when its last reference goes.
* BlockTable -- one request's blocks and token count.  ``append_slots``
  hands out the slot ids (block * block_size + offset) for new tokens,
  allocating blocks as the context crosses block boundaries.  A partially
  filled last block that is shared with another table or the radix tree is
  copied to a private block before the first write into it (copy-on-write);
  the copy is returned as a (src, dst) pair for ``copy_blocks``.
* build_block_tables -- the int32 [B, max_blocks] table (-1 padded) and
  int32 context lengths that paged_attention reads.
* BlockRadixCache -- RadixCache over whole blocks: a key element is the
  tuple of one block's token ids and the value is the block id, so a prefix
  match returns the blocks that hold it.  The tree holds its own reference
  to every block it caches; eviction drops it.
* plan_prefix_groups / build_cascade_plan -- the shared-prefix plan of
  paged_attention_cascade: groups of sequences whose tables begin with the
  same blocks, the prefix pass's work units over them, and the tail
  partitions (tail_partitions) of the tokens after each prefix.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Callable, Iterable

import numpy as np

from .cache_init_params import CacheInitParams
from .radix_cache import RadixCache
from .base_prefix_cache import EvictParams, InsertParams


class BlockAllocator:
    """Reference-counted LIFO free stack of block ids.  Block 0 is reserved."""

    def __init__(self, num_blocks: int):
        if num_blocks <= 1:
            raise ValueError(f"num_blocks must be at least 2 (block 0 is padding), got {num_blocks}")
        self.num_blocks = num_blocks
        self.clear()

    def clear(self) -> None:
        """Every block free again, in the initial order."""
        self._stack = np.arange(self.num_blocks - 1, 0, -1, dtype=np.int64)
        self._top = self.num_blocks - 1
        self._ref = np.zeros(self.num_blocks, dtype=np.int64)

    def alloc(self, n: int) -> list[int]:
        """The ``n`` most recently freed blocks (a fresh allocator: n, n-1,
        ..., 1), each with one reference.  MemoryError if fewer are free."""
        if n <= 0:
            return []
        if n > self._top:
            raise MemoryError(f"Cannot allocate {n} blocks: only {self._top} available")
        out = self._stack[self._top - n:self._top]
        self._top -= n
        self._ref[out] = 1
        return out.tolist()

    def share(self, blocks: Iterable[int]) -> None:
        """One more reference to each of ``blocks`` (all must be allocated)."""
        b = np.asarray(list(blocks), dtype=np.int64)
        if b.size == 0:
            return
        if (b <= 0).any() or (b >= self.num_blocks).any() or (self._ref[b] <= 0).any():
            raise ValueError("share() of a block that is not allocated")
        np.add.at(self._ref, b, 1)

    def free(self, blocks: Iterable[int]) -> None:
        """Drop one reference to each of ``blocks``; those left without
        references go back on the stack in the given order (the next alloc
        returns the last of them first)."""
        b = np.asarray(list(blocks), dtype=np.int64)
        if b.size == 0:
            return
        if (b <= 0).any() or (b >= self.num_blocks).any():
            raise ValueError("free() of a block id outside the pool")
        for blk in b.tolist():  # in order: a block listed twice drops two references
            if self._ref[blk] <= 0:
                raise ValueError(f"free() of block {blk}, which is not allocated")
            self._ref[blk] -= 1
            if self._ref[blk] == 0:
                self._stack[self._top] = blk
                self._top += 1

    def refcount(self, block: int) -> int:
        return int(self._ref[block])

    @property
    def available_size(self) -> int:
        return self._top


class BlockTable:
    """One request's blocks (in context order) and token count."""

    def __init__(self, block_size: int, blocks: list[int] | None = None, num_tokens: int = 0):
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        self.block_size = block_size
        self.blocks: list[int] = list(blocks or [])
        self.num_tokens = num_tokens
        if num_tokens > len(self.blocks) * block_size or num_tokens < 0:
            raise ValueError("num_tokens does not fit the blocks")

    @classmethod
    def from_prefix(cls, allocator: BlockAllocator, block_size: int, blocks: list[int],
                    num_tokens: int | None = None) -> "BlockTable":
        """A table that starts with shared ``blocks`` (one reference taken on
        each).  ``num_tokens`` defaults to full blocks."""
        allocator.share(blocks)
        return cls(block_size, blocks, len(blocks) * block_size if num_tokens is None else num_tokens)

    def fork(self, allocator: BlockAllocator) -> "BlockTable":
        """A second table over the same tokens (all blocks shared)."""
        return BlockTable.from_prefix(allocator, self.block_size, self.blocks, self.num_tokens)

    def append_slots(self, n: int, allocator: BlockAllocator) -> tuple[np.ndarray, list[tuple[int, int]]]:
        """Slots for the next ``n`` tokens, and the (src, dst) block copies to
        run (copy_blocks) before writing them: a shared, partially filled
        last block is replaced by a private copy first."""
        if n < 0:
            raise ValueError("n must be non-negative")
        bs = self.block_size
        copies: list[tuple[int, int]] = []
        if n == 0:
            return np.zeros(0, dtype=np.int32), copies
        cow = bool(self.num_tokens % bs) and allocator.refcount(self.blocks[-1]) > 1
        need = max(0, -(-(self.num_tokens + n) // bs) - len(self.blocks))
        # Every block this call needs is checked for before any state
        # changes, so a MemoryError leaves the table, its pending
        # copy-on-write and the allocator as they were (a retry after
        # eviction then still copies the shared block).
        if need + cow > allocator.available_size:
            raise MemoryError(f"Cannot allocate {need + cow} blocks: only {allocator.available_size} available")
        if cow:
            old = self.blocks[-1]
            (new,) = allocator.alloc(1)
            copies.append((old, new))
            self.blocks[-1] = new
            allocator.free([old])
        if need > 0:
            self.blocks.extend(allocator.alloc(need))
        t = np.arange(self.num_tokens, self.num_tokens + n, dtype=np.int64)
        blk = np.asarray(self.blocks, dtype=np.int64)[t // bs]
        self.num_tokens += n
        return (blk * bs + t % bs).astype(np.int32), copies

    def release(self, allocator: BlockAllocator) -> None:
        """Drop this table's references."""
        allocator.free(self.blocks)
        self.blocks = []
        self.num_tokens = 0


def build_block_tables(tables: list[BlockTable], max_blocks: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """int32 [len(tables), max_blocks] block table padded with -1, and int32
    context lengths (the layout paged_attention reads)."""
    width = max((len(t.blocks) for t in tables), default=0) if max_blocks is None else max_blocks
    out = np.full((len(tables), max(width, 1)), -1, dtype=np.int32)
    ctx = np.zeros(len(tables), dtype=np.int32)
    for i, t in enumerate(tables):
        if len(t.blocks) > out.shape[1]:
            raise ValueError(f"table {i} has {len(t.blocks)} blocks, more than max_blocks={out.shape[1]}")
        out[i, :len(t.blocks)] = t.blocks
        ctx[i] = t.num_tokens
    return out, ctx


PREFIX_ROWS = 128          # query rows of one prefix-pass workgroup
PREFIX_MAX_CHUNK = 4096    # longest prefix chunk of one prefix-pass workgroup
PREFIX_MIN_CHUNK = 256
TAIL_PART = 512            # default tokens per tail partition
TAIL_MAX_PART = 1024       # longest tail partition of the tail pass


@dataclass
class CascadePlan:
    """Shared-prefix plan of paged_attention_cascade (the pkv_cascade_plan of
    include/pagedkv.h).  Device tensors are int32; ``groups`` keeps the
    host-side (members, prefix tokens) of each group for inspection."""

    prefix_lens: "torch.Tensor"
    members: "torch.Tensor"
    tiles: "torch.Tensor"
    parts: "torch.Tensor"
    chunk_tokens: int
    max_chunks: int
    part_tokens: int
    max_parts: int
    groups: list = field(default_factory=list)


def plan_prefix_groups(block_tables: np.ndarray, context_lens: np.ndarray, block_size: int,
                       min_members: int = 2, min_shared_tokens: int = 0) -> list[tuple[np.ndarray, int]]:
    """Groups of sequences whose block tables begin with the same blocks:
    [(member sequence ids, shared prefix tokens)].  Sequences are grouped by
    their first block id; a group's prefix is the longest run of leading
    blocks that every member maps to the same ids and holds in full (so it
    ends at or before each member's context).  Groups with fewer than
    ``min_members`` members, or whose sharing saves fewer than
    ``min_shared_tokens`` token reads ((members - 1) * prefix), are dropped."""
    bt = np.asarray(block_tables)
    ctx = np.asarray(context_lens).astype(np.int64)
    B = bt.shape[0]
    full = np.minimum(ctx // block_size, bt.shape[1]) if B else ctx
    cand = np.nonzero((full >= 1) & (bt[:, 0] >= 0))[0] if B else np.zeros(0, dtype=np.int64)
    groups = []
    if cand.size == 0:
        return groups
    first = bt[cand, 0]
    order = np.argsort(first, kind="stable")
    cand, first = cand[order], first[order]
    cuts = np.nonzero(np.diff(first))[0] + 1
    for mem in np.split(cand, cuts):
        if mem.size < max(min_members, 2):
            continue
        kmax = int(full[mem].min())
        rows = bt[mem, :kmax]
        same = (rows == rows[0]).all(axis=0)
        k = kmax if same.all() else int(np.argmin(same))
        prefix = k * block_size
        if k == 0 or (mem.size - 1) * prefix < min_shared_tokens:
            continue
        groups.append((np.sort(mem).astype(np.int32), prefix))
    return groups


def tail_partitions(tails: np.ndarray, part_tokens: int) -> np.ndarray:
    """The tail partitions [(sequence, k)] of sequences whose tails (tokens
    after the prefix) are ``tails``: max(1, ceil(tail / part_tokens)) per
    sequence, partition k holding tokens [k * part_tokens, min(tail, (k + 1)
    * part_tokens)) of the tail; longest partitions first, then by sequence
    and k.  int32 [num_parts, 2]."""
    tails = np.maximum(np.asarray(tails, dtype=np.int64), 0)
    n = np.maximum(1, -(-tails // part_tokens))
    seq = np.repeat(np.arange(tails.size, dtype=np.int64), n)
    k = np.arange(seq.size, dtype=np.int64) - np.repeat(np.cumsum(n) - n, n)
    length = np.minimum(part_tokens, tails[seq] - k * part_tokens)
    order = np.lexsort((k, seq, -length))
    return np.stack([seq[order], k[order]], axis=1).astype(np.int32)


def build_cascade_plan(block_tables: np.ndarray, context_lens: np.ndarray, block_size: int, num_heads: int,
                       num_kv_heads: int, device=None, num_cus: int = 256, min_members: int = 2,
                       min_shared_tokens: int = 0, chunk_tokens: int | None = None,
                       part_tokens: int | None = None) -> CascadePlan:
    """The paged_attention_cascade plan of a batch from its host-side int32
    block tables [B, max_blocks] and context lengths [B]
    (build_block_tables' output).  Work units of the prefix pass are
    (up to 128 // group members of a group) x (one chunk of its prefix);
    the chunk is the longest power of two in [256, 4096] tokens (a multiple
    of block_size and 16) that still gives every one of ``num_cus`` CUs a
    workgroup (units x KV heads), unless ``chunk_tokens`` fixes it.  The
    tokens after each sequence's prefix are cut into tail partitions of
    ``part_tokens`` (default TAIL_PART tokens), so that no tail wavefront
    streams much more than the others."""
    import torch

    bt = np.asarray(block_tables, dtype=np.int32)
    ctx = np.asarray(context_lens).astype(np.int64)
    B = bt.shape[0]
    if num_kv_heads <= 0 or num_heads % num_kv_heads:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    group = num_heads // num_kv_heads
    per_tile = max(1, PREFIX_ROWS // group)
    groups = plan_prefix_groups(bt, ctx, block_size, min_members, min_shared_tokens)
    step = int(np.lcm(16, block_size))
    if chunk_tokens is None:
        chunk = PREFIX_MAX_CHUNK
        row_tiles = sum(-(-m.size // per_tile) for m, _ in groups)

        def units(ch):
            return sum(-(-m.size // per_tile) * -(-p // ch) for m, p in groups) * num_kv_heads

        while chunk > PREFIX_MIN_CHUNK and row_tiles and units(chunk) < num_cus:
            chunk //= 2
        chunk = max(step, chunk - chunk % step)
    else:
        chunk = int(chunk_tokens)
        if chunk <= 0 or chunk % step or chunk > PREFIX_MAX_CHUNK:
            raise ValueError("chunk_tokens must be a positive multiple of 16 and of block_size, at most 4096")
    if part_tokens is None:
        part = max(step, TAIL_PART - TAIL_PART % step)
    else:
        part = int(part_tokens)
        if part <= 0 or part % step or part > TAIL_MAX_PART:
            raise ValueError("part_tokens must be a positive multiple of 16 and of block_size, at most 1024")
    prefix_lens = np.zeros(B, dtype=np.int32)
    members, tiles = [], []
    max_chunks = 1
    for mem, p in groups:
        base = len(members)
        members.extend(mem.tolist())
        prefix_lens[mem] = p
        nch = -(-p // chunk)
        max_chunks = max(max_chunks, nch)
        for m0 in range(0, mem.size, per_tile):
            mc = min(per_tile, mem.size - m0)
            for c in range(nch):
                tiles.append((base + m0, mc, c * chunk, min(p, (c + 1) * chunk)))
    tail = np.maximum(ctx - prefix_lens, 0)
    parts = tail_partitions(tail, part)
    max_parts = int(max(1, -(-int(tail.max()) // part))) if B else 1
    dev = torch.device(device) if device is not None else torch.device("cpu")

    def t(a, shape=None):
        x = torch.as_tensor(np.asarray(a, dtype=np.int32).reshape(shape) if shape else np.asarray(a, dtype=np.int32))
        return x.to(dev)

    return CascadePlan(prefix_lens=t(prefix_lens), members=t(members),
                       tiles=t(tiles if tiles else np.zeros((0, 4), dtype=np.int32), (-1, 4)),
                       parts=t(parts, (-1, 2)), chunk_tokens=chunk, max_chunks=max_chunks, part_tokens=part,
                       max_parts=max_parts, groups=groups)


class BlockRadixCache:
    """Prefix cache over whole blocks (page_size = block_size)."""

    def __init__(self, block_size: int, allocator: BlockAllocator, params: CacheInitParams | None = None,
                 clock: Callable[[], float] = time.monotonic):
        params = params or CacheInitParams(page_size=block_size)
        self.block_size = block_size
        self.allocator = allocator
        self.tree = RadixCache(params, clock=clock)
        self.tree.set_allocator(allocator)

    def _chunks(self, tokens) -> list[tuple]:
        bs = self.block_size
        return [tuple(tokens[i:i + bs]) for i in range(0, len(tokens) // bs * bs, bs)]

    def match_prefix(self, tokens):
        """(blocks holding the longest cached whole-block prefix of
        ``tokens``, the tree node it ends at)."""
        r = self.tree.match_prefix(self._chunks(tokens))
        return list(r.device_indices), r.last_node

    def insert(self, tokens, blocks: list[int]) -> int:
        """Cache the whole blocks of ``tokens`` (``blocks`` hold them, in
        order).  The tree takes its own reference on blocks it did not hold;
        returns how many leading blocks were already cached (the caller's
        copies of those are duplicates it may free)."""
        chunks = self._chunks(tokens)
        blocks = list(blocks[:len(chunks)])
        if len(blocks) < len(chunks):
            raise ValueError("insert() needs one block per whole block of tokens")
        cached = self.tree.insert(InsertParams(key=chunks, value=blocks)).prefix_len
        self.allocator.share(blocks[cached:])
        return cached

    def evict(self, num_blocks: int) -> int:
        """Drop the tree's reference to about ``num_blocks`` least recently
        used unlocked blocks; returns how many were dropped."""
        return self.tree.evict(EvictParams(num_tokens=num_blocks)).num_tokens_evicted

    def inc_lock_ref(self, node) -> int:
        return self.tree.inc_lock_ref(node)

    def dec_lock_ref(self, node) -> int:
        return self.tree.dec_lock_ref(node)

    @property
    def cached_blocks(self) -> int:
        return self.tree.total_size()
