"""Block-granular KV bookkeeping (BlockAllocator, BlockTable,
build_block_tables, BlockRadixCache).  The allocator is TokenPoolAllocator's
LIFO stack applied to block ids, so its cases restate the reference's
allocator tests (tests/test_memory_pool.py:18-79) for blocks; the rest are
the invariants the paged kernels rely on (every logical token has exactly
one slot, shared prefixes give identical leading block ids, no private block
sits in two tables), checked against brute-force restatements, including a
randomized run of the radix-shared workload's evict/re-allocate churn."""

import numpy as np
import pytest

from sglang_mlx_amd.srt.mem_cache import BlockAllocator, BlockRadixCache, BlockTable, build_block_tables


# ---- BlockAllocator ---------------------------------------------------------

def test_fresh_allocator_hands_out_descending_blocks_and_reserves_block0():
    a = BlockAllocator(10)
    assert a.available_size == 9
    assert a.alloc(3) == [3, 2, 1]
    assert a.alloc(0) == [] and a.alloc(-2) == []
    assert a.alloc(6) == [9, 8, 7, 6, 5, 4]
    assert a.available_size == 0
    with pytest.raises(MemoryError, match="Cannot allocate 1 blocks: only 0 available"):
        a.alloc(1)


def test_free_is_lifo_and_clear_resets():
    a = BlockAllocator(8)
    got = a.alloc(4)            # [4, 3, 2, 1]
    a.free([got[1], got[3]])    # 3 then 1
    assert a.alloc(1) == [1]
    assert a.alloc(1) == [3]
    a.clear()
    assert a.available_size == 7 and a.alloc(2) == [2, 1]


def test_reference_counts():
    a = BlockAllocator(6)
    (b,) = a.alloc(1)
    a.share([b, b])
    assert a.refcount(b) == 3
    a.free([b])
    a.free([b])
    assert a.refcount(b) == 1 and a.available_size == 4
    a.free([b])
    assert a.refcount(b) == 0 and a.available_size == 5
    with pytest.raises(ValueError, match="not allocated"):
        a.free([b])
    with pytest.raises(ValueError, match="not allocated"):
        a.share([b])
    with pytest.raises(ValueError, match="outside the pool"):
        a.free([0])
    with pytest.raises(ValueError):
        BlockAllocator(1)


# ---- BlockTable ---------------------------------------------------------------

def brute_slots(blocks, bs, start, n):
    return [blocks[t // bs] * bs + t % bs for t in range(start, start + n)]


@pytest.mark.parametrize("bs", [1, 8, 16, 32])
def test_append_slots_formula(bs):
    a = BlockAllocator(200)
    t = BlockTable(bs)
    done = 0
    for n in (1, bs - 1 if bs > 1 else 1, 3 * bs + 2, 0, 5):
        slots, copies = t.append_slots(n, a)
        assert copies == []
        assert slots.dtype == np.int32
        assert slots.tolist() == brute_slots(t.blocks, bs, done, n)
        done += n
    assert t.num_tokens == done and len(t.blocks) == -(-done // bs)
    assert len(set(brute_slots(t.blocks, bs, 0, done))) == done


def test_copy_on_write_of_shared_partial_block():
    a = BlockAllocator(32)
    parent = BlockTable(16)
    parent.append_slots(40, a)                 # blocks full, full, 8/16
    child = parent.fork(a)
    assert child.blocks == parent.blocks and all(a.refcount(b) == 2 for b in parent.blocks)
    slots, copies = child.append_slots(4, a)
    old = parent.blocks[2]
    assert len(copies) == 1 and copies[0][0] == old
    new = copies[0][1]
    assert child.blocks == parent.blocks[:2] + [new]
    assert a.refcount(old) == 1 and a.refcount(new) == 1
    assert slots.tolist() == [new * 16 + o for o in range(8, 12)]
    # The parent's own append into its now-private last block needs no copy.
    _, copies = parent.append_slots(2, a)
    assert copies == []
    # Full shared blocks are never copied: a fork at a block boundary.
    t2 = BlockTable(16)
    t2.append_slots(32, a)
    f2 = t2.fork(a)
    _, copies = f2.append_slots(3, a)
    assert copies == [] and f2.blocks[:2] == t2.blocks


def test_failed_append_on_forked_table_changes_nothing():
    # A 5-block pool (ids 1-4): the parent holds [2, 1] (24 tokens, last
    # block half full), another table holds [3], the fork shares [2, 1], and
    # block 4 is free.  Appending 20 tokens to the fork needs the
    # copy-on-write block plus one growth block: the MemoryError must leave
    # table, refcounts and free stack untouched, and the retry once block 3
    # is free must still copy the shared block.
    a = BlockAllocator(5)
    parent = BlockTable(16)
    parent.append_slots(24, a)
    other = BlockTable(16)
    other.append_slots(1, a)
    child = parent.fork(a)
    assert parent.blocks == [2, 1] and other.blocks == [3]

    def state():
        return list(child.blocks), child.num_tokens, a.available_size, [a.refcount(b) for b in range(5)]

    before = state()
    with pytest.raises(MemoryError, match="Cannot allocate 2 blocks: only 1 available"):
        child.append_slots(20, a)
    assert state() == before
    other.release(a)                     # free stack (bottom to top): 4, 3
    slots, copies = child.append_slots(20, a)
    assert copies == [(1, 3)]            # the shared half-full block is copied
    assert child.blocks == [2, 3, 4] and parent.blocks == [2, 1]
    assert a.refcount(1) == 1 and a.refcount(2) == 2 and a.refcount(3) == 1 and a.refcount(4) == 1
    assert slots.tolist() == [3 * 16 + o for o in range(8, 16)] + [4 * 16 + o for o in range(12)]
    assert a.available_size == 0


def test_release_and_build_block_tables():
    a = BlockAllocator(16)
    t1, t2 = BlockTable(4), BlockTable(4)
    t1.append_slots(9, a)
    t2.append_slots(2, a)
    bt, ctx = build_block_tables([t1, t2])
    assert bt.dtype == np.int32 and bt.shape == (2, 3)
    assert bt[0].tolist() == t1.blocks and bt[1].tolist() == t2.blocks + [-1, -1]
    assert ctx.tolist() == [9, 2]
    bt, _ = build_block_tables([t1, t2], max_blocks=5)
    assert bt.shape == (2, 5) and (bt[0, 3:] == -1).all()
    with pytest.raises(ValueError, match="more than max_blocks"):
        build_block_tables([t1], max_blocks=2)
    free0 = a.available_size
    t1.release(a)
    assert a.available_size == free0 + 3 and t1.blocks == [] and t1.num_tokens == 0


# ---- BlockRadixCache ----------------------------------------------------------

def test_radix_match_insert_share_and_evict():
    a = BlockAllocator(64)
    rc = BlockRadixCache(4, a, clock=iter(range(10 ** 6)).__next__)
    prompt = list(range(100, 111))             # 11 tokens: 2 whole blocks + 3
    t = BlockTable(4)
    t.append_slots(len(prompt), a)
    assert rc.insert(prompt, t.blocks) == 0
    assert rc.cached_blocks == 2
    assert all(a.refcount(b) == 2 for b in t.blocks[:2]) and a.refcount(t.blocks[2]) == 1
    blocks, node = rc.match_prefix(prompt + [7, 8, 9])
    assert blocks == t.blocks[:2]
    assert rc.match_prefix(prompt[:3])[0] == []     # less than one block
    assert rc.match_prefix([100, 101, 102, 999, 104])[0] == []
    # A second request reuses the cached prefix.
    t2 = BlockTable.from_prefix(a, 4, blocks)
    t2.append_slots(5, a)
    assert t2.blocks[:2] == t.blocks[:2] and a.refcount(t.blocks[0]) == 3
    # Inserting an already cached prefix reports it and takes no new reference.
    assert rc.insert(prompt, t.blocks) == 2 and a.refcount(t.blocks[0]) == 3
    # Evicting drops only the tree's reference: the blocks stay with the tables.
    rc.inc_lock_ref(node)
    assert rc.evict(10) == 0                 # locked
    rc.dec_lock_ref(node)
    assert rc.evict(10) == 2 and rc.cached_blocks == 0
    assert a.refcount(t.blocks[0]) == 2
    t.release(a)
    t2.release(a)
    assert a.available_size == 63


def test_churn_invariants_against_a_brute_force_restatement():
    # The radix-shared decode workload in miniature: 12 requests share 6
    # prefix blocks, each has 1-5 private blocks; every step frees 10% of the
    # private blocks (LIFO), allocates replacements and rebuilds the tables.
    rng = np.random.default_rng(5)
    bs, nb = 16, 200
    a = BlockAllocator(nb)
    shared = a.alloc(6)
    tables = []
    for _ in range(12):
        t = BlockTable.from_prefix(a, bs, shared)
        t.append_slots(int(rng.integers(1, 5 * bs + 1)), a)
        tables.append(t)
    a.free(shared)                            # only the tables hold the prefix now
    stack_model = list(range(nb - 1, 0, -1))  # restated LIFO: the allocator's order
    held = {b for t in tables for b in t.blocks}
    stack_model = [b for b in stack_model if b not in held]
    for step in range(20):
        private = [(i, j) for i, t in enumerate(tables) for j in range(6, len(t.blocks))]
        pick = rng.choice(len(private), size=max(1, len(private) // 10), replace=False)
        victims = [private[k] for k in pick]
        freed = [tables[i].blocks[j] for i, j in victims]
        a.free(freed)
        stack_model.extend(freed)
        fresh = a.alloc(len(victims))
        assert fresh == stack_model[len(stack_model) - len(victims):]
        del stack_model[len(stack_model) - len(victims):]
        for (i, j), b in zip(victims, fresh):
            tables[i].blocks[j] = b
        bt, ctx = build_block_tables(tables)
        # Invariants.
        assert (bt[:, :6] == np.asarray(shared)).all()
        priv = [b for t in tables for b in t.blocks[6:]]
        assert len(priv) == len(set(priv)) and not set(priv) & set(shared)
        for i, t in enumerate(tables):
            slots = [bt[i, p // bs] * bs + p % bs for p in range(ctx[i])]
            assert len(set(slots)) == ctx[i]
        assert a.available_size == len(stack_model) == nb - 1 - len(priv) - len(shared)
        for b in shared:
            assert a.refcount(b) == len(tables)
