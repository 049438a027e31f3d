"""Host-side KV memory structures (CPU): TokenPoolAllocator, RadixCache, the
eviction strategies and their integration.

KATs transplanted from the reference's tests/test_memory_pool.py:18-79,
:369-445 and tests/test_radix_cache.py:9-192; the allocator's closed form
(fresh pool hands out descending runs, LIFO reuse, memory_pool.py:38-60);
eviction order of every strategy under a logical clock; and randomized
operation sequences checked against invariants (slot conservation,
evictable + protected == total, matches return the inserted slots).
"""

import itertools
import random

import pytest

from sglang_mlx_amd.srt.mem_cache import (CacheInitParams, EvictParams, InsertParams, MHATokenPool, PooledKVCache,
                                          RadixCache, TokenPoolAllocator)


def logical_clock():
    c = itertools.count(1)
    return lambda: float(next(c))


# ---------------------------------------------------------------------------
# TokenPoolAllocator
# ---------------------------------------------------------------------------


class TestTokenPoolAllocator:
    def test_basic_alloc_free(self):
        a = TokenPoolAllocator(10)
        assert a.available_size == 10
        s = a.alloc(3)
        assert len(s) == 3 and a.available_size == 7
        a.free(s)
        assert a.available_size == 10

    def test_slot_zero_reserved(self):
        a = TokenPoolAllocator(100)
        s = a.alloc(100)
        assert 0 not in s and min(s) >= 1

    def test_alloc_zero_and_negative(self):
        a = TokenPoolAllocator(5)
        assert a.alloc(0) == [] and a.alloc(-2) == [] and a.available_size == 5

    def test_overflow_message(self):
        a = TokenPoolAllocator(5)
        with pytest.raises(MemoryError, match="Cannot allocate 6 slots: only 5 available"):
            a.alloc(6)

    def test_exact_capacity_and_clear(self):
        a = TokenPoolAllocator(5)
        assert len(a.alloc(5)) == 5 and a.available_size == 0
        a.clear()
        assert a.available_size == 5 and a.alloc(2) == [2, 1]

    def test_invalid_pool_size(self):
        for n in (0, -1):
            with pytest.raises(ValueError, match="pool_size must be positive"):
                TokenPoolAllocator(n)

    def test_closed_form_order(self):
        # Fresh pool: [P, P-1, ..., 1] as a stack; alloc(n) pops the top n in list order.
        a = TokenPoolAllocator(10)
        assert a.alloc(3) == [3, 2, 1]
        assert a.alloc(2) == [5, 4]
        a.free([2, 9])          # stack is now [10, 9, 8, 7, 6, 2, 9]
        assert a.alloc(1) == [9]
        assert a.alloc(2) == [6, 2]
        b = TokenPoolAllocator(10)
        b.alloc(4)
        b.free([7, 8])
        assert b.alloc(3) == [5, 7, 8]

    def test_no_duplicates_and_conservation(self):
        a = TokenPoolAllocator(50)
        s = a.alloc(20) + a.alloc(20)
        assert len(set(s)) == 40
        rng = random.Random(0)
        held = list(s)
        for _ in range(500):
            if held and rng.random() < 0.5:
                k = rng.randint(1, len(held))
                rng.shuffle(held)
                a.free(held[:k])
                held = held[k:]
            else:
                n = rng.randint(0, a.available_size)
                held += a.alloc(n)
            assert len(set(held)) == len(held)
            assert a.available_size + len(held) == 50

    def test_free_beyond_capacity_grows(self):
        a = TokenPoolAllocator(2)
        a.free([7, 8, 9])
        assert a.available_size == 5 and a.alloc(3) == [7, 8, 9]


# ---------------------------------------------------------------------------
# RadixCache KATs
# ---------------------------------------------------------------------------


def test_basic_match():
    c = RadixCache()
    c.insert(InsertParams(key=[1, 2, 3, 4, 5]))
    assert len(c.match_prefix([1, 2, 3, 4, 5]).device_indices) == 5
    assert len(c.match_prefix([1, 2, 3, 4, 5, 6, 7]).device_indices) == 5
    assert c.match_prefix([9, 9, 9]).device_indices == []
    assert c.match_prefix([]).device_indices == []


def test_value_defaults_to_token_ids_and_explicit_slots():
    c = RadixCache()
    c.insert(InsertParams(key=[5, 6, 7]))
    assert c.match_prefix([5, 6, 7]).device_indices == [5, 6, 7]
    c.insert(InsertParams(key=[8, 9], value=[101, 102]))
    assert c.match_prefix([8, 9, 10]).device_indices == [101, 102]


def test_shared_prefix_and_multi_turn():
    c = RadixCache()
    system = [1, 2, 3, 4, 5]
    c.insert(InsertParams(key=system + [10, 11, 12]))
    assert len(c.match_prefix(system + [20, 21, 22]).device_indices) == 5
    turn1 = [1, 2, 3, 10, 11]
    c2 = RadixCache()
    c2.insert(InsertParams(key=turn1))
    assert len(c2.match_prefix(turn1 + [50, 51, 20, 21]).device_indices) == 5


def test_split_preserves_slots():
    c = RadixCache()
    c.insert(InsertParams(key=[1, 2, 3, 4, 5], value=[11, 12, 13, 14, 15]))
    r = c.insert(InsertParams(key=[1, 2, 3, 6, 7], value=[11, 12, 13, 16, 17]))
    assert r.prefix_len == 3
    assert c.match_prefix([1, 2, 3, 4, 5]).device_indices == [11, 12, 13, 14, 15]
    assert c.match_prefix([1, 2, 3, 6, 7]).device_indices == [11, 12, 13, 16, 17]
    assert c.match_prefix([1, 2, 3]).device_indices == [11, 12, 13]
    c.insert(InsertParams(key=[1, 9, 9], value=[11, 19, 19]))
    assert c.match_prefix([1, 2, 3, 4, 5]).device_indices == [11, 12, 13, 14, 15]
    assert c.match_prefix([1, 9, 9]).device_indices == [11, 19, 19]


def test_match_splits_partially_matched_node():
    c = RadixCache()
    c.insert(InsertParams(key=[1, 2, 3, 4, 5]))
    r = c.match_prefix([1, 2, 3, 9])
    assert r.device_indices == [1, 2, 3] and r.last_node.key == [1, 2, 3]
    assert [n.key for n in r.last_node.children.values()] == [[4, 5]]
    assert c.total_size() == 5


def test_lock_prevents_and_unlock_allows_eviction():
    c = RadixCache()
    c.insert(InsertParams(key=[1, 2, 3, 4, 5]))
    node = c.match_prefix([1, 2, 3, 4, 5]).last_node
    assert c.inc_lock_ref(node) == -5
    assert c.evictable_size() == 0 and c.protected_size() == 5
    c.evict(EvictParams(num_tokens=100))
    assert len(c.match_prefix([1, 2, 3, 4, 5]).device_indices) == 5
    assert c.dec_lock_ref(node) == 5
    c.evict(EvictParams(num_tokens=100))
    assert c.match_prefix([1, 2, 3, 4, 5]).device_indices == []


def test_lock_walks_to_root():
    c = RadixCache()
    c.insert(InsertParams(key=[1, 2, 3, 4, 5]))
    c.insert(InsertParams(key=[1, 2, 3, 6, 7]))
    c.inc_lock_ref(c.match_prefix([1, 2, 3, 4, 5]).last_node)
    assert c.evict(EvictParams(num_tokens=100)).num_tokens_evicted == 2   # only [6, 7]
    assert len(c.match_prefix([1, 2, 3]).device_indices) == 3
    assert c.match_prefix([1, 2, 3, 6, 7]).device_indices == [1, 2, 3]


def test_lru_eviction_and_cascade():
    clk = logical_clock()
    c = RadixCache(clock=clk)
    for k in ([1, 2, 3], [4, 5, 6], [7, 8, 9]):
        c.insert(InsertParams(key=k))
    c.match_prefix([4, 5, 6])
    assert c.evict(EvictParams(num_tokens=3)).num_tokens_evicted == 3
    assert c.match_prefix([1, 2, 3]).device_indices == []
    assert len(c.match_prefix([4, 5, 6]).device_indices) == 3
    c2 = RadixCache()
    c2.insert(InsertParams(key=[1, 2, 3, 4, 5]))
    c2.insert(InsertParams(key=[1, 2, 3, 6, 7]))
    assert c2.evict(EvictParams(num_tokens=100)).num_tokens_evicted == 7
    assert c2.match_prefix([1, 2, 3]).device_indices == [] and c2.total_size() == 0


def test_few_shot_reuse():
    c = RadixCache()
    examples = list(range(100))
    reused = 0
    for i in range(10):
        q = examples + [1000 + i, 1001 + i]
        reused += len(c.match_prefix(q).device_indices)
        c.insert(InsertParams(key=q))
    assert reused == 9 * 100


def test_unknown_policy_and_disable():
    with pytest.raises(ValueError, match="Unknown eviction policy: nope"):
        RadixCache(CacheInitParams(eviction_policy="nope"))
    c = RadixCache(CacheInitParams(disable=True))
    assert c.insert(InsertParams(key=[1, 2])).prefix_len == 0
    assert c.match_prefix([1, 2]).device_indices == []
    assert c.evict(EvictParams(5)).num_tokens_evicted == 0
    assert c.inc_lock_ref(c.root_node) == 0


@pytest.mark.parametrize("policy,expected", [
    ("lru", [[1], [2], [3]]),          # least recently accessed first
    ("mru", [[3], [2], [1]]),
    ("fifo", [[1], [3], [2]]),         # creation order: [1] then [3] then [2]
    ("filo", [[2], [3], [1]]),
    ("lfu", [[1], [2], [3]]),          # hit_count is never incremented (as in the reference): LRU
    ("priority", [[3], [1], [2]]),     # priorities 5, 9, 0 -> lowest first
])
def test_eviction_order_per_strategy(policy, expected):
    # Created in the order [1], [3], [2] (priorities 5, 0, 9), then
    # accessed in the order [1], [2], [3].
    c2 = RadixCache(CacheInitParams(eviction_policy=policy), clock=logical_clock())
    c2.insert(InsertParams(key=[1], priority=5))
    c2.insert(InsertParams(key=[3], priority=0))
    c2.insert(InsertParams(key=[2], priority=9))
    c2.match_prefix([1])
    c2.match_prefix([2])
    c2.match_prefix([3])
    order = []
    for _ in range(3):
        before = {tuple(n.key) for n in c2.root_node.children.values()}
        c2.evict(EvictParams(num_tokens=1))
        after = {tuple(n.key) for n in c2.root_node.children.values()}
        order.append(list((before - after).pop()))
    assert order == expected


# ---------------------------------------------------------------------------
# Integration with the allocator
# ---------------------------------------------------------------------------


def test_eviction_frees_slots():
    a = TokenPoolAllocator(20)
    c = RadixCache()
    c.set_allocator(a)
    s1 = a.alloc(5)
    c.insert(InsertParams(key=[1, 2, 3, 4, 5], value=s1))
    c.insert(InsertParams(key=[6, 7, 8, 9, 10], value=a.alloc(5)))
    assert a.available_size == 10
    c.evict(EvictParams(num_tokens=100))
    assert a.available_size == 20


def test_eviction_partial_free_and_sharing():
    a = TokenPoolAllocator(20)
    c = RadixCache(clock=logical_clock())
    c.set_allocator(a)
    c.insert(InsertParams(key=[1, 2, 3], value=a.alloc(3)))
    c.insert(InsertParams(key=[4, 5, 6], value=a.alloc(3)))
    c.match_prefix([4, 5, 6])
    before = a.available_size
    c.evict(EvictParams(num_tokens=3))
    assert a.available_size - before == 3
    a2 = TokenPoolAllocator(50)
    c2 = RadixCache()
    c2.set_allocator(a2)
    c2.insert(InsertParams(key=[1, 2, 3, 10, 11], value=a2.alloc(5)))
    m = c2.match_prefix([1, 2, 3, 20, 21])
    assert len(m.device_indices) == 3
    c2.insert(InsertParams(key=[1, 2, 3, 20, 21], value=m.device_indices + a2.alloc(2)))
    assert a2.available_size == 43


@pytest.mark.parametrize("seed", range(6))
def test_random_operations_keep_invariants(seed):
    rng = random.Random(seed)
    P = 400
    a = TokenPoolAllocator(P)
    c = RadixCache(CacheInitParams(eviction_policy=rng.choice(["lru", "fifo", "mru", "filo", "priority"])),
                   clock=logical_clock())
    c.set_allocator(a)
    locked = []
    vocab = [rng.randint(0, 6) for _ in range(6)]
    for _ in range(300):
        op = rng.random()
        if op < 0.5:
            key = [rng.choice(vocab) for _ in range(rng.randint(1, 12))]
            m = c.match_prefix(key)
            need = len(key) - len(m.device_indices)
            if need > a.available_size:
                c.evict(EvictParams(num_tokens=need - a.available_size))
            if need > a.available_size:
                continue
            slots = m.device_indices + a.alloc(need)
            r = c.insert(InsertParams(key=key, value=slots, priority=rng.randint(0, 3)))
            assert r.prefix_len == len(m.device_indices)
            assert c.match_prefix(key).device_indices == slots
        elif op < 0.65:
            node = c.match_prefix([rng.choice(vocab)]).last_node
            c.inc_lock_ref(node)
            locked.append(node)
        elif op < 0.8 and locked:
            c.dec_lock_ref(locked.pop(rng.randrange(len(locked))))
        else:
            c.evict(EvictParams(num_tokens=rng.randint(1, 30)))
        assert a.available_size + c.total_size() == P
        assert c.evictable_size() + c.protected_size() == c.total_size()
        live = []
        todo = [c.root_node]
        while todo:
            n = todo.pop()
            live += n.value or []
            todo += n.children.values()
        assert len(set(live)) == len(live)


def test_pool_needs_a_gpu_device_for_store():
    # The pool's store goes through the HIP append kernel; CPU buffers are
    # rejected like any other kernel input.
    import torch
    pool = MHATokenPool(8, 1, 2, 16, dtype=torch.float32, device="cpu")
    with pytest.raises(RuntimeError, match="GPU-only"):
        pool.store(0, [1, 2], torch.zeros(1, 2, 2, 16), torch.zeros(1, 2, 2, 16))
    cache = PooledKVCache(pool, 0)
    cache.set_indices([1, 2, 3], [4])
    assert cache.offset == 3 and cache.make_mask(1) is None and cache.make_mask(2) == "causal"
    cache.set_indices([], [1, 2, 3])
    m = cache.make_mask(3, window_size=2)
    assert m.shape == (3, 3) and not m[2, 0] and m[2, 1] and m[2, 2]
    cache.set_indices([1, 2, 3], [4, 5])
    m = cache.make_mask(2, return_array=True)
    assert m.shape == (2, 5) and m[0, 3] and not m[0, 4] and m[1, 4]
    cache.set_indices([], [])
    assert cache.state == (None, None)
