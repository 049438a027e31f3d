"""MHATokenPool / PooledKVCache on the GPU: stores run the HIP append kernel
(token-major layout), fetches gather back.  Round trips are bit-exact.
Cases transplanted from the reference's tests/test_memory_pool.py:85-363 and
:451-538 (store/fetch round trip, layer independence, non-contiguous and
overwritten slots, prefill then decode, prefix reuse across requests)."""

import numpy as np
import pytest
import torch

from sglang_mlx_amd.srt.mem_cache import (InsertParams, MHATokenPool, PooledKVCache, RadixCache,
                                          TokenPoolAllocator)

pytestmark = pytest.mark.gpu

H, D = 4, 8


def kv(gen, S, dtype=torch.float32):
    shape = (1, H, S, D)
    return (torch.randn(shape, generator=gen, device="cuda").to(dtype),
            torch.randn(shape, generator=gen, device="cuda").to(dtype))


@pytest.fixture
def gen():
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    return g


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_store_fetch_roundtrip(gen, dtype):
    pool = MHATokenPool(32, 2, H, D, dtype=dtype)
    k, v = kv(gen, 5, dtype)
    pool.store(0, [1, 2, 3, 4, 5], k, v)
    ko, vo = pool.fetch(0, [1, 2, 3, 4, 5])
    torch.cuda.synchronize()
    assert ko.shape == k.shape and torch.equal(ko, k) and torch.equal(vo, v)
    assert not pool.k_buffer[0][0].any() and not pool.k_buffer[1].any()


def test_float32_inputs_round_into_half_pool(gen):
    pool = MHATokenPool(16, 1, H, D, dtype=torch.bfloat16)
    k, v = kv(gen, 3)
    pool.store(0, [3, 1, 2], k, v)
    ko, vo = pool.fetch(0, [3, 1, 2])
    torch.cuda.synchronize()
    assert torch.equal(ko, k.to(torch.bfloat16)) and torch.equal(vo, v.to(torch.bfloat16))


def test_layers_are_independent_and_slots_arbitrary(gen):
    pool = MHATokenPool(32, 2, H, D, dtype=torch.float32)
    k0, v0 = kv(gen, 3)
    k1, v1 = kv(gen, 3)
    pool.store(0, [5, 10, 20], k0, v0)
    pool.store(1, [5, 10, 20], k1, v1)
    assert torch.equal(pool.fetch(0, [5, 10, 20])[0], k0)
    assert torch.equal(pool.fetch(1, [5, 10, 20])[0], k1)
    assert torch.equal(pool.fetch(0, [5, 10])[1], v0[:, :, :2])


def test_overwrite_slot(gen):
    pool = MHATokenPool(32, 1, H, D, dtype=torch.float32)
    k1, v1 = kv(gen, 1)
    k2, v2 = kv(gen, 1)
    pool.store(0, [1], k1, v1)
    pool.store(0, [1], k2, v2)
    assert torch.equal(pool.fetch(0, [1])[0], k2)


def test_pooled_cache_prefill_decode_and_reuse(gen):
    alloc = TokenPoolAllocator(32)
    pool = MHATokenPool(32, 2, H, D, dtype=torch.float32)
    radix = RadixCache()
    radix.set_allocator(alloc)
    prompt = [10, 20, 30, 40]
    slots = alloc.alloc(4)
    caches = [PooledKVCache(pool, i) for i in range(2)]
    k_in, v_in = kv(gen, 4)
    for c in caches:
        c.set_indices([], slots)
        assert c.offset == 0
        ko, vo = c.update_and_fetch(k_in, v_in)
        assert torch.equal(ko, k_in) and torch.equal(vo, v_in)
    radix.insert(InsertParams(key=prompt, value=slots))
    new = alloc.alloc(1)
    k_new, v_new = kv(gen, 1)
    for c in caches:
        c.set_indices(slots, new)
        assert c.offset == 4
        ko, _ = c.update_and_fetch(k_new, v_new)
        assert ko.shape == (1, H, 5, D)
        assert torch.equal(ko[:, :, :4], k_in) and torch.equal(ko[:, :, 4:], k_new)
    m = radix.match_prefix([10, 20, 30, 40, 50, 60])
    assert m.device_indices == slots
    c = PooledKVCache(pool, 0)
    c.set_indices(m.device_indices, alloc.alloc(2))
    k2, v2 = kv(gen, 2)
    ko, _ = c.update_and_fetch(k2, v2)
    assert ko.shape == (1, H, 6, D) and torch.equal(ko[:, :, :4], k_in)
    ks, _ = c.state
    assert torch.equal(ks, ko)


def test_store_matches_numpy_scatter_at_scale(gen):
    # 2048 tokens into a 16K-slot bf16 pool, 8 heads x D128, random unique slots.
    pool = MHATokenPool(16384, 1, 8, 128, dtype=torch.bfloat16)
    rng = np.random.default_rng(3)
    slots = (rng.choice(16384, 2048, replace=False) + 1).tolist()
    k = torch.randn((1, 8, 2048, 128), generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn((1, 8, 2048, 128), generator=gen, device="cuda").to(torch.bfloat16)
    pool.store(0, slots, k, v)
    expect = torch.zeros((16385, 8, 128), dtype=torch.bfloat16)
    expect[torch.tensor(slots)] = k[0].transpose(0, 1).cpu()
    torch.cuda.synchronize()
    assert torch.equal(pool.k_buffer[0].cpu(), expect)
