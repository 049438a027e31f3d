"""Decode over float32 caches: the reference's (float query, float cache)
instantiation (paged_attention_inst.metal:69) at every head size and block
size it builds (paged_attention_inst.metal:34-73), against the float64
oracle.

The kernels read the float32 values as stored and run scores and PV on
v_mfma_f32_16x16x4_f32, so nothing is rounded to 16 bits; the bar is
2e-5 abs / 2e-4 rel, a hundredth of float16's (2e-3 / 1e-2).  Cases: every
head size x block size (persistent and partition kernels), split-K
partitions, ALiBi, GQA groups, contexts of 0 and past max_seq_len (zero
rows), masked block ids, and an append of float32 keys/values into float32
caches followed by decode (the path the reference's own fixture takes,
test_paged_attention_kernel.py:138-246, there with a float16 cache).
"""

import math

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from pkv_cases import decode_oracle, make_decode_case
from pkv_torch import to_f64, to_index, to_torch
from sglang_mlx_amd import _ext

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-5, 2e-4


def run(c, partition_size=None, max_seq_len=None):
    args = (to_torch(c.q, "float32"), to_torch(c.k_cache, "float32"), to_torch(c.v_cache, "float32"),
            to_index(c.block_tables), to_index(c.context_lens), c.num_kv_heads, c.scale, c.block_size,
            max_seq_len or c.max_seq_len, None if c.alibi is None else torch.from_numpy(c.alibi).cuda())
    out = (_ext.paged_attention_v1(*args) if partition_size is None
           else _ext.paged_attention_v2(*args, partition_size=partition_size))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    return to_f64(out)


def case(seed, **kw):
    return make_decode_case(seed, cache_dtype="float32", q_dtype="float32", **kw)


def check(c, partition_size=None):
    got = run(c, partition_size)
    ref = decode_oracle(c, partition_size or 0)
    np.testing.assert_allclose(got, ref, atol=ATOL, rtol=RTOL)
    return got, ref


@pytest.mark.parametrize("head_dim", [32, 64, 80, 96, 112, 120, 128, 192, 256])
@pytest.mark.parametrize("block_size", [8, 16, 32])
def test_every_head_and_block_size(head_dim, block_size):
    check(case(6000 + head_dim * 10 + block_size, B=3, Hq=8, Hkv=2, D=head_dim, block_size=block_size,
               ctx_lo=1, ctx_hi=700))


@pytest.mark.parametrize("block_size", [8, 16, 32])
def test_persistent_kernel_batch(block_size):
    # 64 sequences x 8 KV heads = 512 items: the persistent kernel.
    check(case(6100 + block_size, B=64, Hq=32, Hkv=8, D=128, block_size=block_size, ctx_lo=1, ctx_hi=1500))


@pytest.mark.parametrize("partition_size", [32, 256, 512, 4096])
def test_split_k(partition_size):
    check(case(6200 + partition_size, B=3, Hq=28, Hkv=4, D=128, block_size=16, ctx_lo=1, ctx_hi=6000),
          partition_size=partition_size)


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (28, 4), (32, 1)])
def test_gqa_groups_and_alibi(Hq, Hkv):
    check(case(6300 + Hq + Hkv, B=4, Hq=Hq, Hkv=Hkv, D=64, block_size=16, ctx_lo=1, ctx_hi=900, alibi=True))


def test_long_context_v1():
    # One 20K-token sequence: the partition kernel plus the merge.
    check(case(6400, B=1, Hq=16, Hkv=2, D=128, block_size=16, ctx_lo=20000, ctx_hi=20000))


def test_zero_rows_and_masked_blocks():
    c = case(6500, B=4, Hq=8, Hkv=2, D=64, block_size=16, ctx_lo=100, ctx_hi=300, max_seq_len=400)
    c.context_lens[0] = 0
    c.context_lens[1] = 401             # > max_seq_len
    c.block_tables[2, 1] = c.k_cache.shape[0] + 5   # outside the pool: its tokens are masked
    got = run(c)
    assert (got[0] == 0).all() and (got[1] == 0).all()
    # Oracle of row 2 without the masked block's tokens.
    ctx = int(c.context_lens[2])
    keep = np.array([t // 16 != 1 for t in range(ctx)])
    q = orc.decode(c.q, "float32")[2]
    kc, vc = orc.decode(c.k_cache, "float32"), orc.decode(c.v_cache, "float32")
    k, v = orc.gather_kv(kc, vc, np.where(c.block_tables[2] >= 0, np.minimum(c.block_tables[2], kc.shape[0] - 1), 0),
                         ctx)
    ref2 = orc._softmax_attend(q, k[keep], v[keep], c.scale, None)
    np.testing.assert_allclose(got[2], ref2, atol=ATOL, rtol=RTOL)
    ref3 = orc.paged_attention(c.q[3:4], c.k_cache, c.v_cache, c.block_tables[3:4], c.context_lens[3:4],
                               c.num_kv_heads, c.scale, c.block_size, c.max_seq_len, None, "float32", "float32")
    np.testing.assert_allclose(got[3], ref3[0], atol=ATOL, rtol=RTOL)


def test_append_then_decode_float32():
    # float32 keys/values appended into float32 caches (bit copies), then
    # decoded; the reference fixture's geometry (2 sequences, 8 q / 4 kv
    # heads, D 64, bs 16, contexts 25 and 50, tables [[0,1],[2,3,4,5]]).
    rng = np.random.default_rng(6600)
    q = rng.standard_normal((2, 8, 64), dtype=np.float32)
    k = rng.standard_normal((75, 4, 64), dtype=np.float32)
    v = rng.standard_normal((75, 4, 64), dtype=np.float32)
    slots = np.array(list(range(25)) + [32 + i for i in range(50)], dtype=np.int32)
    kc = torch.zeros((20, 4, 16, 16, 4), dtype=torch.float32, device="cuda")
    vc = torch.zeros((20, 4, 64, 16), dtype=torch.float32, device="cuda")
    _ext.reshape_and_cache(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), kc, vc,
                           torch.from_numpy(slots).cuda())
    bt = torch.tensor([[0, 1, -1, -1], [2, 3, 4, 5]], dtype=torch.int32, device="cuda")
    lens = torch.tensor([25, 50], dtype=torch.int32, device="cuda")
    out = _ext.paged_attention_v1(torch.from_numpy(q).cuda(), kc, vc, bt, lens, 4, 1.0 / math.sqrt(64), 16, 64)
    torch.cuda.synchronize()
    kc0 = np.zeros((20, 4, 16, 16, 4), np.float32)
    vc0 = np.zeros((20, 4, 64, 16), np.float32)
    rk, rv = orc.reshape_and_cache_paged5d(k, v, kc0, vc0, slots, "float32", "float32")
    assert np.array_equal(kc.cpu().numpy(), rk) and np.array_equal(vc.cpu().numpy(), rv)
    ref = orc.paged_attention(q, rk, rv, bt.cpu().numpy(), lens.cpu().numpy(), 4, 1.0 / 8.0, 16, 64, None,
                              "float32", "float32")
    np.testing.assert_allclose(out.cpu().double().numpy(), ref, atol=ATOL, rtol=RTOL)
