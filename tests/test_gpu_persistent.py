"""GPU parity of the persistent decode schedule (paged_attention_v1 with at
least one (sequence, KV head) item per resident workgroup: 256 or more on
MI355X).  Tolerances as elsewhere: float16 2e-3 abs / 1e-2 rel, bfloat16
1e-2 abs / 2e-2 rel.  The schedule is static (no counters or atomics), so
repeated calls are bit-identical, also with a split-K call in between that
shares the workspace."""

import numpy as np
import pytest
import torch

from pkv_cases import decode_oracle, make_decode_case, tolerance
from pkv_torch import to_f64, to_index, to_torch
from sglang_mlx_amd import kernels

pytestmark = pytest.mark.gpu


def run(c, partition_size=None):
    args = (to_torch(c.q, c.q_dtype), to_torch(c.k_cache, c.cache_dtype), to_torch(c.v_cache, c.cache_dtype),
            to_index(c.block_tables), to_index(c.context_lens), c.num_kv_heads, c.scale, c.block_size,
            c.max_seq_len, None if c.alibi is None else torch.from_numpy(c.alibi).cuda())
    out = (kernels.paged_attention_v1(*args) if partition_size is None
           else kernels.paged_attention_v2(*args, partition_size=partition_size))
    torch.cuda.synchronize()
    return out


def check(c):
    out = run(c)
    a, r = tolerance(c.q_dtype, c.cache_dtype)
    np.testing.assert_allclose(to_f64(out), decode_oracle(c), atol=a, rtol=r)
    return out


@pytest.mark.parametrize("D,bs", [(64, 8), (64, 16), (128, 16), (128, 32), (256, 16), (96, 8)])
def test_head_and_block_sizes(D, bs):
    c = make_decode_case(3000 + D + bs, B=128, Hq=8, Hkv=4, D=D, block_size=bs, ctx_lo=1, ctx_hi=400,
                         cache_dtype="bfloat16")
    check(c)


@pytest.mark.parametrize("q_dtype,cache_dtype", [("float16", "float16"), ("float32", "bfloat16"),
                                                 ("float32", "float16")])
def test_dtype_pairs(q_dtype, cache_dtype):
    c = make_decode_case(3100, B=128, Hq=16, Hkv=4, D=128, block_size=16, ctx_lo=1, ctx_hi=600,
                         cache_dtype=cache_dtype, q_dtype=q_dtype)
    check(c)


def test_gqa7_alibi_and_zero_rows():
    c = make_decode_case(3200, B=128, Hq=28, Hkv=4, D=128, block_size=16, ctx_lo=1, ctx_hi=900,
                         cache_dtype="bfloat16", alibi=True, max_seq_len=800)
    c.context_lens[::7] = 0            # empty contexts -> zero rows
    out = check(c)                     # ctx > 800 -> zero rows as well
    zero = (c.context_lens == 0) | (c.context_lens > 800)
    assert zero.any() and torch.count_nonzero(out[torch.from_numpy(zero)]).item() == 0


def test_more_sequences_than_the_ordering_limit():
    # 1100 sequences: served in index order (no longest-first ordering).
    c = make_decode_case(3300, B=1100, Hq=4, Hkv=1, D=64, block_size=16, ctx_lo=1, ctx_hi=200,
                         cache_dtype="float16")
    check(c)


def test_masked_block_ids():
    c = make_decode_case(3400, B=128, Hq=8, Hkv=4, D=64, block_size=16, ctx_lo=64, ctx_hi=300,
                         cache_dtype="bfloat16")
    nb = c.k_cache.shape[0]
    c.block_tables[5, 1] = nb + 7      # outside the pool: its tokens are masked out
    c.block_tables[9, 0] = -5
    out = to_f64(run(c))
    ref = decode_oracle_masked(c, nb)
    a, r = tolerance(c.q_dtype, c.cache_dtype)
    np.testing.assert_allclose(out, ref, atol=a, rtol=r)


def decode_oracle_masked(c, nb):
    """Oracle with the tokens of out-of-pool blocks removed."""
    from oracle import pagedkv_oracle as orc
    B = c.q.shape[0]
    out = np.zeros(c.q.shape)
    q64 = orc.decode(c.q, c.q_dtype)
    kc, vc = orc.decode(c.k_cache, c.cache_dtype), orc.decode(c.v_cache, c.cache_dtype)
    for s in range(B):
        ctx = int(c.context_lens[s])
        t = np.arange(ctx)
        blk = c.block_tables[s][t // c.block_size]
        keep = (blk >= 0) & (blk < nb)
        if not keep.any():
            continue
        k = kc[blk[keep], :, :, (t % c.block_size)[keep], :].reshape(keep.sum(), c.num_kv_heads, -1)
        v = vc[blk[keep], :, :, (t % c.block_size)[keep]]
        out[s] = orc._softmax_attend(q64[s], k, v, c.scale, None)
    return out


def test_repeated_calls_are_bit_identical():
    c = make_decode_case(3500, B=128, Hq=8, Hkv=4, D=128, block_size=16, ctx_lo=100, ctx_hi=2000,
                         cache_dtype="bfloat16")
    first = run(c)
    outs = [run(c) for _ in range(4)]
    run(c, partition_size=256)         # split-K call sharing the workspace in between
    outs.append(run(c))
    for o in outs:
        assert torch.equal(o, first)
    a, r = tolerance(c.q_dtype, c.cache_dtype)
    np.testing.assert_allclose(to_f64(first), decode_oracle(c), atol=a, rtol=r)


@pytest.mark.parametrize("D", [64, 128])
def test_split_k_ignores_unwritten_workspace(D):
    # The merge reads its first step of partials before it knows a row's
    # partition count; entries a row did not write this call (its context is
    # shorter than max_seq_len) must not reach the output, even as NaN.
    from sglang_mlx_amd import _ext, _lib
    c = make_decode_case(3600 + D, B=3, Hq=8, Hkv=2, D=D, block_size=16, ctx_lo=300, ctx_hi=900,
                         cache_dtype="bfloat16", max_seq_len=4096)
    run(c, partition_size=256)                 # creates the cached workspace
    for scratch in list(_ext._ws_cache.values()):
        scratch[_lib.PKV_COUNTER_BYTES:].fill_(0xFF)  # every partition-state word a NaN (counters stay zero)
    torch.cuda.synchronize()
    for ps in (256, None):                     # split-K, and v1 (which splits these few rows too)
        out = run(c, partition_size=ps)
        a, r = tolerance(c.q_dtype, c.cache_dtype)
        np.testing.assert_allclose(to_f64(out), decode_oracle(c), atol=a, rtol=r)


@pytest.mark.parametrize("B", [32, 48, 63])
def test_one_to_two_items_per_workgroup(B):
    # Llama-3-8B heads: 256 to 504 (sequence, KV head) items over 256
    # workgroups, so some workgroups take one item and some two.
    c = make_decode_case(3700 + B, B=B, Hq=32, Hkv=8, D=128, block_size=16, ctx_lo=300, ctx_hi=3000,
                         cache_dtype="bfloat16")
    check(c)


@pytest.mark.parametrize("case", ["fused_b40", "fused_b1", "deep_b1"])
def test_fused_merge_leaves_counters_zero(case):
    # The partition kernel merges its own partitions when a row has at most
    # 8 (B40 at 2K: 512-token partitions, 4 per row; B1 at 1K: 4 of 256);
    # deeper rows (B1 at 40K: 80 partitions) take the merge kernel.  v1 and
    # v2 share the workspace; every call leaves the counter region zero, and
    # the results hold.
    from sglang_mlx_amd import _ext, _lib
    kw = dict(fused_b40=dict(seed=3800, B=40, Hq=8, Hkv=2, ctx_lo=1500, ctx_hi=2000),
              fused_b1=dict(seed=3801, B=1, Hq=28, Hkv=4, ctx_lo=1024, ctx_hi=1024),
              deep_b1=dict(seed=3802, B=1, Hq=28, Hkv=4, ctx_lo=40000, ctx_hi=40000))[case]
    c = make_decode_case(D=128, block_size=16, cache_dtype="bfloat16", **kw)
    outs = []
    for ps in (None, 512, None):
        outs.append(run(c, partition_size=ps))
        torch.cuda.synchronize()
        for scratch in _ext._ws_cache.values():
            assert int(scratch[:_lib.PKV_COUNTER_BYTES].count_nonzero()) == 0
    a, r = tolerance(c.q_dtype, c.cache_dtype)
    ref = decode_oracle(c)
    for out in outs:
        np.testing.assert_allclose(to_f64(out), ref, atol=a, rtol=r)
    assert torch.equal(outs[0], outs[2])  # the merge order does not depend on which workgroup merges
