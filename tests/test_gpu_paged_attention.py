"""GPU parity of paged_attention_v1 / v2 against the float64 oracle.

Tolerances (written per case through pkv_cases.tolerance): float16
2e-3 abs / 1e-2 rel, bfloat16 1e-2 abs / 2e-2 rel.

Cases transplanted from the reference's kernel tests
(tests/test_paged_attention_kernel.py:212-378): the two-sequence fixture,
the head-dim x block-size sweep, a 2112-token context, zero output for an
empty context and for context > max_seq_len.  Then the decode workloads:
tiny fp16 (B4, 32/8 heads, D64), Llama-3-8B layer at full size (B64, 32/8,
D128, ctx U[512,4096], bf16), every head size x block size, GQA groups of
1, 4, 7 and 32, ALiBi, split-K partitions, and determinism across calls
sharing one workspace.
"""

import math

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from pkv_cases import decode_oracle, make_decode_case, tolerance
from pkv_torch import to_f64, to_index, to_torch
from sglang_mlx_amd import _ext

pytestmark = pytest.mark.gpu


def run_case(c, partition_size=None):
    args = (to_torch(c.q, c.q_dtype), to_torch(c.k_cache, c.cache_dtype), to_torch(c.v_cache, c.cache_dtype),
            to_index(c.block_tables), to_index(c.context_lens), c.num_kv_heads, c.scale, c.block_size,
            c.max_seq_len, None if c.alibi is None else torch.from_numpy(c.alibi).cuda())
    if partition_size is None:
        out = _ext.paged_attention_v1(*args)
    else:
        out = _ext.paged_attention_v2(*args, partition_size=partition_size)
    torch.cuda.synchronize()
    assert out.dtype == args[0].dtype and tuple(out.shape) == tuple(c.q.shape)
    return out


def check(c, partition_size=None, atol=None, rtol=None):
    out = to_f64(run_case(c, partition_size))
    ref = decode_oracle(c)
    a, r = tolerance(c.q_dtype, c.cache_dtype)
    np.testing.assert_allclose(out, ref, atol=atol or a, rtol=rtol or r)
    return out, ref


def test_reference_fixture():
    # test_paged_attention_kernel.py:138-246: 2 seqs, 8 q / 4 kv heads, D 64,
    # bs 16, contexts 25 and 50, tables [[0,1,-1,-1],[2,3,4,5]], float32
    # query over a float16 cache filled from float32 K/V, max_seq_len 64.
    rng = np.random.default_rng(101)
    q = rng.standard_normal((2, 8, 64), dtype=np.float32)
    k = rng.standard_normal((75, 4, 64), dtype=np.float32)
    v = rng.standard_normal((75, 4, 64), dtype=np.float32)
    slots = np.array(list(range(25)) + [32 + i for i in range(50)], dtype=np.int32)
    kc = torch.zeros((20, 4, 8, 16, 8), dtype=torch.float16, device="cuda")
    vc = torch.zeros((20, 4, 64, 16), dtype=torch.float16, device="cuda")
    kc, vc = _ext.reshape_and_cache(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), kc, vc,
                                    torch.from_numpy(slots).cuda())
    bt = torch.tensor([[0, 1, -1, -1], [2, 3, 4, 5]], dtype=torch.int32, device="cuda")
    lens = torch.tensor([25, 50], dtype=torch.int32, device="cuda")
    out = _ext.paged_attention_v1(torch.from_numpy(q).cuda(), kc, vc, bt, lens, 4, 1.0 / math.sqrt(64), 16, 64)
    torch.cuda.synchronize()
    kc_np = kc.cpu().view(torch.int16).numpy().view(np.uint16)
    vc_np = vc.cpu().view(torch.int16).numpy().view(np.uint16)
    ref = orc.paged_attention(q, kc_np, vc_np, bt.cpu().numpy(), lens.cpu().numpy(), 4, 1.0 / 8.0, 16, 64,
                              None, "float32", "float16")
    got = out.cpu().double().numpy()
    np.testing.assert_allclose(got, ref, atol=5e-3)           # the reference test's bar
    np.testing.assert_allclose(got, ref, atol=2e-3, rtol=1e-2)  # the float16 bar


@pytest.mark.parametrize("head_dim", [32, 128])
@pytest.mark.parametrize("block_size", [8, 16])
def test_reference_shape_sweep(head_dim, block_size):
    # test_paged_attention_kernel.py:248-282.
    rng = np.random.default_rng(7 + head_dim + block_size)
    q = rng.standard_normal((1, 4, head_dim), dtype=np.float32)
    k = rng.standard_normal((16, 2, head_dim), dtype=np.float32)
    v = rng.standard_normal((16, 2, head_dim), dtype=np.float32)
    kc = torch.zeros((4, 2, head_dim // 8, block_size, 8), dtype=torch.float16, device="cuda")
    vc = torch.zeros((4, 2, head_dim, block_size), dtype=torch.float16, device="cuda")
    _ext.reshape_and_cache(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), kc, vc,
                           torch.arange(16, dtype=torch.int32, device="cuda"))
    bt = torch.tensor([[0, 1, -1, -1] if block_size == 8 else [0, -1, -1, -1]], dtype=torch.int32,
                      device="cuda")
    lens = torch.tensor([16], dtype=torch.int32, device="cuda")
    scale = 1.0 / math.sqrt(head_dim)
    out = _ext.paged_attention_v1(torch.from_numpy(q).cuda(), kc, vc, bt, lens, 2, scale, block_size, 16)
    ref = orc.paged_attention(q, kc.cpu().view(torch.int16).numpy().view(np.uint16),
                              vc.cpu().view(torch.int16).numpy().view(np.uint16), bt.cpu().numpy(),
                              lens.cpu().numpy(), 2, scale, block_size, 16, None, "float32", "float16")
    np.testing.assert_allclose(out.cpu().double().numpy(), ref, atol=2e-3, rtol=1e-2)


def test_context_longer_than_legacy_2048_limit():
    # test_paged_attention_kernel.py:284-330: D 32, bs 16, 2112 tokens,
    # 2 q heads over 1 kv head, unsigned tables and lengths.
    c = make_decode_case(2112, B=1, Hq=2, Hkv=1, D=32, block_size=16, ctx_lo=2112, ctx_hi=2112,
                         cache_dtype="float16", q_dtype="float32")
    check(c)


def test_empty_context_returns_zero():
    c = make_decode_case(5, B=1, Hq=2, Hkv=1, D=32, block_size=16, ctx_lo=16, ctx_hi=16,
                         cache_dtype="float16", q_dtype="float32", max_seq_len=16)
    c.context_lens[:] = 0
    out = run_case(c)
    assert torch.count_nonzero(out).item() == 0


def test_context_over_max_seq_len_returns_zero():
    c = make_decode_case(6, B=2, Hq=2, Hkv=1, D=32, block_size=16, ctx_lo=16, ctx_hi=16,
                         cache_dtype="float16", q_dtype="float32", max_seq_len=8)
    out = run_case(c)
    assert torch.count_nonzero(out).item() == 0


def test_tiny_fp16_workload():
    # B4, 32 q / 8 kv heads, D64, bs16, ctx U[64,512], fp16, 256-block pool.
    c = make_decode_case(1001, B=4, Hq=32, Hkv=8, D=64, block_size=16, ctx_lo=64, ctx_hi=512,
                         cache_dtype="float16", num_blocks=256)
    check(c)


def test_llama3_8b_layer_full_size():
    # B64, 32 q / 8 kv heads (GQA 4), D128, bs16, ctx U[512,4096], bf16,
    # non-overlapping permuted tables over a pool of 1.1x the needed blocks.
    c = make_decode_case(1003, B=64, Hq=32, Hkv=8, D=128, block_size=16, ctx_lo=512, ctx_hi=4096,
                         cache_dtype="bfloat16", max_seq_len=4096)
    check(c)


@pytest.mark.parametrize("head_dim", [32, 64, 80, 96, 112, 120, 128, 192, 256])
@pytest.mark.parametrize("block_size", [8, 16, 32])
def test_head_and_block_sizes(head_dim, block_size):
    c = make_decode_case(head_dim * 10 + block_size, B=3, Hq=8, Hkv=2, D=head_dim, block_size=block_size,
                         ctx_lo=1, ctx_hi=700, cache_dtype="bfloat16")
    check(c)


@pytest.mark.parametrize("q_dtype,cache_dtype", [("bfloat16", "bfloat16"), ("float16", "float16"),
                                                 ("float32", "bfloat16"), ("float32", "float16")])
def test_dtype_pairs(q_dtype, cache_dtype):
    c = make_decode_case(77, B=5, Hq=16, Hkv=4, D=128, block_size=16, ctx_lo=1, ctx_hi=1500,
                         cache_dtype=cache_dtype, q_dtype=q_dtype)
    check(c)


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (28, 4), (32, 1), (40, 2)])
def test_gqa_groups(Hq, Hkv):
    c = make_decode_case(Hq * 3 + Hkv, B=4, Hq=Hq, Hkv=Hkv, D=128, block_size=16, ctx_lo=100, ctx_hi=1300,
                         cache_dtype="bfloat16")
    check(c)


def test_alibi():
    c = make_decode_case(91, B=4, Hq=8, Hkv=2, D=64, block_size=16, ctx_lo=1, ctx_hi=900,
                         cache_dtype="float16", alibi=True)
    check(c)


@pytest.mark.parametrize("partition_size", [16, 64, 256, 512, 1024, 2048, 4096])
def test_split_k_partitions(partition_size):
    c = make_decode_case(500 + partition_size, B=3, Hq=28, Hkv=4, D=128, block_size=16, ctx_lo=1,
                         ctx_hi=5000, cache_dtype="bfloat16")
    check(c, partition_size=partition_size)


def test_split_k_long_context_qwen2():
    # Qwen2-7B shape (28 q / 4 kv heads, GQA 7), 32K context, 512-token
    # partitions (64 of them, two merge levels).
    c = make_decode_case(1004, B=1, Hq=28, Hkv=4, D=128, block_size=16, ctx_lo=32768, ctx_hi=32768,
                         cache_dtype="bfloat16")
    check(c, partition_size=512)
    check(c)


def test_v1_long_context_matches_split_k():
    # Four Qwen2-7B sequences at 64K: v1 picks 4096-token partitions (16 of
    # them per sequence).  The merged result does not depend on how the context
    # is partitioned, so v1 must match v2 with 512-token partitions (which the
    # oracle pins at smaller sizes) up to float32 summation order and bf16
    # rounding.  Inputs are generated on the GPU (537 MB of KV).
    B, Hq, Hkv, D, bs, ctx = 4, 28, 4, 128, 16, 65536
    g = torch.Generator(device="cuda")
    g.manual_seed(1007)
    nblk = ctx // bs
    nb = B * nblk + 1
    q = torch.randn((B, Hq, D), generator=g, device="cuda").to(torch.bfloat16)
    kc = torch.randn((nb, Hkv, D // 8, bs, 8), generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn((nb, Hkv, D, bs), generator=g, device="cuda").to(torch.bfloat16)
    perm = torch.randperm(nb - 1, generator=torch.Generator().manual_seed(1007)) + 1
    bt = perm.reshape(B, nblk).to(torch.int32).cuda()
    lens = torch.full((B,), ctx, dtype=torch.int32, device="cuda")
    args = (q, kc, vc, bt, lens, Hkv, 1.0 / math.sqrt(D), bs, ctx)
    v1 = _ext.paged_attention_v1(*args)
    v2 = _ext.paged_attention_v2(*args, partition_size=512)
    torch.cuda.synchronize()
    np.testing.assert_allclose(v1.float().cpu().numpy(), v2.float().cpu().numpy(), atol=1e-2, rtol=2e-2)
    assert torch.isfinite(v1.float()).all()


def test_radix_shared_prefix_tables():
    # Every table starts with the same 8 blocks (128 tokens), then private blocks.
    c = make_decode_case(1005, B=16, Hq=32, Hkv=8, D=128, block_size=16, ctx_lo=128 + 64, ctx_hi=128 + 512,
                         cache_dtype="bfloat16", shared_prefix_blocks=8)
    assert (c.block_tables[:, :8] == c.block_tables[0, :8]).all()
    check(c)


def test_repeat_calls_are_bit_identical():
    c = make_decode_case(1006, B=8, Hq=32, Hkv=8, D=128, block_size=16, ctx_lo=600, ctx_hi=3000,
                         cache_dtype="bfloat16")
    outs = [run_case(c) for _ in range(3)] + [run_case(c, partition_size=256) for _ in range(2)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
    assert torch.equal(outs[3], outs[4])
