"""GPU parity of the shared-prefix (cascade) decode, paged_attention_cascade,
against the oracle and against paged_attention_v1 on the same inputs.

The plan comes from the host's block tables (build_cascade_plan): a prefix
pass attends every member's query rows to each group's shared blocks, a tail
pass streams each sequence's remaining tokens in partitions, and a merge
folds the partial states.  Cases: one group of 256 (the radix-shared shape),
several groups with different prefixes plus unshared sequences, prefixes
split into many chunks (more than four per row: the merge folds them four at
a time), tails in many partitions (16-token partitions, 2600-token tails)
and in one (1024-token partitions), sequences without a prefix over several
partitions, empty and over-long contexts, block ids outside the pool inside
a shared prefix, ALiBi, block sizes 8/16/32, head sizes 64/128, GQA
1/2/4/7/8, float16 and bfloat16 queries, FP8 E4M3 caches with k_scale /
v_scale, shapes the cascade kernels leave to the one-pass decode (float32
query, head size 96), and repeated calls (bit-identical)."""

import math

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from pkv_cases import X_OF, normal, tolerance
from pkv_torch import to_f64, to_index, to_torch
from sglang_mlx_amd import kernels
from sglang_mlx_amd.srt.mem_cache import build_cascade_plan
from test_gpu_grouped import FP8, FP8_TOL, expected_masked, fp8_radix_case, radix_case

pytestmark = pytest.mark.gpu


def groups_case(seed, groups, unshared, Hq=32, Hkv=8, D=128, bs=16, dtype="bfloat16", q_dtype=None,
                suffix=(1, 300), alibi=False):
    """``groups``: [(members, prefix tokens)]; each group's members share its
    prefix blocks (whole blocks), then hold private suffixes; ``unshared``
    more sequences hold private blocks only.  Sequences are interleaved."""
    rng = np.random.default_rng(seed)
    q_dtype = q_dtype or dtype
    owner = []
    for gi, (m, _) in enumerate(groups):
        owner += [gi] * m
    owner += [-1] * unshared
    owner = rng.permutation(np.array(owner))
    B = owner.size
    pre = np.array([groups[o][1] if o >= 0 else 0 for o in owner])
    ctx = (pre + rng.integers(suffix[0], suffix[1] + 1, size=B)).astype(np.int32)
    nblk = -(-ctx // bs)
    gblk = [-(-p // bs) for _, p in groups]
    nb = int(sum(gblk) + (nblk - np.array([gblk[o] if o >= 0 else 0 for o in owner])).sum() + 2)
    perm = iter(rng.permutation(np.arange(1, nb)).tolist())
    gids = [[next(perm) for _ in range(n)] for n in gblk]
    bt = np.full((B, int(nblk.max())), -1, dtype=np.int32)
    for s in range(B):
        head = gids[owner[s]] if owner[s] >= 0 else []
        bt[s, :len(head)] = head
        for j in range(len(head), nblk[s]):
            bt[s, j] = next(perm)
    x = X_OF[dtype]
    kc = normal(rng, (nb, Hkv, D // x, bs, x), dtype)
    vc = normal(rng, (nb, Hkv, D, bs), dtype)
    q = normal(rng, (B, Hq, D), q_dtype)
    slopes = rng.uniform(0.01, 0.2, size=Hq).astype(np.float32) if alibi else None
    return dict(q=q, kc=kc, vc=vc, bt=bt, ctx=ctx, Hkv=Hkv, bs=bs, dt=dtype, qd=q_dtype, alibi=slopes,
                scale=1.0 / math.sqrt(D))


def plan_of(c, **kw):
    Hq = c["q"].shape[1]
    return build_cascade_plan(c["bt"], c["ctx"], c["bs"], Hq, c["Hkv"], device="cuda", **kw)


def run_cascade(c, plan, fp8=False):
    alibi = None if c["alibi"] is None else torch.from_numpy(c["alibi"]).cuda()
    dt = FP8 if fp8 else c["dt"]
    scales = dict(k_scale=c["ks"], v_scale=c["vs"]) if fp8 else {}
    out = kernels.paged_attention_cascade(to_torch(c["q"], c["qd"]), to_torch(c["kc"], dt), to_torch(c["vc"], dt),
                                          to_index(c["bt"]), to_index(c["ctx"]), c["Hkv"], c["scale"], c["bs"],
                                          int(c["bt"].shape[1] * c["bs"]), plan, alibi, **scales)
    torch.cuda.synchronize()
    return out


def oracle(c, fp8=False):
    extra = dict(cache_dtype=FP8, k_scale=c["ks"], v_scale=c["vs"]) if fp8 else dict(cache_dtype=c["dt"])
    return orc.paged_attention(c["q"], c["kc"], c["vc"], c["bt"], c["ctx"], c["Hkv"], c["scale"], c["bs"],
                               int(c["bt"].shape[1] * c["bs"]), c["alibi"], q_dtype=c["qd"], **extra)


def check(c, plan=None, fp8=False, **kw):
    plan = plan if plan is not None else plan_of(c, **kw)
    got = to_f64(run_cascade(c, plan, fp8))
    a, r = FP8_TOL[c["qd"]] if fp8 else tolerance(c["qd"], c["dt"])
    np.testing.assert_allclose(got, oracle(c, fp8), atol=a, rtol=r)
    return plan, got


@pytest.mark.parametrize("prefix", [2048, 256, 250])
def test_one_group_of_256(prefix):
    c = radix_case(7000 + prefix, B=256, Hq=32, Hkv=8, D=128, bs=16, prefix_tokens=prefix, suffix_lo=64,
                   suffix_hi=512)
    plan, _ = check(c)
    assert len(plan.groups) == 1 and plan.groups[0][0].size == 256 and plan.tiles.shape[0] > 0


def test_several_groups_and_unshared():
    c = groups_case(7100, [(40, 512), (3, 64), (100, 1024), (1, 320)], unshared=37)
    plan, _ = check(c)
    assert sorted(p for _, p in plan.groups) == [64, 512, 1024]


@pytest.mark.parametrize("chunk", [16, 64])
def test_many_chunks_per_row(chunk):
    # 1024-token prefix in 16- and 64-token chunks: 64 / 16 partials per row
    c = groups_case(7200 + chunk, [(50, 1024), (20, 272)], unshared=5, D=64, dtype="float16")
    plan, _ = check(c, chunk_tokens=chunk)
    assert plan.max_chunks == 1024 // chunk


def test_empty_overlong_and_masked():
    c = radix_case(7300, B=200, Hq=32, Hkv=8, D=64, bs=16, prefix_tokens=512, suffix_lo=1, suffix_hi=100,
                   dtype="float16")
    c["ctx"][[3, 77, 150]] = 0
    c["ctx"][120] = c["bt"].shape[1] * 16 + 5   # past max_seq_len: zero row
    c["bt"][:, 2] = -1                           # a shared block masked out in every sequence
    plan = plan_of(c)
    assert plan.groups and plan.groups[0][1] >= 3 * 16
    c2 = dict(c)
    got = to_f64(run_cascade(c2, plan))
    np.testing.assert_allclose(got, expected_masked(c), atol=2e-3, rtol=1e-2)
    assert not got[[3, 77, 120, 150]].any()


@pytest.mark.parametrize("bs", [8, 32])
def test_block_sizes_and_alibi(bs):
    check(groups_case(7400 + bs, [(60, 384), (70, 96)], unshared=10, bs=bs, alibi=True))


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (28, 4), (64, 8)])  # GQA 1, 2, 7, 8
def test_group_sizes(Hq, Hkv):
    check(groups_case(7500 + Hq, [(80, 320), (30, 160)], unshared=6, Hq=Hq, Hkv=Hkv, D=128))


@pytest.mark.parametrize("q_dtype,D", [("float16", 128), ("float16", 64), ("bfloat16", 64)])
def test_query_types_head_sizes(q_dtype, D):
    check(groups_case(7600 + D, [(90, 512)], unshared=20, D=D, dtype=q_dtype))


@pytest.mark.parametrize("bs", [8, 16, 32])
def test_fp8_one_group(bs):
    c = fp8_radix_case(7700 + bs, D=128, bs=bs, q_dtype="bfloat16", prefix_tokens=512, suffix_hi=300)
    check(c, fp8=True)


@pytest.mark.parametrize("q_dtype,D", [("float16", 128), ("bfloat16", 64), ("float16", 64)])
def test_fp8_query_types_head_sizes(q_dtype, D):
    c = fp8_radix_case(7800 + D, D=D, bs=16, q_dtype=q_dtype, prefix_tokens=320, suffix_hi=200)
    check(c, fp8=True)


@pytest.mark.parametrize("q_dtype,D,tail", [("float32", 128, 300), ("bfloat16", 96, 300)])
def test_shapes_left_to_the_one_pass_decode(q_dtype, D, tail):
    c = radix_case(7900 + D, B=64, Hq=32, Hkv=8, D=D, bs=16, prefix_tokens=256, suffix_lo=tail - 100,
                   suffix_hi=tail, dtype="bfloat16", q_dtype=q_dtype)
    plan, got = check(c)
    ref = kernels.paged_attention_v1(to_torch(c["q"], c["qd"]), to_torch(c["kc"], c["dt"]),
                                     to_torch(c["vc"], c["dt"]), to_index(c["bt"]), to_index(c["ctx"]), c["Hkv"],
                                     c["scale"], c["bs"], int(c["bt"].shape[1] * c["bs"]))
    np.testing.assert_array_equal(got, to_f64(ref))  # the same kernels ran


@pytest.mark.parametrize("part", [None, 16, 1024])
def test_long_tails_in_partitions(part):
    c = radix_case(7950, B=64, Hq=32, Hkv=8, D=128, bs=16, prefix_tokens=256, suffix_lo=2500, suffix_hi=2600)
    plan, _ = check(c, part_tokens=part)
    assert plan.max_parts == -(-int((c["ctx"] - 256).max()) // plan.part_tokens)


@pytest.mark.parametrize("part", [None, 32])
def test_no_groups_is_plain_tail_decode(part):
    # no prefix anywhere: rows of one partition are written by the tail
    # pass, longer ones by the merge
    c = groups_case(8000, [], unshared=300, suffix=(1, 700))
    plan, _ = check(c, part_tokens=part)
    assert plan.tiles.shape[0] == 0 and plan.max_parts > 1


def test_very_short_tails():
    # tails of 1-8 tokens behind a 2048-token prefix
    c = radix_case(8050, B=128, Hq=32, Hkv=8, D=128, bs=16, prefix_tokens=2048, suffix_lo=1, suffix_hi=8)
    check(c)


def test_repeat_calls_are_bit_identical():
    c = groups_case(8100, [(128, 768), (64, 256)], unshared=64)
    plan = plan_of(c)
    a = to_f64(run_cascade(c, plan))
    # another call on the same workspace in between, with other shapes
    check(groups_case(8101, [(32, 128)], unshared=8, D=64))
    b = to_f64(run_cascade(c, plan))
    np.testing.assert_array_equal(a, b)


def test_matches_v1_on_the_radix_shape():
    c = radix_case(8200, B=256, Hq=32, Hkv=8, D=128, bs=16, prefix_tokens=2048, suffix_lo=64, suffix_hi=512)
    got = to_f64(run_cascade(c, plan_of(c)))
    ref = kernels.paged_attention_v1(to_torch(c["q"], c["qd"]), to_torch(c["kc"], c["dt"]),
                                     to_torch(c["vc"], c["dt"]), to_index(c["bt"]), to_index(c["ctx"]), c["Hkv"],
                                     c["scale"], c["bs"], int(c["bt"].shape[1] * c["bs"]))
    np.testing.assert_allclose(got, to_f64(ref), atol=1e-2, rtol=2e-2)
