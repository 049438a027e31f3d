"""Host side of the shared-prefix (cascade) decode: build_cascade_plan and
plan_prefix_groups (CPU only).

* Known answers on hand-made block tables: grouping by first block, the
  longest common run of leading blocks held in full by every member, groups
  of one and short prefixes dropped, tiles, chunk choice, tail partitions
  and their order.
* Invariants on random radix-shaped batches: every member maps the group's
  prefix to the first member's blocks; the tiles of a group cover its prefix
  [0, P) chunk by chunk for every member exactly once; member counts fit 128
  query rows; the tail partitions cover every sequence's tail [P, ctx)
  exactly once (one empty partition for an empty tail), longest first.
* The plan's meaning, restated in float64 with the oracle's partial
  softmax states: per tile, the member rows against the first member's
  blocks over [token_begin, token_end); per tail partition, its tokens over
  the sequence's own blocks; all merged by log-sum-exp.  This equals the
  oracle's paged_attention to float64 rounding on random batches, and a
  planted mistake in a plan (a prefix one block short, a member left out
  of its tiles, a tail partition left out) makes it differ.
"""

import numpy as np
import pytest

from oracle import pagedkv_oracle as orc
from sglang_mlx_amd.srt.mem_cache import build_cascade_plan, plan_prefix_groups, tail_partitions


def np_plan(plan):
    return dict(prefix_lens=plan.prefix_lens.numpy(), members=plan.members.numpy(), tiles=plan.tiles.numpy(),
                parts=plan.parts.numpy(), chunk=plan.chunk_tokens, max_chunks=plan.max_chunks,
                part_tokens=plan.part_tokens, max_parts=plan.max_parts)


def test_groups_known_answers():
    bt = np.array([[5, 6, 7, -1],
                   [5, 6, 9, 10],
                   [5, 6, 7, 11],
                   [3, 4, -1, -1],
                   [8, -1, -1, -1],
                   [3, 4, 12, -1],
                   [5, 13, -1, -1]], dtype=np.int32)
    ctx = np.array([40, 64, 50, 20, 10, 48, 30])
    g = plan_prefix_groups(bt, ctx, 16)
    # {0,1,2,6} share block 5 only (6 holds block 13 next); {3,5}: seq 3
    # holds one whole block (20 tokens), so their prefix is one block.
    assert [(m.tolist(), p) for m, p in g] == [([3, 5], 16), ([0, 1, 2, 6], 16)]
    # seq 6 out: {0, 1, 2} share two blocks
    g = plan_prefix_groups(bt[:6], ctx[:6], 16)
    assert [(m.tolist(), p) for m, p in g] == [([3, 5], 16), ([0, 1, 2], 32)]
    # (members - 1) * prefix: 16 for {3, 5}, 64 for {0, 1, 2}
    assert [(m.tolist(), p) for m, p in plan_prefix_groups(bt[:6], ctx[:6], 16, min_shared_tokens=40)] == \
        [([0, 1, 2], 32)]
    assert plan_prefix_groups(bt[:6], ctx[:6], 16, min_members=3)[0][1] == 32
    assert plan_prefix_groups(np.zeros((0, 4), np.int32), np.zeros(0), 16) == []


def test_plan_known_answers():
    bt = np.array([[5, 6, 7, -1], [5, 6, 9, 10], [5, 6, 7, 11], [3, 4, -1, -1], [8, -1, -1, -1]], dtype=np.int32)
    ctx = np.array([40, 64, 50, 20, 10])
    p = np_plan(build_cascade_plan(bt, ctx, 16, 32, 8))
    assert p["prefix_lens"].tolist() == [32, 32, 32, 0, 0]
    assert p["members"].tolist() == [0, 1, 2]
    assert p["tiles"].tolist() == [[0, 3, 0, 32]]
    assert p["chunk"] == 256 and p["max_chunks"] == 1
    # tails 8, 32, 18, 20, 10: one partition each, longest first, ties by index
    assert p["part_tokens"] == 512 and p["max_parts"] == 1
    assert p["parts"].tolist() == [[1, 0], [3, 0], [2, 0], [4, 0], [0, 0]]
    p = np_plan(build_cascade_plan(bt, ctx, 16, 32, 8, chunk_tokens=16, part_tokens=16))
    assert p["tiles"].tolist() == [[0, 3, 0, 16], [0, 3, 16, 32]] and p["max_chunks"] == 2
    # 16-token partitions: lengths 8 | 16 16 | 16 2 | 16 4 | 10
    assert p["max_parts"] == 2
    assert p["parts"].tolist() == [[1, 0], [1, 1], [2, 0], [3, 0], [4, 0], [0, 0], [3, 1], [2, 1]]
    for bad in (dict(chunk_tokens=24), dict(part_tokens=24), dict(part_tokens=2048), dict(part_tokens=0)):
        with pytest.raises(ValueError):
            build_cascade_plan(bt, ctx, 16, 32, 8, **bad)
    with pytest.raises(ValueError):
        build_cascade_plan(bt, ctx, 16, 30, 8)


def test_tail_partitions_known_answers():
    assert tail_partitions(np.array([0, 5, 64, 65]), 32).tolist() == \
        [[2, 0], [2, 1], [3, 0], [3, 1], [1, 0], [3, 2], [0, 0]]
    assert tail_partitions(np.array([], dtype=np.int64), 16).shape == (0, 2)
    assert tail_partitions(np.array([-3]), 16).tolist() == [[0, 0]]


def test_chunk_fills_the_cus():
    # 256 members x GQA 4 (8 row tiles) x 8 KV heads with a 2048-token
    # prefix: 512-token chunks give 8 x 4 x 8 = 256 workgroups.
    B, npb = 256, 128
    rng = np.random.default_rng(1)
    bt = np.full((B, npb + 40), -1, np.int32)
    bt[:, :npb] = np.arange(1, npb + 1)
    ctx = npb * 16 + rng.integers(64, 513, size=B)
    for s in range(B):
        n = -(-(ctx[s] - npb * 16) // 16)
        bt[s, npb:npb + n] = 1000 + 40 * s + np.arange(n)
    p = np_plan(build_cascade_plan(bt, ctx, 16, 32, 8))
    assert p["chunk"] == 512 and p["max_chunks"] == 4 and p["tiles"].shape[0] == 32
    assert (p["tiles"][:, 1] == 32).all()
    p = np_plan(build_cascade_plan(bt, ctx, 16, 28, 4))  # GQA 7: 18 members per tile
    assert (p["tiles"][:, 1] <= 18).all() and p["tiles"][:, 1].max() == 18


def radix_batch(rng, B, bs, groups, pool_extra=50):
    """Random radix-shaped batch: groups [(members, prefix blocks)], then
    unshared sequences; private suffixes of random length."""
    owner = []
    for gi, (m, _) in enumerate(groups):
        owner += [gi] * m
    owner += [-1] * (B - len(owner))
    owner = rng.permutation(np.array(owner))
    nxt = 1
    gblocks = []
    for _, nbk in groups:
        gblocks.append(list(range(nxt, nxt + nbk)))
        nxt += nbk
    pre = np.array([len(gblocks[o]) * bs if o >= 0 else 0 for o in owner])
    ctx = pre + rng.integers(1, 5 * bs, size=B)
    width = int((-(-ctx // bs)).max())
    bt = np.full((B, width), -1, np.int32)
    for s in range(B):
        head = gblocks[owner[s]] if owner[s] >= 0 else []
        n = -(-ctx[s] // bs)
        bt[s, :len(head)] = head
        bt[s, len(head):n] = np.arange(nxt, nxt + n - len(head))
        nxt += n - len(head)
    return bt, ctx.astype(np.int32), nxt + pool_extra


@pytest.mark.parametrize("seed", range(6))
def test_plan_invariants(seed):
    rng = np.random.default_rng(100 + seed)
    bs = [8, 16, 32][seed % 3]
    bt, ctx, _ = radix_batch(rng, 90, bs, [(30, 7), (2, 3), (40, 20), (1, 4)])
    Hq, Hkv = [(32, 8), (28, 4), (8, 8)][seed % 3]
    p = np_plan(build_cascade_plan(bt, ctx, bs, Hq, Hkv, num_cus=64))
    group = Hq // Hkv
    B = bt.shape[0]
    tail = ctx - p["prefix_lens"]
    P = p["part_tokens"]
    assert P % 16 == 0 and P % bs == 0
    seen = {}
    lengths = []
    for s_, k in p["parts"].tolist():
        seen.setdefault(s_, []).append(k)
        lengths.append(min(P, tail[s_] - k * P))
    for s_ in range(B):
        n = max(1, -(-int(tail[s_]) // P))
        assert sorted(seen[s_]) == list(range(n)) and n <= p["max_parts"]
    assert (np.diff(lengths) <= 0).all()
    assert p["chunk"] % 16 == 0 and p["chunk"] % bs == 0
    covered = {}
    for mb, mc, t0, t1 in p["tiles"].tolist():
        assert 0 < mc and mc * group <= 128 and t0 % p["chunk"] == 0 and 0 < t1 - t0 <= p["chunk"]
        mem = p["members"][mb:mb + mc]
        first = mem[0]
        for s in mem:
            P = p["prefix_lens"][s]
            assert t1 <= P <= ctx[s] and P % bs == 0
            nbk = -(-t1 // bs)
            assert (bt[s, :nbk] == bt[first, :nbk]).all()
            covered.setdefault(int(s), []).append((t0, t1))
    for s in range(B):
        P = int(p["prefix_lens"][s])
        spans = sorted(covered.get(s, []))
        if P == 0:
            assert not spans
            continue
        assert spans[0][0] == 0 and spans[-1][1] == P
        assert all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
        assert -(-P // p["chunk"]) <= p["max_chunks"]


def cascade_restated(q, kc, vc, bt, ctx, Hkv, scale, bs, max_seq_len, plan, alibi=None):
    """The two passes the plan describes, in float64: prefix partials per
    tile (rows of its members, tokens [t0, min(t1, ctx)) from the first
    member's blocks), the tail [prefix, ctx) from each sequence's own blocks,
    log-sum-exp merged.  q, kc, vc: float64 values."""
    B, Hq, D = q.shape
    parts = {s: [] for s in range(B)}
    for mb, mc, t0, t1 in plan["tiles"].tolist():
        mem = plan["members"][mb:mb + mc]
        first = int(mem[0])
        for s in mem.tolist():
            c = int(ctx[s])
            if c == 0 or c > max_seq_len:
                continue
            hi = min(t1, c)
            if hi <= t0:
                continue
            k, v = orc.gather_kv(kc, vc, bt[first], hi)
            bias = None if alibi is None else orc.alibi_bias(alibi, c)
            parts[s].append(orc.partition_stats(q[s], k, v, scale, bias, t0, hi))
    out = np.zeros_like(q)
    for s, kp in plan["parts"].tolist():
        c = int(ctx[s])
        if c == 0 or c > max_seq_len:
            continue
        P = min(int(plan["prefix_lens"][s]), c)
        lo = P + kp * plan["part_tokens"]
        hi = min(c, lo + plan["part_tokens"])
        if lo < hi:
            k, v = orc.gather_kv(kc, vc, bt[s], c)
            bias = None if alibi is None else orc.alibi_bias(alibi, c)
            parts[s].append(orc.partition_stats(q[s], k, v, scale, bias, lo, hi))
    for s in range(B):
        c = int(ctx[s])
        if c == 0 or c > max_seq_len:
            continue
        ps = parts[s]
        out[s] = orc.lse_merge(np.stack([x[0] for x in ps]), np.stack([x[1] for x in ps]),
                               np.stack([x[2] for x in ps]))
    return out


def restated_case(seed, bs=16, Hq=8, Hkv=2, D=32, alibi=False):
    rng = np.random.default_rng(seed)
    bt, ctx, nb = radix_batch(rng, 24, bs, [(9, 5), (4, 2), (6, 9)])
    x = 4
    kc = rng.standard_normal((nb, Hkv, D // x, bs, x))
    vc = rng.standard_normal((nb, Hkv, D, bs))
    q = rng.standard_normal((bt.shape[0], Hq, D))
    slopes = rng.uniform(0.01, 0.2, size=Hq) if alibi else None
    return q, kc, vc, bt, ctx, Hkv, 1 / np.sqrt(D), bs, bt.shape[1] * bs, slopes


@pytest.mark.parametrize("seed,bs,alibi,chunk,part", [(1, 16, False, None, None), (2, 8, True, 16, 16),
                                                     (3, 32, False, 32, 32)])
def test_plan_restated_equals_single_softmax(seed, bs, alibi, chunk, part):
    q, kc, vc, bt, ctx, Hkv, scale, bs, msl, slopes = restated_case(seed, bs=bs, alibi=alibi)
    ctx[3] = 0
    plan = np_plan(build_cascade_plan(bt, ctx, bs, q.shape[1], Hkv, chunk_tokens=chunk, part_tokens=part))
    if part is not None:
        assert plan["max_parts"] > 1
    assert plan["tiles"].shape[0] > 0
    got = cascade_restated(q, kc, vc, bt, ctx, Hkv, scale, bs, msl, plan, slopes)
    exp = orc.paged_attention(q.astype(np.float32), kc.astype(np.float32), vc.astype(np.float32), bt, ctx, Hkv,
                              scale, bs, msl, slopes)
    # float32 inputs on the oracle side: compare against the same values
    got32 = cascade_restated(q.astype(np.float32).astype(np.float64), kc.astype(np.float32).astype(np.float64),
                             vc.astype(np.float32).astype(np.float64), bt, ctx, Hkv, scale, bs, msl, plan, slopes)
    np.testing.assert_allclose(got32, exp, atol=1e-12, rtol=1e-10)
    assert got.shape == exp.shape


def test_planted_plan_mistakes_are_caught():
    q, kc, vc, bt, ctx, Hkv, scale, bs, msl, slopes = restated_case(4)
    q, kc, vc = (a.astype(np.float32).astype(np.float64) for a in (q, kc, vc))
    plan = np_plan(build_cascade_plan(bt, ctx, bs, q.shape[1], Hkv))
    exp = orc.paged_attention(q, kc, vc, bt, ctx, Hkv, scale, bs, msl)
    np.testing.assert_allclose(cascade_restated(q, kc, vc, bt, ctx, Hkv, scale, bs, msl, plan), exp,
                               atol=1e-12, rtol=1e-10)
    # a prefix one block short in one member: its tail re-counts a block
    bad = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in plan.items()}
    s = int(bad["members"][0])
    bad["prefix_lens"][s] -= bs
    assert not np.allclose(cascade_restated(q, kc, vc, bt, ctx, Hkv, scale, bs, msl, bad)[s], exp[s], atol=1e-6)
    # a member left out of its group's tiles: its prefix is never counted
    bad = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in plan.items()}
    t = bad["tiles"][0].copy()
    bad["tiles"][0] = (t[0] + 1, t[1] - 1, t[2], t[3])
    s = int(plan["members"][t[0]])
    assert not np.allclose(cascade_restated(q, kc, vc, bt, ctx, Hkv, scale, bs, msl, bad)[s], exp[s], atol=1e-6)
    # a tail partition left out: its tokens are never counted
    plan = np_plan(build_cascade_plan(bt, ctx, bs, q.shape[1], Hkv, part_tokens=16))
    np.testing.assert_allclose(cascade_restated(q, kc, vc, bt, ctx, Hkv, scale, bs, msl, plan), exp,
                               atol=1e-12, rtol=1e-10)
    bad = dict(plan)
    s, k = plan["parts"][0]
    assert k >= 0 and (plan["parts"][:, 0] == s).sum() > 1
    bad["parts"] = plan["parts"][1:]
    assert not np.allclose(cascade_restated(q, kc, vc, bt, ctx, Hkv, scale, bs, msl, bad)[s], exp[s], atol=1e-6)
