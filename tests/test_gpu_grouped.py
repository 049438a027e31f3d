"""GPU parity of the grouped persistent decode (items of four sequences whose
query heads share one MFMA; tiles that all four map to the same blocks are
loaded once) against the oracle.  The launcher picks it when a batch gives
at least two such items per resident workgroup (here 256 sequences x 8 KV
heads and up) with GQA groups of at most 4 and contexts up to 8192 tokens.
Cases: radix-shared prefixes (whole and partially filled last blocks),
unshared batches, partial groups, empty and over-long contexts, masked
block ids, ALiBi, MHA and GQA 2, block sizes 8/16/32, fp16 and float32
queries (also with 8-token blocks at head size 128), FP8 E4M3 caches with
k_scale / v_scale, and more than 1024 sequences (no longest-first order)."""

import math

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from pkv_cases import X_OF, normal, tolerance
from pkv_torch import to_f64, to_index, to_torch
from sglang_mlx_amd import kernels

pytestmark = pytest.mark.gpu


def radix_case(seed, B, Hq, Hkv, D, bs, prefix_tokens, suffix_lo, suffix_hi, dtype="bfloat16", q_dtype=None,
               share=True, alibi=False):
    """Every sequence starts with the same prefix blocks (when share), then
    private blocks; the pool holds random values everywhere."""
    rng = np.random.default_rng(seed)
    q_dtype = q_dtype or dtype
    npb = -(-prefix_tokens // bs)
    ctx = (prefix_tokens + rng.integers(suffix_lo, suffix_hi + 1, size=B)).astype(np.int32)
    nblk = -(-ctx // bs)
    private = nblk - (npb if share else 0)
    nb = int(private.sum() + npb + 2)
    perm = rng.permutation(np.arange(1, nb))
    prefix_ids = perm[:npb]
    pos = npb
    width = int(nblk.max())
    bt = np.full((B, width), -1, dtype=np.int32)
    for s in range(B):
        if share:
            bt[s, :npb] = prefix_ids
            bt[s, npb:nblk[s]] = perm[pos:pos + private[s]]
        else:
            bt[s, :nblk[s]] = perm[pos:pos + private[s]]
        pos += private[s]
    x = X_OF[dtype]
    kc = normal(rng, (nb, Hkv, D // x, bs, x), dtype)
    vc = normal(rng, (nb, Hkv, D, bs), dtype)
    q = normal(rng, (B, Hq, D), q_dtype)
    slopes = rng.uniform(0.01, 0.2, size=Hq).astype(np.float32) if alibi else None
    return dict(q=q, kc=kc, vc=vc, bt=bt, ctx=ctx, Hkv=Hkv, bs=bs, dt=dtype, qd=q_dtype, alibi=slopes,
                scale=1.0 / math.sqrt(D))


def run(c):
    alibi = None if c["alibi"] is None else torch.from_numpy(c["alibi"]).cuda()
    out = kernels.paged_attention_v1(to_torch(c["q"], c["qd"]), to_torch(c["kc"], c["dt"]), to_torch(c["vc"], c["dt"]),
                                     to_index(c["bt"]), to_index(c["ctx"]), c["Hkv"], c["scale"], c["bs"],
                                     int(c["bt"].shape[1] * c["bs"]), alibi)
    torch.cuda.synchronize()
    return out


def oracle(c):
    return orc.paged_attention(c["q"], c["kc"], c["vc"], c["bt"], c["ctx"], c["Hkv"], c["scale"], c["bs"],
                               int(c["bt"].shape[1] * c["bs"]), c["alibi"], q_dtype=c["qd"], cache_dtype=c["dt"])


def expected_masked(c):
    """Oracle attention with the kernels' masking of block ids outside
    [0, num_blocks): such blocks' tokens are left out of the softmax."""
    kc = orc.decode(c["kc"], c["dt"])
    vc = orc.decode(c["vc"], c["dt"])
    nb, H, dx, bs, x = kc.shape
    q = orc.decode(c["q"], c["qd"])
    out = np.zeros(q.shape)
    max_seq_len = c["bt"].shape[1] * bs
    for s in range(q.shape[0]):
        ctx = int(c["ctx"][s])
        if ctx == 0 or ctx > max_seq_len:
            continue
        t = np.arange(ctx)
        b = c["bt"][s, t // bs].astype(np.int64)
        ok = (b >= 0) & (b < nb)
        k = kc[b[ok], :, :, (t % bs)[ok], :].reshape(-1, H, dx * x)
        v = vc[b[ok], :, :, (t % bs)[ok]]
        bias = None if c["alibi"] is None else orc.alibi_bias(c["alibi"], ctx)[:, ok]
        out[s] = orc._softmax_attend(q[s], k, v, c["scale"], bias)
    return out


def check(c):
    a, r = tolerance(c["qd"], c["dt"])
    np.testing.assert_allclose(to_f64(run(c)), oracle(c), atol=a, rtol=r)


@pytest.mark.parametrize("prefix", [256, 250])  # whole blocks / a partly filled last shared block
def test_radix_shared_prefix(prefix):
    check(radix_case(6000 + prefix, B=256, Hq=32, Hkv=8, D=128, bs=16, prefix_tokens=prefix, suffix_lo=1,
                     suffix_hi=200))


def test_unshared_batch_and_partial_group():
    check(radix_case(6100, B=258, Hq=32, Hkv=8, D=128, bs=16, prefix_tokens=0, suffix_lo=1, suffix_hi=400,
                     share=False))


def test_empty_overlong_and_masked():
    c = radix_case(6200, B=256, Hq=32, Hkv=8, D=64, bs=16, prefix_tokens=128, suffix_lo=1, suffix_hi=100,
                   dtype="float16")
    c["ctx"][[3, 77, 200]] = 0
    c["ctx"][150] = c["bt"].shape[1] * 16 + 5   # past max_seq_len: zero row
    c["bt"][:, 2] = -1                           # a shared block masked out in every sequence
    c["bt"][10, 5] = c["kc"].shape[0] + 3        # one sequence's shared block out of the pool
    out = to_f64(run(c))
    np.testing.assert_allclose(out, expected_masked(c), atol=2e-3, rtol=1e-2)
    assert not out[[3, 77, 150, 200]].any()


@pytest.mark.parametrize("bs", [8, 32])
def test_block_sizes_and_alibi(bs):
    check(radix_case(6300 + bs, B=256, Hq=32, Hkv=8, D=128, bs=bs, prefix_tokens=192, suffix_lo=1, suffix_hi=150,
                     alibi=True))


@pytest.mark.parametrize("Hq,Hkv,B", [(8, 8, 1024), (16, 8, 256)])  # MHA (group 1), GQA 2
def test_group_sizes(Hq, Hkv, B):
    check(radix_case(6400 + Hq, B=B, Hq=Hq, Hkv=Hkv, D=64, bs=16, prefix_tokens=64, suffix_lo=1, suffix_hi=60))


@pytest.mark.parametrize("q_dtype,dtype", [("float32", "bfloat16"), ("float32", "float16"), ("float16", "float16")])
def test_query_types(q_dtype, dtype):
    check(radix_case(6500, B=256, Hq=32, Hkv=8, D=96, bs=16, prefix_tokens=160, suffix_lo=1, suffix_hi=120,
                     dtype=dtype, q_dtype=q_dtype))


@pytest.mark.parametrize("q_dtype,D", [("float32", 128), ("float32", 112), ("bfloat16", 128)])
def test_float32_query_8_token_blocks(q_dtype, D):
    check(radix_case(6700 + D, B=256, Hq=32, Hkv=8, D=D, bs=8, prefix_tokens=120, suffix_lo=1, suffix_hi=90,
                     dtype="bfloat16", q_dtype=q_dtype))


FP8 = "fp8_e4m3"
FP8_TOL = {"bfloat16": (1e-2, 2e-2), "float16": (2e-3, 1e-2), "float32": (2e-3, 1e-2)}


def fp8_radix_case(seed, D, bs, q_dtype, prefix_tokens=160, suffix_hi=150, k_scale=0.05, v_scale=0.02):
    """radix_case's block tables, contexts and queries over FP8 caches that
    hold codes of N(0, 1.5) keys / k_scale and N(0, 0.5) values / v_scale."""
    c = radix_case(seed, B=256, Hq=32, Hkv=8, D=D, bs=bs, prefix_tokens=prefix_tokens, suffix_lo=1,
                   suffix_hi=suffix_hi, dtype="bfloat16", q_dtype=q_dtype)
    rng = np.random.default_rng(seed + 1)
    nb = c["kc"].shape[0]
    kx = (rng.standard_normal((nb, 8, D // 16, bs, 16)) * 1.5).astype(np.float32)
    vx = (rng.standard_normal((nb, 8, D, bs)) * 0.5).astype(np.float32)
    c["kc"] = orc.fp8_e4m3_encode(kx / np.float32(k_scale))
    c["vc"] = orc.fp8_e4m3_encode(vx / np.float32(v_scale))
    c.update(dt=FP8, ks=k_scale, vs=v_scale)
    return c


def check_fp8(c):
    out = kernels.paged_attention_v1(to_torch(c["q"], c["qd"]), to_torch(c["kc"], FP8), to_torch(c["vc"], FP8),
                                     to_index(c["bt"]), to_index(c["ctx"]), c["Hkv"], c["scale"], c["bs"],
                                     int(c["bt"].shape[1] * c["bs"]), None, k_scale=c["ks"], v_scale=c["vs"])
    torch.cuda.synchronize()
    exp = orc.paged_attention(c["q"], c["kc"], c["vc"], c["bt"], c["ctx"], c["Hkv"], c["scale"], c["bs"],
                              int(c["bt"].shape[1] * c["bs"]), None, q_dtype=c["qd"], cache_dtype=FP8,
                              k_scale=c["ks"], v_scale=c["vs"])
    a, r = FP8_TOL[c["qd"]]
    np.testing.assert_allclose(to_f64(out), exp, atol=a, rtol=r)


@pytest.mark.parametrize("bs", [8, 16, 32])
def test_fp8_radix_shared_prefix(bs):
    check_fp8(fp8_radix_case(6800 + bs, D=128, bs=bs, q_dtype="bfloat16"))


@pytest.mark.parametrize("q_dtype,D,bs", [("float16", 128, 16), ("float32", 112, 8), ("float32", 64, 16),
                                          ("bfloat16", 96, 16)])
def test_fp8_query_types_head_sizes(q_dtype, D, bs):
    # 64 and 128 take the wide FP8 tiles (permuted query dims), 96 and 112
    # the 8-code k-steps.
    check_fp8(fp8_radix_case(6900 + D + bs, D=D, bs=bs, q_dtype=q_dtype))


@pytest.mark.parametrize("width", [256, 257])
def test_fp8_group_context_bound(width):
    # FP8 tables 4096 tokens wide (256 blocks of 16) still take the grouped
    # kernel's FP8 shape (two workgroups of four wavefronts per CU, at most
    # 4096 tokens); one block wider falls back to the one-sequence kernel.
    # Both match the oracle.
    c = fp8_radix_case(7100 + width, D=128, bs=16, q_dtype="bfloat16")
    pad = width - c["bt"].shape[1]
    c["bt"] = np.concatenate([c["bt"], np.full((c["bt"].shape[0], pad), -1, np.int32)], axis=1)
    check_fp8(c)


def test_fp8_empty_overlong_and_masked():
    c = fp8_radix_case(7000, D=64, bs=16, q_dtype="float16", prefix_tokens=128, suffix_hi=100)
    c["ctx"][[3, 77, 200]] = 0
    c["ctx"][150] = c["bt"].shape[1] * 16 + 5   # past max_seq_len: zero row
    c["bt"][:, 2] = -1                           # a shared block masked out in every sequence
    c["bt"][10, 5] = c["kc"].shape[0] + 3        # one sequence's shared block out of the pool
    out = kernels.paged_attention_v1(to_torch(c["q"], c["qd"]), to_torch(c["kc"], FP8), to_torch(c["vc"], FP8),
                                     to_index(c["bt"]), to_index(c["ctx"]), c["Hkv"], c["scale"], c["bs"],
                                     int(c["bt"].shape[1] * c["bs"]), None, k_scale=c["ks"], v_scale=c["vs"])
    torch.cuda.synchronize()
    # The masked oracle over the values the codes stand for.
    ref = dict(c, kc=(orc.fp8_e4m3_decode(c["kc"]) * np.float32(c["ks"])).astype(np.float32),
               vc=(orc.fp8_e4m3_decode(c["vc"]) * np.float32(c["vs"])).astype(np.float32), dt="float32")
    got = to_f64(out)
    np.testing.assert_allclose(got, expected_masked(ref), atol=2e-3, rtol=1e-2)
    assert not got[[3, 77, 150, 200]].any()


def _poison_last_token_v(c, s, code):
    """V of sequence s's last context token (KV head 0, dim 5) set to `code`
    (an inf pattern of the cache type)."""
    t = int(c["ctx"][s]) - 1
    c["vc"][c["bt"][s, t // c["bs"]], 0, 5, t % c["bs"]] = code


def _check_nonfinite(got, exp, a, r):
    np.testing.assert_array_equal(np.isfinite(got), np.isfinite(exp))
    fin = np.isfinite(exp)
    np.testing.assert_allclose(got[fin], exp[fin], atol=a, rtol=r)


def test_nonfinite_v_in_one_private_tail():
    # One sequence's private V holds +inf: its own output turns non-finite
    # (as the oracle's), while the other sequences of its item, which share
    # the MFMA columns and get p = 0 for that tile, stay finite and exact.
    c = radix_case(7100, B=256, Hq=32, Hkv=8, D=64, bs=16, prefix_tokens=96, suffix_lo=20, suffix_hi=80)
    for s in (5, 130):
        _poison_last_token_v(c, s, 0x7F80)
    got = to_f64(run(c))
    exp = oracle(c)
    assert not np.isfinite(exp[5]).all() and np.isfinite(np.delete(exp, [5, 130], axis=0)).all()
    _check_nonfinite(got, exp, *tolerance(c["qd"], c["dt"]))


def test_fp8_nonfinite_v_in_one_private_tail():
    c = fp8_radix_case(7200, D=128, bs=16, q_dtype="bfloat16", prefix_tokens=96, suffix_hi=80)
    for s in (7, 200):
        _poison_last_token_v(c, s, 0x78)  # +inf in the reference's E4M3
    out = kernels.paged_attention_v1(to_torch(c["q"], c["qd"]), to_torch(c["kc"], FP8), to_torch(c["vc"], FP8),
                                     to_index(c["bt"]), to_index(c["ctx"]), c["Hkv"], c["scale"], c["bs"],
                                     int(c["bt"].shape[1] * c["bs"]), None, k_scale=c["ks"], v_scale=c["vs"])
    torch.cuda.synchronize()
    exp = orc.paged_attention(c["q"], c["kc"], c["vc"], c["bt"], c["ctx"], c["Hkv"], c["scale"], c["bs"],
                              int(c["bt"].shape[1] * c["bs"]), None, q_dtype=c["qd"], cache_dtype=FP8,
                              k_scale=c["ks"], v_scale=c["vs"])
    assert not np.isfinite(exp[7]).all() and np.isfinite(np.delete(exp, [7, 200], axis=0)).all()
    _check_nonfinite(to_f64(out), exp, *FP8_TOL[c["qd"]])


def test_more_than_1024_sequences():
    check(radix_case(6600, B=1100, Hq=8, Hkv=2, D=64, bs=16, prefix_tokens=48, suffix_lo=1, suffix_hi=40))


def bound_case(seed, bound, D, bs, fp8=False, q_dtype="bfloat16"):
    """Contexts that reach the grouped kernel's bound: 256 sequences over 8 KV
    heads (GQA 4, so 512 items of four sequences: two per CU); 192 share a
    prefix of bound - 256 tokens and 64 a prefix of bound / 2, each then
    holds 1-256 private tokens, sequence 0 exactly bound tokens in all.  The
    block tables are bound tokens wide."""
    rng = np.random.default_rng(seed)
    B, Hq, Hkv = 256, 32, 8
    grp = np.array([0] * 192 + [1] * 64)
    pre = np.where(grp == 0, bound - 256, bound // 2)
    tail = rng.integers(1, 257, size=B)
    tail[0] = 256
    ctx = (pre + tail).astype(np.int32)
    nblk = -(-ctx // bs)
    heads = [pre[0] // bs, pre[-1] // bs]
    private = nblk - np.array([heads[g] for g in grp])
    nb = int(sum(heads) + private.sum() + 2)
    perm = rng.permutation(np.arange(1, nb))
    shared = [perm[:heads[0]], perm[heads[0]:heads[0] + heads[1]]]
    pos = heads[0] + heads[1]
    bt = np.full((B, bound // bs), -1, dtype=np.int32)
    for s in range(B):
        h = shared[grp[s]]
        bt[s, :h.size] = h
        bt[s, h.size:nblk[s]] = perm[pos:pos + private[s]]
        pos += private[s]
    q = normal(rng, (B, Hq, D), q_dtype)
    c = dict(q=q, bt=bt, ctx=ctx, Hkv=Hkv, bs=bs, qd=q_dtype, alibi=None, scale=1.0 / math.sqrt(D))
    if fp8:
        ks, vs = 0.05, 0.02
        kx = (rng.standard_normal((nb, Hkv, D // 16, bs, 16)) * 1.5).astype(np.float32)
        vx = (rng.standard_normal((nb, Hkv, D, bs)) * 0.5).astype(np.float32)
        c.update(kc=orc.fp8_e4m3_encode(kx / np.float32(ks)), vc=orc.fp8_e4m3_encode(vx / np.float32(vs)), dt=FP8,
                 ks=ks, vs=vs)
    else:
        x = X_OF["bfloat16"]
        c.update(kc=normal(rng, (nb, Hkv, D // x, bs, x), "bfloat16"), vc=normal(rng, (nb, Hkv, D, bs), "bfloat16"),
                 dt="bfloat16")
    return c


@pytest.mark.parametrize("dt,D,bs,bound", [("bfloat16", 128, 16, 8192), ("bfloat16", 128, 32, 8192),
                                           ("bfloat16", 64, 8, 8192), ("fp8", 128, 16, 4096),
                                           ("fp8", 128, 32, 4096), ("fp8", 64, 16, 4096), ("fp8", 64, 8, 4096)])
def test_group_contexts_at_the_bound(dt, D, bs, bound):
    # The grouped kernel at the longest contexts its launcher admits (8192
    # tokens over 16-bit caches, 4096 over FP8 at head sizes 64 and 128):
    # the job lists, packed tile indices and block ids held in registers at
    # their fullest, shared and private tiles mixed.  The whole batch runs;
    # 16 of its rows (the longest among them) are checked against the oracle.
    fp8 = dt == "fp8"
    c = bound_case(9100 + D + bs + bound, bound, D, bs, fp8=fp8)
    scales = dict(k_scale=c["ks"], v_scale=c["vs"]) if fp8 else {}
    out = kernels.paged_attention_v1(to_torch(c["q"], c["qd"]), to_torch(c["kc"], c["dt"]), to_torch(c["vc"], c["dt"]),
                                     to_index(c["bt"]), to_index(c["ctx"]), c["Hkv"], c["scale"], bs, bound, None,
                                     **scales)
    torch.cuda.synchronize()
    rng = np.random.default_rng(bound + D + bs)
    sel = np.concatenate([[0], rng.choice(np.arange(1, 256), size=15, replace=False)])
    extra = dict(cache_dtype=FP8, k_scale=c["ks"], v_scale=c["vs"]) if fp8 else dict(cache_dtype=c["dt"])
    exp = orc.paged_attention(c["q"][sel], c["kc"], c["vc"], c["bt"][sel], c["ctx"][sel], c["Hkv"], c["scale"], bs,
                              bound, None, q_dtype=c["qd"], **extra)
    a, r = FP8_TOL[c["qd"]] if fp8 else tolerance(c["qd"], c["dt"])
    assert int(c["ctx"][0]) == bound
    np.testing.assert_allclose(to_f64(out)[sel], exp, atol=a, rtol=r)
