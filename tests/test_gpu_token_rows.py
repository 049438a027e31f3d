"""GPU parity of paged decode on the token-row layout (MHATokenPool's
[rows, Hkv, D] with slot tables, and the flash layout [blocks, block_size,
Hkv, D] with block tables) against the oracle, and the gather-free pool
decode (MHATokenPool.decode, decode_batch) against the reference's
gather + attention path.  The token-row caches are laid out as paged 5-D
caches for the oracle (token_major_to_paged5d), so both read the same
values.  Tolerances as elsewhere: float16 2e-3 abs / 1e-2 rel, bfloat16
1e-2 / 2e-2."""

import math

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from pkv_cases import X_OF, normal, tolerance
from pkv_torch import to_f64, to_index, to_torch
from sglang_mlx_amd import kernels
from sglang_mlx_amd.srt.mem_cache import MHATokenPool, PooledKVCache, TokenPoolAllocator, decode_batch

pytestmark = pytest.mark.gpu


def rows_case(seed, B, Hq, Hkv, D, bs, ctx_lo, ctx_hi, cache_dtype="bfloat16", q_dtype=None, alibi=False):
    rng = np.random.default_rng(seed)
    q_dtype = q_dtype or cache_dtype
    ctx = rng.integers(ctx_lo, ctx_hi + 1, size=B).astype(np.int32)
    nblk = -(-ctx // bs)
    nb = int(nblk.sum() * 1.2) + 2
    perm = rng.permutation(np.arange(1, nb))
    width = int(nblk.max())
    bt = np.full((B, width), -1, dtype=np.int32)
    pos = 0
    for s in range(B):
        bt[s, :nblk[s]] = perm[pos:pos + nblk[s]]
        pos += nblk[s]
    kt = normal(rng, (nb * bs, Hkv, D), cache_dtype)
    vt = normal(rng, (nb * bs, Hkv, D), cache_dtype)
    q = normal(rng, (B, Hq, D), q_dtype)
    slopes = (rng.uniform(0.01, 0.2, size=Hq).astype(np.float32) if alibi else None)
    return dict(q=q, kt=kt, vt=vt, bt=bt, ctx=ctx, nb=nb, bs=bs, Hkv=Hkv, D=D, cache=cache_dtype, qd=q_dtype,
                alibi=slopes, scale=1.0 / math.sqrt(D))


def oracle(c):
    x = X_OF[c["cache"]]
    k5, v4 = orc.token_major_to_paged5d(c["kt"], c["vt"], c["bs"], x)
    return orc.paged_attention(c["q"], k5, v4, c["bt"], c["ctx"], c["Hkv"], c["scale"], c["bs"],
                               int(c["bt"].shape[1] * c["bs"]), c["alibi"], q_dtype=c["qd"],
                               cache_dtype=c["cache"])


def expected_masked(c):
    """Oracle attention with the kernel's masking: tokens whose block id lies
    outside [0, num_blocks) are left out of the softmax; contexts of 0 or past
    max_seq_len give zero rows."""
    bs, nb = c["bs"], c["nb"]
    q = orc.decode(c["q"], c["qd"])
    out = np.zeros(q.shape, dtype=np.float64)
    max_seq_len = int(c["bt"].shape[1] * bs)
    for s in range(q.shape[0]):
        ctx = int(c["ctx"][s])
        if ctx == 0 or ctx > max_seq_len:
            continue
        t = np.arange(ctx)
        b = c["bt"][s, t // bs].astype(np.int64)
        ok = (b >= 0) & (b < nb)
        if not ok.any():
            continue
        rows = (b * bs + t % bs)[ok]
        k = orc.decode(c["kt"][rows], c["cache"])
        v = orc.decode(c["vt"][rows], c["cache"])
        bias = None if c["alibi"] is None else orc.alibi_bias(c["alibi"], ctx)[:, ok]
        out[s] = orc._softmax_attend(q[s], k, v, c["scale"], bias)
    return out


def run(c, partition_size=None):
    kt, vt = to_torch(c["kt"], c["cache"]), to_torch(c["vt"], c["cache"])
    if c["bs"] > 1:
        kt = kt.view(c["nb"], c["bs"], c["Hkv"], c["D"])
        vt = vt.view(c["nb"], c["bs"], c["Hkv"], c["D"])
    alibi = None if c["alibi"] is None else torch.from_numpy(c["alibi"]).cuda()
    args = (to_torch(c["q"], c["qd"]), kt, vt, to_index(c["bt"]), to_index(c["ctx"]), c["Hkv"], c["scale"], c["bs"],
            int(c["bt"].shape[1] * c["bs"]), alibi)
    out = (kernels.paged_attention_v1(*args) if partition_size is None
           else kernels.paged_attention_v2(*args, partition_size=partition_size))
    torch.cuda.synchronize()
    return out


def check(c, partition_size=None):
    a, r = tolerance(c["qd"], c["cache"])
    np.testing.assert_allclose(to_f64(run(c, partition_size)), oracle(c), atol=a, rtol=r)


@pytest.mark.parametrize("bs", [1, 8, 16, 32])
def test_block_sizes(bs):
    check(rows_case(4000 + bs, B=5, Hq=8, Hkv=2, D=128, bs=bs, ctx_lo=1, ctx_hi=700))


@pytest.mark.parametrize("D", [32, 64, 80, 96, 112, 120, 192, 256])
def test_head_sizes(D):
    check(rows_case(4100 + D, B=3, Hq=8, Hkv=4, D=D, bs=1, ctx_lo=1, ctx_hi=300))


@pytest.mark.parametrize("q_dtype,cache_dtype", [("float16", "float16"), ("float32", "bfloat16"),
                                                 ("float32", "float16")])
def test_dtype_pairs(q_dtype, cache_dtype):
    check(rows_case(4200, B=4, Hq=16, Hkv=4, D=128, bs=1, ctx_lo=1, ctx_hi=500, cache_dtype=cache_dtype,
                    q_dtype=q_dtype))


def test_gqa7_alibi_and_split_k():
    c = rows_case(4300, B=3, Hq=28, Hkv=4, D=128, bs=1, ctx_lo=100, ctx_hi=3000, alibi=True)
    check(c)
    check(c, partition_size=64)
    check(c, partition_size=1024)


def test_masked_rows_and_empty_contexts():
    c = rows_case(4400, B=6, Hq=8, Hkv=2, D=64, bs=1, ctx_lo=10, ctx_hi=400, cache_dtype="float16")
    c["ctx"][2] = 0
    out = to_f64(run(c))
    assert np.count_nonzero(out[2]) == 0
    ref = oracle(c)
    np.testing.assert_allclose(out, ref, atol=2e-3, rtol=1e-2)
    # Slots outside the pool are masked out (their tokens contribute nothing).
    nrows = c["kt"].shape[0]
    c["bt"][1, 3] = nrows + 5
    c["bt"][4, 0] = -7
    out = to_f64(run(c))
    for s in (1, 4):
        keep = np.arange(c["ctx"][s])
        row = c["bt"][s][keep]
        ok = (row >= 0) & (row < nrows)
        qh = orc.decode(c["q"][s], "float16")
        k = orc.decode(c["kt"][row[ok]], "float16")
        v = orc.decode(c["vt"][row[ok]], "float16")
        np.testing.assert_allclose(out[s], orc._softmax_attend(qh, k, v, c["scale"], None), atol=2e-3, rtol=1e-2)


def test_llama3_8b_layer_matches_the_paged_layout():
    # 64 sequences, ctx U[512, 4096], bf16, slot tables over a token-major
    # pool, against the paged 5-D kernel on the same values (whose parity
    # with the oracle is pinned by the paged tests).
    c = rows_case(1003, B=64, Hq=32, Hkv=8, D=128, bs=1, ctx_lo=512, ctx_hi=4096)
    out_rows = run(c)
    # The same tokens in 16-token blocks of the paged layout.
    bs = 16
    rng = np.random.default_rng(7)
    B = c["bt"].shape[0]
    nblk = -(-c["ctx"] // bs)
    nb = int(nblk.sum()) + 1
    bt16 = np.full((B, int(nblk.max())), -1, dtype=np.int32)
    kt16 = np.zeros((nb * bs, c["Hkv"], c["D"]), dtype=np.uint16)
    vt16 = np.zeros_like(kt16)
    nxt = 1
    for s in range(B):
        for j in range(nblk[s]):
            bt16[s, j] = nxt
            toks = np.arange(j * bs, min((j + 1) * bs, c["ctx"][s]))
            kt16[nxt * bs + toks % bs] = c["kt"][c["bt"][s, toks]]
            vt16[nxt * bs + toks % bs] = c["vt"][c["bt"][s, toks]]
            nxt += 1
    k5, v4 = orc.token_major_to_paged5d(kt16, vt16, bs, 8)
    out_paged = kernels.paged_attention_v1(to_torch(c["q"], "bfloat16"), to_torch(k5, "bfloat16"),
                                           to_torch(v4, "bfloat16"), to_index(bt16), to_index(c["ctx"]), 8,
                                           c["scale"], bs, int(bt16.shape[1] * bs))
    torch.cuda.synchronize()
    np.testing.assert_allclose(to_f64(out_rows), to_f64(out_paged), atol=1e-2, rtol=2e-2)


def test_pool_decode_batch_matches_gather_and_attention():
    # The reference's decode path: update_and_fetch gathers each request's
    # K/V, then attention over them; decode_batch reads the pool rows in place.
    torch.manual_seed(0)
    H, D, Hq, L = 4, 64, 8, 2
    alloc = TokenPoolAllocator(256)
    pool = MHATokenPool(256, L, H, D, dtype=torch.float16)
    lens = [37, 5, 64]
    caches = []
    for n in lens:
        c = PooledKVCache(pool, 1)
        c.set_indices([], alloc.alloc(n + 1))
        k = torch.randn((1, H, n, D), device="cuda", dtype=torch.float16)
        c.update_and_fetch(k, torch.randn_like(k))
        caches.append(c)
    # This step's token for every request, then the batched decode.
    q = torch.randn((len(lens), Hq, D), device="cuda", dtype=torch.float16)
    gathered = []
    for c in caches:
        k1 = torch.randn((1, H, 1, D), device="cuda", dtype=torch.float16)
        gathered.append(c.update_and_fetch(k1, torch.randn_like(k1)))
    scale = 1.0 / math.sqrt(D)
    out = decode_batch(caches, q, scale)
    torch.cuda.synchronize()
    for i, (kk, vv) in enumerate(gathered):
        k = kk[0].transpose(0, 1).cpu().numpy().astype(np.float64)   # [T, H, D]
        v = vv[0].transpose(0, 1).cpu().numpy().astype(np.float64)
        exp = orc._softmax_attend(q[i].cpu().numpy().astype(np.float64), k, v, scale, None)
        np.testing.assert_allclose(out[i].float().cpu().numpy(), exp, atol=2e-3, rtol=1e-2)
    with pytest.raises(ValueError, match="same pool layer"):
        other = PooledKVCache(pool, 0)
        decode_batch([caches[0], other], q[:2], scale)


# The persistent kernel takes token-row batches with at least two
# (sequence, KV head) items per resident workgroup (512 here) and
# max_seq_len <= 4096 (2048 above head size 128).
@pytest.mark.parametrize("D,bs,q_dtype,cache_dtype", [
    (128, 1, "bfloat16", "bfloat16"), (128, 16, "bfloat16", "bfloat16"), (128, 8, "float16", "float16"),
    (64, 1, "float32", "bfloat16"), (96, 32, "float32", "float16"), (120, 1, "float16", "float16"),
    (32, 1, "bfloat16", "bfloat16"), (256, 1, "bfloat16", "bfloat16"), (192, 16, "float32", "bfloat16"),
    (256, 8, "float32", "float16"),
])
def test_persistent_rows(D, bs, q_dtype, cache_dtype):
    c = rows_case(4500 + D + bs, B=128, Hq=8, Hkv=4, D=D, bs=bs, ctx_lo=1, ctx_hi=600, cache_dtype=cache_dtype,
                  q_dtype=q_dtype, alibi=(D == 128 and bs == 1))
    a, r = tolerance(q_dtype, cache_dtype)
    np.testing.assert_allclose(to_f64(run(c)), oracle(c), atol=a, rtol=r)
    # Masked block ids, an empty and an over-long context.
    rng = np.random.default_rng(D)
    for s in rng.choice(128, size=20, replace=False):
        n = -(-int(c["ctx"][s]) // bs)
        c["bt"][s, rng.integers(0, n)] = rng.choice([-1, c["nb"], c["nb"] + 1000])
    c["ctx"][7] = 0
    c["ctx"][9] = c["bt"].shape[1] * bs + 1
    np.testing.assert_allclose(to_f64(run(c)), expected_masked(c), atol=a, rtol=r)


def test_persistent_rows_longest_contexts():
    # Contexts up to the 4096-token bound of the persistent token-row path.
    c = rows_case(4600, B=64, Hq=32, Hkv=8, D=128, bs=1, ctx_lo=3000, ctx_hi=4096, cache_dtype="float16")
    assert c["bt"].shape[1] <= 4096
    np.testing.assert_allclose(to_f64(run(c)), oracle(c), atol=2e-3, rtol=1e-2)
