"""The CPU baseline of bench.py (oracle/cpu_baseline.py: the reference's
gather + scaled_dot_product_attention decode restated in torch on the host)
against the float64 oracle, on float32 caches so that the comparison sees
the algorithm rather than 16-bit rounding: the token-major gather and the
paged 5-D relayout of tests/bench_paged_vs_gather.py:86-92 both give the
oracle's softmax attention (up to the 1e-6 the reference kernel adds to the
denominator and SDPA does not).  A planted mistake (a transposed K chunk in
the relayout) is shown to fail the same check."""

import numpy as np
import torch

from oracle import cpu_baseline as cb
from oracle import pagedkv_oracle as orc


def case(seed=7, B=3, Hq=8, Hkv=2, D=64, bs=16, nb=40):
    rng = np.random.default_rng(seed)
    x = 4  # 16 bytes of float32
    kc = rng.standard_normal((nb, Hkv, D // x, bs, x)).astype(np.float32)
    vc = rng.standard_normal((nb, Hkv, D, bs)).astype(np.float32)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    ctx = np.array([1, 37, 200], dtype=np.int32)[:B]
    width = -(-int(ctx.max()) // bs)
    bt = np.stack([rng.permutation(np.arange(1, nb))[:width] for _ in range(B)]).astype(np.int32)
    return q, kc, vc, bt, ctx, Hkv, 1.0 / np.sqrt(D), bs


def expected(q, kc, vc, bt, ctx, Hkv, scale, bs):
    return orc.paged_attention(q, kc, vc, bt, ctx, Hkv, scale, bs,
                               bt.shape[1] * bs, None, q_dtype="float32", cache_dtype="float32")


def test_paged5d_relayout_matches_oracle():
    q, kc, vc, bt, ctx, Hkv, scale, bs = case()
    out = cb.gather_sdpa_decode_paged5d(torch.from_numpy(q), torch.from_numpy(kc), torch.from_numpy(vc),
                                        torch.from_numpy(bt), torch.from_numpy(ctx), bs, scale)
    np.testing.assert_allclose(out.double().numpy(), expected(q, kc, vc, bt, ctx, Hkv, scale, bs),
                               atol=2e-6, rtol=2e-5)


def test_token_major_pool_matches_oracle():
    q, kc, vc, bt, ctx, Hkv, scale, bs = case(seed=8)
    k_pool, v_pool = cb.paged5d_to_token_major(torch.from_numpy(kc), torch.from_numpy(vc))
    assert k_pool.shape == (kc.shape[0] * bs, Hkv, q.shape[2])
    # Slot = block * bs + offset holds that token's row of every head.
    blk, off, h = 5, 3, 1
    np.testing.assert_array_equal(k_pool[blk * bs + off, h].numpy(), kc[blk, h, :, off, :].reshape(-1))
    np.testing.assert_array_equal(v_pool[blk * bs + off, h].numpy(), vc[blk, h, :, off])
    out = cb.gather_sdpa_decode(torch.from_numpy(q), k_pool, v_pool, torch.from_numpy(bt), torch.from_numpy(ctx),
                                bs, scale)
    np.testing.assert_allclose(out.double().numpy(), expected(q, kc, vc, bt, ctx, Hkv, scale, bs),
                               atol=2e-6, rtol=2e-5)


def test_planted_relayout_mistake_fails():
    q, kc, vc, bt, ctx, Hkv, scale, bs = case(seed=9)
    k_pool, v_pool = cb.paged5d_to_token_major(torch.from_numpy(kc), torch.from_numpy(vc))
    bad = k_pool.reshape(k_pool.shape[0], Hkv, -1, 4).flip(2).reshape(k_pool.shape)  # chunks reversed
    out = cb.gather_sdpa_decode(torch.from_numpy(q), bad, v_pool, torch.from_numpy(bt), torch.from_numpy(ctx),
                                bs, scale)
    err = np.abs(out.double().numpy() - expected(q, kc, vc, bt, ctx, Hkv, scale, bs)).max()
    assert err > 1e-2


def test_scatter_append_matches_oracle():
    # the append's CPU baseline against the oracle's restatement
    # (reshape_and_cache_paged5d), float16, with padding and ragged slots
    rng = np.random.default_rng(11)
    N, H, D, bs, x, nb = 53, 8, 128, 16, 8, 9
    k = rng.standard_normal((N, H, D)).astype(np.float16)
    v = rng.standard_normal((N, H, D)).astype(np.float16)
    slots = rng.choice(nb * bs, N, replace=False).astype(np.int64)
    slots[[0, 7, 30]] = -1
    kc = np.zeros((nb, H, D // x, bs, x), np.float16)
    vc = np.zeros((nb, H, D, bs), np.float16)
    kb, vb = (a.view(np.uint16) for a in (k, v))
    ek, ev = orc.reshape_and_cache_paged5d(kb, vb, kc.view(np.uint16), vc.view(np.uint16), slots, "float16",
                                           "float16")
    tk, tv = torch.from_numpy(kc.copy()), torch.from_numpy(vc.copy())
    cb.scatter_append_paged5d(torch.from_numpy(k), torch.from_numpy(v), tk, tv, torch.from_numpy(slots))
    assert np.array_equal(tk.numpy().view(np.uint16), ek) and np.array_equal(tv.numpy().view(np.uint16), ev)
    # a planted mistake (the head dimension split as [x, D/x] instead of
    # [D/x, x]) is caught
    keep = torch.from_numpy(slots >= 0)
    s_ = torch.from_numpy(slots)[keep]
    bad_k = torch.from_numpy(kc.copy())
    bad_k.permute(0, 3, 1, 2, 4)[s_ // bs, s_ % bs] = \
        torch.from_numpy(k)[keep].reshape(-1, H, x, D // x).transpose(2, 3)
    assert not np.array_equal(bad_k.numpy().view(np.uint16), ek)
