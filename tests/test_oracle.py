"""Pins the CPU oracle (oracle/pagedkv_oracle.py) before anything is checked
against it.  CPU only.

Each oracle function is checked against something independent of its own
formula:
  * conversions     -- torch's float32 -> bfloat16 / float16 casts (round to
                       nearest even), IEEE special values, the reference's
                       NaN -> 0x7FC0 rule (utils.metal:21-35);
  * append          -- a brute-force element loop over the reference's index
                       formula (tests/test_paged_attention_kernel.py:46-63,
                       reshape_and_cache.metal:54-65), read-back through
                       gather_kv, untouched-slot and padding invariants, and
                       the token-major <-> paged 5-D equivalence;
  * attention       -- torch's float64 scaled_dot_product_attention (GQA by
                       enable_gqa), closed forms (one token, equal keys, a
                       dominant logit, ALiBi geometric weights), the
                       reference's zero-output KATs, block-permutation and
                       GQA invariances;
  * split-K         -- equality with the unpartitioned oracle at every
                       partition size and boundary.
A planted mistake (dropped 1e-6, wrong GQA map, transposed K chunk, missing
ALiBi offset) is shown to fail these checks.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import pagedkv_oracle as orc
from pkv_cases import X_OF, make_append_case, make_decode_case

# ---------------------------------------------------------------------------
# Conversions
# ---------------------------------------------------------------------------

SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 1e-8, -1e-8, 6.1e-5, 5.96e-8, 2.98e-8,
                     3.4e38, -3.4e38, np.inf, -np.inf, 1.00390625, 1.01171875, 1.0 + 2**-8, 1.0 + 3 * 2**-8,
                     2**-133, 2**-126, 2**-149], dtype=np.float32)


def _torch_bits(x: np.ndarray, dtype) -> np.ndarray:
    return torch.from_numpy(x).to(dtype).view(torch.int16).numpy().view(np.uint16)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 200000),
                        SPECIALS]).astype(np.float32)
    # Exact ties: low 16 bits 0x8000 with both parities of bit 16.
    ties = (rng.integers(0, 2**15, 1000).astype(np.uint32) << 17 | 0x8000).astype(np.uint32)
    ties = np.concatenate([ties, ties | 0x10000]).view(np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)]])
    np.testing.assert_array_equal(orc.f32_to_bf16_bits(x), _torch_bits(x, torch.bfloat16))


def test_bf16_nan_is_canonical():
    payloads = np.array([0x7F800001, 0x7FC00000, 0xFFC00001, 0x7FFFFFFF, 0xFF800001], dtype=np.uint32)
    np.testing.assert_array_equal(orc.f32_to_bf16_bits(payloads.view(np.float32)), np.full(5, 0x7FC0))


def test_f16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 200000),
                        SPECIALS]).astype(np.float32)
    np.testing.assert_array_equal(orc.f32_to_f16_bits(x), _torch_bits(x, torch.float16))


@pytest.mark.filterwarnings("ignore:invalid value encountered in cast:RuntimeWarning")
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_decode_is_exact_inverse_of_storage(dtype):
    bits = np.arange(0, 2**16, dtype=np.uint32).astype(np.uint16)
    vals = orc.decode(bits, dtype)
    finite = np.isfinite(vals)
    back = orc.to_storage(vals[finite].astype(np.float32), dtype)
    np.testing.assert_array_equal(back, bits[finite])
    tdt = torch.float16 if dtype == "float16" else torch.bfloat16
    ref = torch.from_numpy(bits.view(np.int16)).view(tdt).to(torch.float64).numpy()
    np.testing.assert_array_equal(vals[finite], ref[finite])


# ---------------------------------------------------------------------------
# Append
# ---------------------------------------------------------------------------


def brute_paged5d(key, value, kc, vc, slots, kv_dtype, cache_dtype):
    """Element loop over the reference's index formula."""
    kc, vc = kc.copy(), vc.copy()
    nb, H, dx, bs, x = kc.shape
    D = dx * x
    for i, slot in enumerate(slots):
        if slot < 0:
            continue
        b, off = slot // bs, slot % bs
        for h in range(H):
            for d in range(D):
                k = orc.convert_elements(key[i, h, d:d + 1], kv_dtype, cache_dtype)[0]
                v = orc.convert_elements(value[i, h, d:d + 1], kv_dtype, cache_dtype)[0]
                kc[b, h, d // x, off, d % x] = k
                vc[b, h, d, off] = v
    return kc, vc


PAIRS = [("bfloat16", "bfloat16"), ("float16", "float16"), ("float32", "float32"),
         ("float32", "float16"), ("float32", "bfloat16")]


@pytest.mark.parametrize("kv_dtype,cache_dtype", PAIRS)
@pytest.mark.parametrize("block_size", [8, 16])
def test_append_paged5d_matches_element_loop(kv_dtype, cache_dtype, block_size):
    nb, H, D = 6, 2, 32
    x = X_OF[cache_dtype]
    case = make_append_case(3, N=40, H=H, D=D, num_slots=nb * block_size, block_size=block_size,
                            kv_dtype=kv_dtype, cache_dtype=cache_dtype, pad_frac=0.1)
    rng = np.random.default_rng(4)
    kc0 = orc.to_storage(rng.standard_normal((nb, H, D // x, block_size, x), dtype=np.float32), cache_dtype)
    vc0 = orc.to_storage(rng.standard_normal((nb, H, D, block_size), dtype=np.float32), cache_dtype)
    got = orc.reshape_and_cache_paged5d(case.key, case.value, kc0, vc0, case.slot_mapping, kv_dtype, cache_dtype)
    ref = brute_paged5d(case.key, case.value, kc0, vc0, case.slot_mapping, kv_dtype, cache_dtype)
    np.testing.assert_array_equal(got[0], ref[0])
    np.testing.assert_array_equal(got[1], ref[1])


def test_append_read_back_and_untouched_slots():
    nb, H, D, bs = 8, 4, 64, 16
    case = make_append_case(5, N=60, H=H, D=D, num_slots=nb * bs, block_size=bs, pad_frac=0.2)
    zeros_k = np.zeros((nb, H, D // 8, bs, 8), np.uint16)
    zeros_v = np.zeros((nb, H, D, bs), np.uint16)
    kc, vc = orc.reshape_and_cache_paged5d(case.key, case.value, zeros_k, zeros_v, case.slot_mapping,
                                           "bfloat16", "bfloat16")
    written = set()
    for i, s in enumerate(case.slot_mapping):
        if s < 0:
            continue
        written.add(int(s))
        row = np.array([s // bs])
        # Read slot s back through the block-table gather: token (s % bs) of a
        # one-block table (bit patterns carried as float64, compared exactly).
        k, v = orc.gather_kv(kc.astype(np.float64), vc.astype(np.float64), row, s % bs + 1)
        np.testing.assert_array_equal(k[-1], case.key[i].astype(np.float64))
        np.testing.assert_array_equal(v[-1], case.value[i].astype(np.float64))
    untouched = [s for s in range(nb * bs) if s not in written]
    tm_k, _ = orc.reshape_and_cache_token_major(case.key, case.value, np.zeros((nb * bs, H, D), np.uint16),
                                                np.zeros((nb * bs, H, D), np.uint16), case.slot_mapping,
                                                "bfloat16", "bfloat16")
    assert not tm_k[untouched].any()
    assert (case.slot_mapping < 0).sum() == 12


@pytest.mark.parametrize("kv_dtype,cache_dtype", PAIRS)
def test_token_major_equals_paged5d_after_relayout(kv_dtype, cache_dtype):
    nb, H, D, bs = 10, 2, 64, 16
    x = X_OF[cache_dtype]
    case = make_append_case(6, N=100, H=H, D=D, num_slots=nb * bs, block_size=bs, kv_dtype=kv_dtype,
                            cache_dtype=cache_dtype)
    rng = np.random.default_rng(7)
    tk0 = orc.to_storage(rng.standard_normal((nb * bs, H, D), dtype=np.float32), cache_dtype)
    tv0 = orc.to_storage(rng.standard_normal((nb * bs, H, D), dtype=np.float32), cache_dtype)
    tk, tv = orc.reshape_and_cache_token_major(case.key, case.value, tk0, tv0, case.slot_mapping, kv_dtype,
                                               cache_dtype)
    k50, v40 = orc.token_major_to_paged5d(tk0, tv0, bs, x)
    k5, v4 = orc.reshape_and_cache_paged5d(case.key, case.value, k50, v40, case.slot_mapping, kv_dtype,
                                           cache_dtype)
    rk, rv = orc.token_major_to_paged5d(tk, tv, bs, x)
    np.testing.assert_array_equal(k5, rk)
    np.testing.assert_array_equal(v4, rv)


def test_append_padding_is_noop():
    case = make_append_case(8, N=16, H=2, D=32, num_slots=64, block_size=16)
    case.slot_mapping[:] = -1
    kc0 = np.arange(4 * 2 * 4 * 16 * 8, dtype=np.uint16).reshape(4, 2, 4, 16, 8)
    vc0 = np.arange(4 * 2 * 32 * 16, dtype=np.uint16).reshape(4, 2, 32, 16)
    kc, vc = orc.reshape_and_cache_paged5d(case.key, case.value, kc0, vc0, case.slot_mapping, "bfloat16",
                                           "bfloat16")
    np.testing.assert_array_equal(kc, kc0)
    np.testing.assert_array_equal(vc, vc0)


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------


def torch_sdpa_reference(c) -> np.ndarray:
    """torch float64 SDPA on the gathered K/V, GQA by enable_gqa."""
    q64 = orc.decode(c.q, c.q_dtype)
    kc64 = orc.decode(c.k_cache, c.cache_dtype)
    vc64 = orc.decode(c.v_cache, c.cache_dtype)
    B, Hq, D = q64.shape
    out = np.zeros((B, Hq, D))
    for s in range(B):
        ctx = int(c.context_lens[s])
        if ctx == 0 or ctx > c.max_seq_len:
            continue
        k, v = orc.gather_kv(kc64, vc64, c.block_tables[s], ctx)
        qt = torch.from_numpy(q64[s]).reshape(1, Hq, 1, D)
        kt = torch.from_numpy(np.ascontiguousarray(k.transpose(1, 0, 2)))[None]
        vt = torch.from_numpy(np.ascontiguousarray(v.transpose(1, 0, 2)))[None]
        bias = None
        if c.alibi is not None:
            bias = torch.from_numpy(orc.alibi_bias(c.alibi, ctx)).reshape(1, Hq, 1, ctx)
        o = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=bias, scale=c.scale, enable_gqa=True)
        out[s] = o.reshape(Hq, D).numpy()
    return out


@pytest.mark.parametrize("Hq,Hkv,D,bs,cd,qd,alibi", [
    (8, 2, 64, 16, "bfloat16", "bfloat16", False),
    (28, 4, 128, 16, "bfloat16", "bfloat16", False),
    (4, 4, 32, 8, "float16", "float32", False),
    (8, 1, 80, 32, "float16", "float16", True),
    (6, 3, 96, 16, "bfloat16", "float32", True),
])
def test_attention_matches_torch_sdpa(Hq, Hkv, D, bs, cd, qd, alibi):
    c = make_decode_case(Hq * 7 + D, B=3, Hq=Hq, Hkv=Hkv, D=D, block_size=bs, ctx_lo=1, ctx_hi=300,
                         cache_dtype=cd, q_dtype=qd, alibi=alibi)
    got = orc.paged_attention(c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens, c.num_kv_heads,
                              c.scale, c.block_size, c.max_seq_len, c.alibi, c.q_dtype, c.cache_dtype)
    ref = torch_sdpa_reference(c)
    # The reference kernel's denominator is (sum + 1e-6); with sum >= 1 that
    # is at most a 1e-6 relative difference from SDPA.
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)


def _one_seq(k_tok, v_tok, q, bs=16, scale=1.0, alibi=None, max_seq_len=None):
    """Single-sequence oracle call on float32 token-major K/V [T, Hkv, D]."""
    T, Hkv, D = k_tok.shape
    nb = -(-T // bs) + 1
    tk = np.zeros((nb * bs, Hkv, D), np.float32)
    tv = np.zeros((nb * bs, Hkv, D), np.float32)
    tk[bs:bs + T] = k_tok
    tv[bs:bs + T] = v_tok
    k5, v4 = orc.token_major_to_paged5d(tk, tv, bs, 4)
    bt = np.arange(1, nb, dtype=np.int32)[None]
    return orc.paged_attention(q[None].astype(np.float32), k5, v4, bt, np.array([T], np.int32), Hkv, scale, bs,
                               max_seq_len or T, alibi, "float32", "float32")[0]


def test_single_token_returns_its_value():
    rng = np.random.default_rng(9)
    k = rng.standard_normal((1, 2, 32)).astype(np.float32)
    v = rng.standard_normal((1, 2, 32)).astype(np.float32)
    q = rng.standard_normal((4, 32)).astype(np.float32)
    out = _one_seq(k, v, q)
    expect = np.repeat(v[0].astype(np.float64), 2, axis=0) / (1 + 1e-6)
    np.testing.assert_allclose(out, expect, rtol=1e-12, atol=0)


def test_equal_keys_give_mean_of_values():
    rng = np.random.default_rng(10)
    T = 37
    k = np.repeat(rng.standard_normal((1, 1, 64)).astype(np.float32), T, axis=0)
    v = rng.standard_normal((T, 1, 64)).astype(np.float32)
    q = rng.standard_normal((3, 64)).astype(np.float32)
    out = _one_seq(k, v, q, scale=0.3)
    expect = v[:, 0].astype(np.float64).mean(0) * T / (T + 1e-6)
    np.testing.assert_allclose(out, np.broadcast_to(expect, out.shape), rtol=1e-12, atol=1e-15)


def test_dominant_logit_selects_its_value():
    rng = np.random.default_rng(11)
    T, D = 50, 32
    k = np.zeros((T, 1, D), np.float32)
    k[17, 0, 0] = 1.0
    v = rng.standard_normal((T, 1, D)).astype(np.float32)
    q = np.zeros((1, D), np.float32)
    q[0, 0] = 1.0
    out = _one_seq(k, v, q, scale=200.0)  # logit 200 vs 0: others weigh e^-200
    np.testing.assert_allclose(out[0], v[17, 0].astype(np.float64) / (1 + 1e-6), rtol=1e-12, atol=1e-12)


def test_alibi_geometric_weights():
    # q = 0: logits are alibi only, slope * (t - ctx + 1); weights are a
    # geometric series r^(ctx-1-t), r = e^-slope.
    rng = np.random.default_rng(12)
    T, D = 30, 32
    k = rng.standard_normal((T, 1, D)).astype(np.float32)
    v = rng.standard_normal((T, 1, D)).astype(np.float32)
    q = np.zeros((2, D), np.float32)
    slopes = np.array([0.5, 0.125], np.float32)
    out = _one_seq(k, v, q, alibi=slopes)
    for h, s in enumerate(slopes.astype(np.float64)):
        r = math.exp(-s)
        w = r ** (T - 1 - np.arange(T))
        total = (1 - r ** T) / (1 - r)
        expect = (w[:, None] * v[:, 0]).sum(0) / (total + 1e-6)
        np.testing.assert_allclose(out[h], expect, rtol=1e-12, atol=1e-14)


def test_zero_output_kats():
    # test_paged_attention_kernel.py:332-378: ctx 0, ctx > max_seq_len; a
    # negative context read as uint32 is > max_seq_len as well.
    c = make_decode_case(13, B=3, Hq=2, Hkv=1, D=32, block_size=16, ctx_lo=16, ctx_hi=16,
                         cache_dtype="float16", q_dtype="float32", max_seq_len=16)
    c.context_lens[:] = [0, 16, -1]
    out = orc.paged_attention(c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens, 1, c.scale, 16, 8,
                              None, "float32", "float16")
    assert not out.any()
    out = orc.paged_attention(c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens, 1, c.scale, 16, 16,
                              None, "float32", "float16")
    assert not out[0].any() and out[1].any() and not out[2].any()


def test_block_permutation_invariance():
    c = make_decode_case(14, B=2, Hq=8, Hkv=2, D=64, block_size=16, ctx_lo=100, ctx_hi=200)
    base = orc.paged_attention(c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens, 2, c.scale, 16,
                               c.max_seq_len, None, "bfloat16", "bfloat16")
    rng = np.random.default_rng(15)
    perm = rng.permutation(c.k_cache.shape[0])  # new block j holds old block perm[j]
    inv = np.argsort(perm)
    bt = np.where(c.block_tables >= 0, inv[np.maximum(c.block_tables, 0)], -1).astype(np.int32)
    out = orc.paged_attention(c.q, c.k_cache[perm], c.v_cache[perm], bt, c.context_lens, 2, c.scale, 16,
                              c.max_seq_len, None, "bfloat16", "bfloat16")
    np.testing.assert_array_equal(out, base)


def test_gqa_group_shares_kv_head():
    c = make_decode_case(16, B=2, Hq=8, Hkv=2, D=64, block_size=16, ctx_lo=50, ctx_hi=90, q_dtype="float32",
                         cache_dtype="bfloat16")
    c.q[:, 1:4] = c.q[:, 0:1]   # heads 0..3 read KV head 0
    c.q[:, 4:8] = c.q[:, 0:1]   # heads 4..7 read KV head 1
    out = orc.paged_attention(c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens, 2, c.scale, 16,
                              c.max_seq_len, None, "float32", "bfloat16")
    for h in range(1, 4):
        np.testing.assert_array_equal(out[:, h], out[:, 0])
    for h in range(5, 8):
        np.testing.assert_array_equal(out[:, h], out[:, 4])
    assert np.abs(out[:, 4] - out[:, 0]).max() > 1e-3


@pytest.mark.parametrize("partition_size", [16, 48, 64, 256, 512])
def test_split_k_equals_single_pass(partition_size):
    c = make_decode_case(17 + partition_size, B=4, Hq=14, Hkv=2, D=64, block_size=16, ctx_lo=1, ctx_hi=1100,
                         alibi=True)
    c.context_lens[0] = partition_size       # exactly one partition
    c.context_lens[1] = partition_size + 1   # one token into the second
    one = orc.paged_attention(c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens, 2, c.scale, 16,
                              c.max_seq_len, c.alibi, "bfloat16", "bfloat16")
    split = orc.paged_attention_split(c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens, 2, c.scale, 16,
                                      c.max_seq_len, partition_size, c.alibi, "bfloat16", "bfloat16")
    np.testing.assert_allclose(split, one, rtol=1e-12, atol=1e-13)


# ---------------------------------------------------------------------------
# Planted mistakes: each must be caught by one of the checks above.
# ---------------------------------------------------------------------------


def test_planted_mistakes_are_caught(monkeypatch):
    c = make_decode_case(18, B=2, Hq=8, Hkv=2, D=64, block_size=16, ctx_lo=1, ctx_hi=60)
    ref = torch_sdpa_reference(c)

    def run():
        return orc.paged_attention(c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens, 2, c.scale, 16,
                                   c.max_seq_len, None, "bfloat16", "bfloat16")

    good = run()
    np.testing.assert_allclose(good, ref, rtol=2e-6, atol=2e-6)

    # Wrong GQA map: head h reads KV head h % Hkv instead of h // group.
    orig = orc._softmax_attend

    def wrong_gqa(qh, k, v, scale, bias):
        Hq = qh.shape[0]
        Hkv = k.shape[1]
        perm = np.array([(h % Hkv) * (Hq // Hkv) + h // Hkv for h in range(Hq)])
        return orig(qh[np.argsort(perm)], k, v, scale, bias)[perm]

    monkeypatch.setattr(orc, "_softmax_attend", wrong_gqa)
    assert np.abs(run() - ref).max() > 1e-2
    monkeypatch.setattr(orc, "_softmax_attend", orig)

    # Transposed K chunk index (d % x, d / x swapped) in the gather.
    orig_gather = orc.gather_kv

    def bad_gather(kc64, vc64, row, ctx):
        k, v = orig_gather(kc64, vc64, row, ctx)
        D = k.shape[-1]
        return k.reshape(ctx, -1, D // 8, 8).swapaxes(2, 3).reshape(ctx, -1, D), v

    monkeypatch.setattr(orc, "gather_kv", bad_gather)
    assert np.abs(run() - ref).max() > 1e-2
    monkeypatch.setattr(orc, "gather_kv", orig_gather)

    # ALiBi without the (ctx - 1) offset changes nothing (softmax shift
    # invariance) -- but a wrong sign does.
    c2 = make_decode_case(19, B=2, Hq=8, Hkv=2, D=64, block_size=16, ctx_lo=20, ctx_hi=60, alibi=True)
    ref2 = torch_sdpa_reference(c2)
    orig_bias = orc.alibi_bias
    monkeypatch.setattr(orc, "alibi_bias", lambda s, ctx: -orig_bias(s, ctx))
    bad = orc.paged_attention(c2.q, c2.k_cache, c2.v_cache, c2.block_tables, c2.context_lens, 2, c2.scale, 16,
                              c2.max_seq_len, c2.alibi, "bfloat16", "bfloat16")
    assert np.abs(bad - ref2).max() > 1e-2
    monkeypatch.setattr(orc, "alibi_bias", orig_bias)

    # Dropped 1e-6 in the denominator is caught by the single-token closed form.
    monkeypatch.setattr(orc, "_softmax_attend", lambda qh, k, v, scale, bias: np.repeat(
        v[0], qh.shape[0] // v.shape[1], axis=0) if k.shape[0] == 1 else orig(qh, k, v, scale, bias))
    with pytest.raises(AssertionError):
        test_single_token_returns_its_value()
