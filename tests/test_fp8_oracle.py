"""Pins the oracle's FP8 E4M3 codec (float8.metal) and convert_fp8
(convert_fp8.metal) on the CPU.

* Decode: the 240 codes whose exponent is below 15 mean the same in the
  reference's format and OCP E4M3FN, so torch's float8_e4m3fn decoding is an
  independent check of them; exponent 15 is +-inf / NaN in the reference.
* Encode: every finite code survives decode -> encode; in the normal range
  the result equals torch's round-to-nearest-even conversion; in the
  subnormal range a brute-force search over the nine multiples of 2^-9 with
  the reference's tie rule (half up) and wrap (2^-6 -> 0) gives the same
  codes; the reference's fall-through for 256 <= |x| < 2^14 and the specials
  are checked as known answers.
"""

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc

CODES = np.arange(256, dtype=np.uint8)
FINITE = CODES[((CODES >> 3) & 0xF) != 15]


def torch_fn_decode(codes):
    return torch.from_numpy(np.asarray(codes, dtype=np.uint8)).view(torch.float8_e4m3fn).float().numpy()


def torch_fn_encode(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_shared_codes_match_e4m3fn():
    got = orc.fp8_e4m3_decode(FINITE)
    exp = torch_fn_decode(FINITE)
    assert len(FINITE) == 240
    np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_decode_known_values_and_exponent_15():
    d = orc.fp8_e4m3_decode(CODES)
    assert d[0x38] == 1.0 and d[0x40] == 2.0 and d[0xB8] == -1.0
    assert d[0x77] == 240.0 and d[0xF7] == -240.0          # largest finite
    assert d[0x08] == 2.0 ** -6 and d[0x01] == 2.0 ** -9    # smallest normal / subnormal
    assert d[0x07] == 7 * 2.0 ** -9
    assert d[0x00] == 0.0 and np.signbit(d[0x80])
    assert d[0x78] == np.inf and d[0xF8] == -np.inf
    for c in list(range(0x79, 0x80)) + list(range(0xF9, 0x100)):
        assert d[c:c + 1].view(np.uint32)[0] == 0x7FC00000, hex(c)   # unsigned NAN (float8.metal:29-30)
    # So a negative NaN code re-encodes as the positive NaN code.
    assert orc.convert_fp8(np.uint8([0xFA]), "fp8_e4m3", "fp8_e4m3", 1.0)[0] == 0x79


def test_encode_round_trips_every_finite_code():
    np.testing.assert_array_equal(orc.fp8_e4m3_encode(orc.fp8_e4m3_decode(FINITE)), FINITE)


def test_encode_normal_range_is_round_to_nearest_even():
    rng = np.random.default_rng(0)
    mag = np.exp2(rng.uniform(-6, np.log2(256), size=200000)).astype(np.float32)
    mag = mag[(mag >= 2.0 ** -6) & (mag < 256)]
    x = np.concatenate([mag, -mag])
    # Exact ties: midpoints between neighbouring finite codes.
    pos = orc.fp8_e4m3_decode(np.arange(0x08, 0x78, dtype=np.uint8)).astype(np.float64)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids, np.float32([248.0, -248.0, 240.0, 247.99998])])
    np.testing.assert_array_equal(orc.fp8_e4m3_encode(x), torch_fn_encode(x))


def test_encode_subnormal_range_by_search():
    rng = np.random.default_rng(1)
    x = rng.uniform(2.0 ** -9, 2.0 ** -6, size=100000).astype(np.float32)
    ties = ((np.arange(1, 8) + 0.5) * 2.0 ** -9).astype(np.float32)   # exact midpoints
    x = np.concatenate([x, ties, np.float32([2.0 ** -9, 2.0 ** -6 - 2.0 ** -30])])
    x = x[(x >= 2.0 ** -9) & (x < 2.0 ** -6)]
    cand = np.arange(9, dtype=np.float64) * 2.0 ** -9
    xd = x.astype(np.float64)[:, None]
    dist = np.abs(xd - cand[None, :])
    best = dist.min(axis=1, keepdims=True)
    k = np.where(dist == best, np.arange(9)[None, :], -1).max(axis=1)  # ties go up
    exp = np.where(k == 8, 0, k).astype(np.uint8)                     # 2^-6 wraps to 0
    np.testing.assert_array_equal(orc.fp8_e4m3_encode(x), exp)
    np.testing.assert_array_equal(orc.fp8_e4m3_encode(-x), (exp | 0x80).astype(np.uint8))
    # The midpoints round up (k + 1), where round-to-nearest-even would not.
    np.testing.assert_array_equal(orc.fp8_e4m3_encode(ties), np.arange(2, 9) % 8)


def test_encode_below_two_to_minus_nine_is_zero():
    # The reference returns +-0 once the biased exponent is below -2
    # (|x| < 2^-9), even where 2^-9 would be nearer.
    x = np.float32([2.0 ** -10, 1.5 * 2.0 ** -10, 1.99 * 2.0 ** -10, 1e-30, 1e-45])
    np.testing.assert_array_equal(orc.fp8_e4m3_encode(x), 0)
    np.testing.assert_array_equal(orc.fp8_e4m3_encode(-x), 0x80)


def test_encode_specials_and_overflow_behaviour():
    e = orc.fp8_e4m3_encode
    assert e(np.float32([np.inf]))[0] == 0x78 and e(np.float32([-np.inf]))[0] == 0xF8
    assert e(np.float32([np.nan]))[0] == 0x79 and e(-np.float32([np.nan]))[0] == 0xF9
    assert e(np.float32([0.0]))[0] == 0x00 and e(np.float32([-0.0]))[0] == 0x80
    assert e(np.float32([248.0]))[0] == 0x78 and e(np.float32([255.9]))[0] == 0x78   # carry past 2^7 -> inf
    # 256 <= |x| < 2^14: the reference's subnormal branch keeps 3 low bits.
    assert e(np.float32([256.0]))[0] == 0x00 and e(np.float32([300.0]))[0] == 0x00
    assert e(np.float32([8192.001953125]))[0] == 0x01 and e(np.float32([-8192.001953125]))[0] == 0x81
    assert e(np.float32([16383.0]))[0] == 0x00
    # |x| >= 2^14: undefined shifts in the reference, +-inf here.
    assert e(np.float32([16384.0]))[0] == 0x78 and e(np.float32([-3e38]))[0] == 0xF8


@pytest.mark.parametrize("src,dst", [
    ("fp8_e4m3", "float32"), ("fp8_e4m3", "float16"), ("fp8_e4m3", "bfloat16"),
    ("float32", "fp8_e4m3"), ("float16", "fp8_e4m3"), ("bfloat16", "fp8_e4m3"), ("fp8_e4m3", "fp8_e4m3"),
    ("float32", "float16"), ("bfloat16", "float32"), ("float16", "bfloat16"),
])
def test_convert_fp8_against_torch(src, dst):
    rng = np.random.default_rng(2)
    scale = 0.37
    if src == "fp8_e4m3":
        s = FINITE[rng.integers(0, len(FINITE), size=4096)]
        val = torch.from_numpy(torch_fn_decode(s))
    else:
        val = torch.from_numpy((rng.standard_normal(4096) * 30).astype(np.float32))
        val = val.to({"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[src]).float()
        s = orc.to_storage(val.numpy(), src)
    got = orc.convert_fp8(s, src, dst, scale)
    if dst == "fp8_e4m3":
        v = (val / torch.tensor(scale, dtype=torch.float32)) if src != "fp8_e4m3" else val * scale
        v = v.float().numpy()
        keep = (np.abs(v) < 240) & (np.abs(v) >= 2.0 ** -6)
        np.testing.assert_array_equal(got[keep], torch_fn_encode(v[keep]))
    else:
        v = val * scale
        tdt = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[dst]
        exp = orc.to_storage(v.to(tdt).float().numpy(), dst)
        np.testing.assert_array_equal(got, exp)


def test_fp8_cache_attention_is_attention_over_dequantised_caches():
    # The FP8 branch of the attention oracle equals the pinned float32 path
    # run on decode(code) * scale.
    rng = np.random.default_rng(3)
    B, Hq, Hkv, D, bs, nb = 3, 8, 2, 64, 16, 12
    kc = orc.fp8_e4m3_encode(rng.standard_normal((nb, Hkv, D // 16, bs, 16)).astype(np.float32) / 0.5)
    vc = orc.fp8_e4m3_encode(rng.standard_normal((nb, Hkv, D, bs)).astype(np.float32) / 0.25)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    bt = rng.permutation(nb)[:B * 4].reshape(B, 4).astype(np.int32)
    ctx = np.array([1, 37, 64], dtype=np.int32)
    got = orc.paged_attention(q, kc, vc, bt, ctx, Hkv, 0.125, bs, 64, cache_dtype="fp8_e4m3",
                              k_scale=0.5, v_scale=0.25)
    kf = (orc.fp8_e4m3_decode(kc) * np.float32(0.5)).astype(np.float32)
    vf = (orc.fp8_e4m3_decode(vc) * np.float32(0.25)).astype(np.float32)
    exp = orc.paged_attention(q, kf, vf, bt, ctx, Hkv, 0.125, bs, 64)
    np.testing.assert_allclose(got, exp, rtol=1e-12, atol=1e-12)
