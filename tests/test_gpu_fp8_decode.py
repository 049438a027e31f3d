"""GPU parity of paged decode over FP8 E4M3 caches (paged 5-D layout,
x = 16) against the oracle, which attends in float64 over
decode(code) * k_scale and decode(code) * v_scale.  The caches are written by
the FP8 append from float inputs, as a server would fill them.  Covers the
persistent kernel (64 sequences x 8 KV heads) and the partition kernel,
split-K, every block size, head sizes, query types, GQA and ALiBi, and
caches holding exponent-15 codes (+-inf, NaN).  Tolerances as for the
16-bit caches of the same query type: bfloat16 1e-2 abs / 2e-2 rel, float16
and float32 queries (float16 operands) 2e-3 / 1e-2."""

import math

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from pkv_cases import normal
from pkv_torch import to_f64, to_index, to_torch
from sglang_mlx_amd import kernels

pytestmark = pytest.mark.gpu
FP8 = "fp8_e4m3"
TOL = {"bfloat16": (1e-2, 2e-2), "float16": (2e-3, 1e-2), "float32": (2e-3, 1e-2)}


def fp8_case(seed, B, Hq, Hkv, D, bs, ctx_lo, ctx_hi, q_dtype="bfloat16", alibi=False, k_scale=0.05,
             v_scale=0.02):
    rng = np.random.default_rng(seed)
    ctx = rng.integers(ctx_lo, ctx_hi + 1, size=B).astype(np.int32)
    nblk = -(-ctx // bs)
    nb = int(nblk.sum() * 1.1) + 2
    perm = rng.permutation(np.arange(1, nb))
    width = int(nblk.max())
    bt = np.full((B, width), -1, dtype=np.int32)
    pos = 0
    for s in range(B):
        bt[s, :nblk[s]] = perm[pos:pos + nblk[s]]
        pos += nblk[s]
    # Values about 10 standard deviations inside E4M3's finite range (240).
    kx = (rng.standard_normal((nb, Hkv, D // 16, bs, 16)) * 1.5).astype(np.float32)
    vx = (rng.standard_normal((nb, Hkv, D, bs)) * 0.5).astype(np.float32)
    kc = orc.fp8_e4m3_encode(kx / np.float32(k_scale) * np.float32(min(k_scale / 0.06, 1.0)))
    vc = orc.fp8_e4m3_encode(vx / np.float32(v_scale) * np.float32(min(v_scale / 0.02, 1.0)))
    q = normal(rng, (B, Hq, D), q_dtype)
    slopes = rng.uniform(0.01, 0.2, size=Hq).astype(np.float32) if alibi else None
    return dict(q=q, kc=kc, vc=vc, bt=bt, ctx=ctx, Hkv=Hkv, D=D, bs=bs, qd=q_dtype, alibi=slopes,
                scale=1.0 / math.sqrt(D), ks=k_scale, vs=v_scale)


def oracle(c):
    return orc.paged_attention(c["q"], c["kc"], c["vc"], c["bt"], c["ctx"], c["Hkv"], c["scale"], c["bs"],
                               int(c["bt"].shape[1] * c["bs"]), c["alibi"], q_dtype=c["qd"], cache_dtype=FP8,
                               k_scale=c["ks"], v_scale=c["vs"])


def run(c, partition_size=None):
    alibi = None if c["alibi"] is None else torch.from_numpy(c["alibi"]).cuda()
    args = (to_torch(c["q"], c["qd"]), to_torch(c["kc"], FP8), to_torch(c["vc"], FP8), to_index(c["bt"]),
            to_index(c["ctx"]), c["Hkv"], c["scale"], c["bs"], int(c["bt"].shape[1] * c["bs"]), alibi)
    if partition_size is None:
        out = kernels.paged_attention_v1(*args, k_scale=c["ks"], v_scale=c["vs"])
    else:
        out = kernels.paged_attention_v2(*args, partition_size=partition_size, k_scale=c["ks"], v_scale=c["vs"])
    torch.cuda.synchronize()
    return out


def check(c, partition_size=None):
    a, r = TOL[c["qd"]]
    np.testing.assert_allclose(to_f64(run(c, partition_size)), oracle(c), atol=a, rtol=r)


@pytest.mark.parametrize("bs", [8, 16, 32])
@pytest.mark.parametrize("q_dtype", ["bfloat16", "float16", "float32"])
def test_persistent(bs, q_dtype):
    # 64 x 8 = 512 (sequence, KV head) items: the persistent kernel.
    check(fp8_case(5000 + bs, B=64, Hq=32, Hkv=8, D=128, bs=bs, ctx_lo=1, ctx_hi=700, q_dtype=q_dtype))


@pytest.mark.parametrize("D", [32, 64, 80, 96, 112, 192, 256])
def test_head_sizes_partition_path(D):
    check(fp8_case(5100 + D, B=3, Hq=8, Hkv=2, D=D, bs=16, ctx_lo=1, ctx_hi=600))


@pytest.mark.parametrize("bs", [8, 32])
@pytest.mark.parametrize("D", [64, 192, 256])
def test_wide_head_sizes_block_sizes(D, bs):
    # Head sizes that are multiples of 64 load 16 K codes and 8 V codes per
    # lane (the query takes the permuted head dims); 8-token blocks take each
    # lane's block, 32-token blocks a token offset inside the block.
    check(fp8_case(5150 + D + bs, B=3, Hq=8, Hkv=2, D=D, bs=bs, ctx_lo=1, ctx_hi=600, q_dtype="float16"))
    check(fp8_case(5160 + D + bs, B=2, Hq=8, Hkv=2, D=D, bs=bs, ctx_lo=300, ctx_hi=900), partition_size=256)


@pytest.mark.parametrize("D", [64, 256])
def test_persistent_wide_head_sizes(D):
    check(fp8_case(5170 + D, B=64, Hq=16, Hkv=8, D=D, bs=16, ctx_lo=1, ctx_hi=500))


@pytest.mark.parametrize("bs", [8, 32])
def test_gqa7_alibi_split_k(bs):
    c = fp8_case(5200 + bs, B=4, Hq=28, Hkv=4, D=128, bs=bs, ctx_lo=100, ctx_hi=3000, q_dtype="float16",
                 alibi=True)
    check(c)
    check(c, partition_size=256)
    check(c, partition_size=2048)


def test_power_of_two_and_unit_scales():
    check(fp8_case(5300, B=5, Hq=8, Hkv=2, D=128, bs=16, ctx_lo=1, ctx_hi=300, k_scale=1.0, v_scale=0.0625))


def test_llama3_8b_layer():
    c = fp8_case(1003, B=64, Hq=32, Hkv=8, D=128, bs=16, ctx_lo=512, ctx_hi=4096)
    check(c)


@pytest.mark.parametrize("D,bs", [(64, 16), (128, 8), (96, 32)])
def test_exponent_15_codes(D, bs):
    # +-inf and NaN codes in K and V: rows where the oracle is non-finite are
    # exactly the kernel's non-finite rows (the hardware would read these
    # codes as E4M3FN numbers 256..448 without the fix-up).
    c = fp8_case(5400 + D + bs, B=8, Hq=8, Hkv=2, D=D, bs=bs, ctx_lo=20, ctx_hi=200)
    kc, vc, bt = c["kc"], c["vc"], c["bt"]
    kc[bt[0, 0], 0, 1, 3, 5] = 0x78   # +inf in K of sequence 0
    kc[bt[1, 0], 1, 0, 2, 0] = 0xF8   # -inf
    kc[bt[2, 0], 0, 2, 1, 7] = 0x7D   # NaN
    vc[bt[3, 0], 1, 9, 4] = 0x78      # +inf in V
    vc[bt[4, 0], 0, 3, 0] = 0xFB      # NaN
    got = to_f64(run(c))
    exp = oracle(c)
    np.testing.assert_array_equal(np.isfinite(got), np.isfinite(exp))
    fin = np.isfinite(exp)
    np.testing.assert_allclose(got[fin], exp[fin], atol=1e-2, rtol=2e-2)
    assert not np.isfinite(exp[0]).all() or not np.isfinite(exp[2]).all()


def test_append_then_decode_round_trip():
    # Values go in through reshape_and_cache (FP8, k/v scales) and come back
    # through the decode kernel; against the 16-bit cache path on the values
    # the codes stand for.
    rng = np.random.default_rng(9)
    Hkv, D, bs, nb, N = 4, 128, 16, 64, 700
    key = rng.standard_normal((N, Hkv, D)).astype(np.float32)
    value = rng.standard_normal((N, Hkv, D)).astype(np.float32)
    slots = np.arange(16, 16 + N, dtype=np.int32)
    kc = torch.zeros((nb, Hkv, D // 16, bs, 16), dtype=torch.uint8, device="cuda")
    vc = torch.zeros((nb, Hkv, D, bs), dtype=torch.uint8, device="cuda")
    kernels.reshape_and_cache(torch.from_numpy(key).cuda().bfloat16(), torch.from_numpy(value).cuda().bfloat16(),
                              kc, vc, to_index(slots), k_scale=0.03, v_scale=0.02)
    q = torch.randn((2, 16, D), device="cuda").bfloat16()
    bt = torch.arange(1, 1 + 45, dtype=torch.int32, device="cuda").view(1, 45).repeat(2, 1)
    lens = torch.tensor([N, N // 2], dtype=torch.int32, device="cuda")
    out = kernels.paged_attention_v1(q, kc, vc, bt, lens, Hkv, 1 / math.sqrt(D), bs, 45 * bs, k_scale=0.03,
                                     v_scale=0.02)
    torch.cuda.synchronize()
    kf = (orc.fp8_e4m3_decode(kc.cpu().numpy()) * np.float32(0.03)).astype(np.float32)
    vf = (orc.fp8_e4m3_decode(vc.cpu().numpy()) * np.float32(0.02)).astype(np.float32)
    exp = orc.paged_attention(q.float().cpu().numpy(), kf, vf, bt.cpu().numpy(), lens.cpu().numpy(), Hkv,
                              1 / math.sqrt(D), bs, 45 * bs)
    np.testing.assert_allclose(to_f64(out), exp, atol=1e-2, rtol=2e-2)
