"""GPU parity of the FP8 E4M3 codec and convert_fp8 (convert_fp8.metal)
against the oracle, bit for bit.

Decoding covers all 256 codes into every wider type at two scales (the
hardware conversion plus the exponent-15 fix-up); encoding covers every
float16 and bfloat16 bit pattern and float32 inputs drawn from all 256
exponents, with the encoder's boundary cases (2^-6 wrap, 248 carry, the
256 <= |x| < 2^14 fall-through, 2^14 and up, specials) listed explicitly."""

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from sglang_mlx_amd import kernels

pytestmark = pytest.mark.gpu

TORCH = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16, "fp8_e4m3": torch.uint8}
NP_BITS = {"float32": np.float32, "float16": np.uint16, "bfloat16": np.uint16, "fp8_e4m3": np.uint8}


def to_dev(arr, dtype):
    a = np.ascontiguousarray(arr)
    if dtype in ("float16", "bfloat16"):
        return torch.from_numpy(a.view(np.int16)).cuda().view(TORCH[dtype])
    return torch.from_numpy(a).cuda()


def to_host(t, dtype):
    if dtype in ("float16", "bfloat16"):
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def run(src_arr, src_dtype, dst_dtype, scale):
    src = to_dev(src_arr, src_dtype)
    dst = torch.empty(src.numel(), dtype=TORCH[dst_dtype], device="cuda")
    kernels.convert_fp8(dst, src, scale)
    torch.cuda.synchronize()
    return to_host(dst, dst_dtype)


def same_bits(got, exp):
    if got.dtype == np.float32:
        got, exp = got.view(np.uint32), exp.view(np.uint32)
    np.testing.assert_array_equal(got, exp)


def f32_sample(seed=0):
    rng = np.random.default_rng(seed)
    exps = np.repeat(np.arange(256, dtype=np.uint32), 512)
    mants = rng.integers(0, 1 << 23, size=exps.size, dtype=np.uint32)
    mants[::7] &= 0x7F0000  # short mantissas: exact ties and carries
    bits = (exps << 23) | mants
    x = np.concatenate([bits, bits | 0x80000000]).view(np.float32)
    extra = np.float32([0.0, -0.0, np.inf, -np.inf, np.nan, 248.0, -248.0, 255.9, 256.0, 300.0, 8192.001953125,
                        16383.0, 16384.0, 3e38, 2.0 ** -6 - 2.0 ** -11, 2.0 ** -6, 2.0 ** -9, 2.0 ** -10,
                        1.5 * 2.0 ** -9, 2.5 * 2.0 ** -9, 240.0, 1e-45])
    return np.concatenate([x, extra, -extra])


@pytest.mark.parametrize("dst", ["float32", "float16", "bfloat16", "fp8_e4m3"])
@pytest.mark.parametrize("scale", [1.0, 0.37])
def test_decode_every_code(dst, scale):
    codes = np.tile(np.arange(256, dtype=np.uint8), 9)[:2301]  # not a multiple of 8: tail path too
    same_bits(run(codes, "fp8_e4m3", dst, scale), orc.convert_fp8(codes, "fp8_e4m3", dst, scale))


@pytest.mark.parametrize("src", ["float16", "bfloat16"])
@pytest.mark.parametrize("scale", [1.0, 0.37, 3.0])
def test_encode_every_16_bit_pattern(src, scale):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    same_bits(run(bits, src, "fp8_e4m3", scale), orc.convert_fp8(bits, src, "fp8_e4m3", scale))


@pytest.mark.parametrize("scale", [1.0, 2.5, 1 / 64])
def test_encode_float32_all_exponents(scale):
    x = f32_sample()
    same_bits(run(x, "float32", "fp8_e4m3", scale), orc.convert_fp8(x, "float32", "fp8_e4m3", scale))


@pytest.mark.parametrize("src,dst", [(s, d) for s in ("float32", "float16", "bfloat16")
                                     for d in ("float32", "float16", "bfloat16")])
def test_wide_pairs(src, dst):
    x = f32_sample(1)
    s = orc.to_storage(x, src)
    same_bits(run(s, src, dst, 0.75), orc.convert_fp8(s, src, dst, 0.75))


def test_unaligned_and_strided_views():
    # Offset views (not 16-byte aligned) take the scalar path; a strided
    # source is made contiguous first.
    codes = np.arange(256, dtype=np.uint8)
    src = to_dev(np.tile(codes, 2), "fp8_e4m3")[3:259]
    dst_full = torch.zeros(300, dtype=torch.bfloat16, device="cuda")
    dst = dst_full[5:261]
    kernels.convert_fp8(dst, src, 1.0)
    torch.cuda.synchronize()
    exp = orc.convert_fp8(np.tile(codes, 2)[3:259], "fp8_e4m3", "bfloat16", 1.0)
    same_bits(to_host(dst, "bfloat16"), exp)
    assert not dst_full[:5].view(torch.int16).any() and not dst_full[261:].view(torch.int16).any()
    x = torch.randn(64, 16, device="cuda")
    out = torch.empty(64 * 8, dtype=torch.uint8, device="cuda")
    kernels.convert_fp8(out, x[:, ::2], 0.5)
    torch.cuda.synchronize()
    same_bits(out.cpu().numpy(), orc.convert_fp8(x[:, ::2].contiguous().cpu().numpy().ravel(), "float32",
                                                 "fp8_e4m3", 0.5))
