"""GPU parity of the FP8 append (reshape_and_cache into uint8 caches of E4M3
codes) against the oracle, bit for bit over whole caches: every source
dtype, the paged 5-D layout (x = 16, block sizes 8/16/32), the token-major
MHATokenPool buffer and the flash layout, power-of-two and general scales.
Sources span the codec's whole range (subnormals, the 2^-6 wrap, values
past 240 and past 256, specials) so the encoder's every branch is written
through the kernel; caches start from random bytes so untouched slots are
checked too."""

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from pkv_cases import run_slots
from pkv_torch import to_index, to_numpy, to_torch
from sglang_mlx_amd import kernels, _ext

pytestmark = pytest.mark.gpu
FP8 = "fp8_e4m3"


def wide_values(rng, shape, dtype):
    x = rng.standard_normal(shape) * np.exp2(rng.uniform(-12, 9, size=shape))
    flat = x.reshape(-1)
    flat[::97] = np.inf
    flat[5::97] = -np.inf
    flat[11::97] = np.nan
    flat[17::97] = 0.0
    flat[23::97] = -0.0
    flat[29::97] = 300.0
    flat[31::97] = 2.0 ** -6 - 2.0 ** -11
    return orc.to_storage(x.astype(np.float32), dtype)


def case(seed, N, H, D, num_slots, kv_dtype):
    rng = np.random.default_rng(seed)
    slots = (rng.choice(num_slots - 1, size=N, replace=False) + 1).astype(np.int32)
    slots[rng.choice(N, size=max(1, N // 20), replace=False)] = -1
    return wide_values(rng, (N, H, D), kv_dtype), wide_values(rng, (N, H, D), kv_dtype), slots, rng


@pytest.mark.parametrize("kv_dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("bs", [8, 16, 32])
@pytest.mark.parametrize("scales", [(1.0, 1.0), (0.5, 4.0), (0.37, 1.7)])
def test_paged5d(kv_dtype, bs, scales):
    H, D, nb = 4, 128, 40
    key, value, slots, rng = case(bs, 200, H, D, nb * bs, kv_dtype)
    kc0 = rng.integers(0, 256, size=(nb, H, D // 16, bs, 16), dtype=np.uint8)
    vc0 = rng.integers(0, 256, size=(nb, H, D, bs), dtype=np.uint8)
    kc, vc = to_torch(kc0, FP8), to_torch(vc0, FP8)
    out = kernels.reshape_and_cache(to_torch(key, kv_dtype), to_torch(value, kv_dtype), kc, vc, to_index(slots),
                                    k_scale=scales[0], v_scale=scales[1])
    assert out[0] is kc
    torch.cuda.synchronize()
    rk, rv = orc.reshape_and_cache_paged5d(key, value, kc0, vc0, slots, kv_dtype, FP8, *scales)
    np.testing.assert_array_equal(to_numpy(kc), rk)
    np.testing.assert_array_equal(to_numpy(vc), rv)


@pytest.mark.parametrize("kv_dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("bs", [16, 32])
def test_paged5d_large_append_of_slot_runs(kv_dtype, bs):
    # 4096 tokens x 8 heads x D 128 whose slots come in runs: whole blocks
    # are written as 16-byte units of 16 codes gathered over the run's
    # tokens, the rest per token; the whole cache is compared.
    H, D = 8, 128
    nb = 1024 if bs == 16 else 600
    rng = np.random.default_rng(77 + bs)
    slots = run_slots(rng, 4096, nb, bs)
    key, value = wide_values(rng, (4096, H, D), kv_dtype), wide_values(rng, (4096, H, D), kv_dtype)
    kc0 = rng.integers(0, 256, size=(nb, H, D // 16, bs, 16), dtype=np.uint8)
    vc0 = rng.integers(0, 256, size=(nb, H, D, bs), dtype=np.uint8)
    kc, vc = to_torch(kc0, FP8), to_torch(vc0, FP8)
    kernels.reshape_and_cache(to_torch(key, kv_dtype), to_torch(value, kv_dtype), kc, vc, to_index(slots),
                              k_scale=0.37, v_scale=1.7)
    torch.cuda.synchronize()
    rk, rv = orc.reshape_and_cache_paged5d(key, value, kc0, vc0, slots, kv_dtype, FP8, 0.37, 1.7)
    np.testing.assert_array_equal(to_numpy(kc), rk)
    np.testing.assert_array_equal(to_numpy(vc), rv)


@pytest.mark.parametrize("kv_dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("D", [64, 80, 120, 128, 256])
@pytest.mark.parametrize("flash", [False, True])
def test_token_major_and_flash(kv_dtype, D, flash):
    H, num_slots = 8, 1024
    key, value, slots, rng = case(D, 300, H, D, num_slots, kv_dtype)
    kc0 = rng.integers(0, 256, size=(num_slots, H, D), dtype=np.uint8)
    vc0 = rng.integers(0, 256, size=(num_slots, H, D), dtype=np.uint8)
    kc, vc = to_torch(kc0, FP8), to_torch(vc0, FP8)
    k, v, s = to_torch(key, kv_dtype), to_torch(value, kv_dtype), to_index(slots)
    if flash:
        _ext.reshape_and_cache_flash(k, v, kc.view(64, 16, H, D), vc.view(64, 16, H, D), s, 0.37, 2.0)
    else:
        kernels.reshape_and_cache(k, v, kc, vc, s, k_scale=0.37, v_scale=2.0)
    torch.cuda.synchronize()
    rk, rv = orc.reshape_and_cache_token_major(key, value, kc0, vc0, slots, kv_dtype, FP8, 0.37, 2.0)
    np.testing.assert_array_equal(to_numpy(kc), rk)
    np.testing.assert_array_equal(to_numpy(vc), rv)


def test_strided_source_rows():
    # Rows of a wider buffer (stride > H*D) go in as they are.
    H, D, num_slots = 8, 128, 512
    key, value, slots, rng = case(3, 100, H, D, num_slots, "bfloat16")
    wide_k = np.zeros((100, H * D + 64), dtype=np.uint16)
    wide_k[:, :H * D] = key.reshape(100, -1)
    kt = to_torch(wide_k, "bfloat16")[:, :H * D].view(100, H, D)
    kc = torch.zeros((num_slots, H, D), dtype=torch.uint8, device="cuda")
    vc = torch.zeros_like(kc)
    kernels.reshape_and_cache(kt, to_torch(value, "bfloat16"), kc, vc, to_index(slots), k_scale=0.25, v_scale=0.25)
    torch.cuda.synchronize()
    rk, rv = orc.reshape_and_cache_token_major(key, value, np.zeros((num_slots, H, D), np.uint8),
                                               np.zeros((num_slots, H, D), np.uint8), slots, "bfloat16", FP8,
                                               0.25, 0.25)
    np.testing.assert_array_equal(to_numpy(kc), rk)
    np.testing.assert_array_equal(to_numpy(vc), rv)


def test_rejections():
    kc = torch.zeros((16, 8, 128), dtype=torch.uint8, device="cuda")
    k = torch.zeros((4, 8, 128), dtype=torch.bfloat16, device="cuda")
    s = torch.arange(4, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="finite and nonzero"):
        kernels.reshape_and_cache(k, k, kc, kc.clone(), s, k_scale=0.0)
    with pytest.raises(ValueError, match="16-byte aligned"):
        kb = torch.zeros((4 * 8 * 128 + 8,), dtype=torch.bfloat16, device="cuda")[4:4 + 4 * 8 * 128].view(4, 8, 128)
        kernels.reshape_and_cache(kb, kb, kc, kc.clone(), s)


@pytest.mark.parametrize("start", [0, 7])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_paged5d_consecutive_slots(start, D):
    # Slots start .. start+N-1, as a prefill writes them: whole blocks in the
    # middle, partial blocks at the ends.
    H, nb, bs, N = 4, 64, 16, 700
    rng = np.random.default_rng(D + start)
    key, value = wide_values(rng, (N, H, D), "bfloat16"), wide_values(rng, (N, H, D), "bfloat16")
    slots = np.arange(start, start + N, dtype=np.int32)
    kc0 = rng.integers(0, 256, size=(nb, H, D // 16, bs, 16), dtype=np.uint8)
    vc0 = rng.integers(0, 256, size=(nb, H, D, bs), dtype=np.uint8)
    kc, vc = to_torch(kc0, FP8), to_torch(vc0, FP8)
    kernels.reshape_and_cache(to_torch(key, "bfloat16"), to_torch(value, "bfloat16"), kc, vc, to_index(slots),
                              k_scale=0.5, v_scale=4.0)
    torch.cuda.synchronize()
    rk, rv = orc.reshape_and_cache_paged5d(key, value, kc0, vc0, slots, "bfloat16", FP8, 0.5, 4.0)
    np.testing.assert_array_equal(to_numpy(kc), rk)
    np.testing.assert_array_equal(to_numpy(vc), rv)
