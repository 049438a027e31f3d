"""GPU parity of reshape_and_cache against the oracle: bit-exact, whole caches.

Cases: the reference test's fixture geometry and shape sweep
(tests/test_paged_attention_kernel.py:138-210, :248-282), every
(kv dtype -> cache dtype) pair of reshape_and_cache.metal:91-95 in both
layouts, strided and misaligned sources, padding-only and empty batches,
the 4096-token append workload at full size (65,536 slots, 5% padding), and
large appends whose slots come in runs of consecutive slots (whole and
partial blocks, as a prefill writes them) mixed with scattered slots.
Caches start from random bits so untouched slots are checked too.
"""

import dataclasses

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from pkv_cases import X_OF, make_append_case, make_run_append_case
from pkv_torch import to_index, to_numpy, to_torch
from sglang_mlx_amd import _ext

pytestmark = pytest.mark.gpu


def random_bits(rng, shape, dtype):
    if dtype == "float32":
        return rng.standard_normal(shape, dtype=np.float32)
    return orc.to_storage(rng.standard_normal(shape, dtype=np.float32), dtype)


def check_paged5d(case, nb, H, D, seed=7):
    x, bs = X_OF[case.cache_dtype], case.block_size
    rng = np.random.default_rng(seed)
    kc0 = random_bits(rng, (nb, H, D // x, bs, x), case.cache_dtype)
    vc0 = random_bits(rng, (nb, H, D, bs), case.cache_dtype)
    kc, vc = to_torch(kc0, case.cache_dtype), to_torch(vc0, case.cache_dtype)
    out = _ext.reshape_and_cache(to_torch(case.key, case.kv_dtype), to_torch(case.value, case.kv_dtype),
                                 kc, vc, to_index(case.slot_mapping))
    assert isinstance(out, list) and out[0] is kc and out[1] is vc
    torch.cuda.synchronize()
    rk, rv = orc.reshape_and_cache_paged5d(case.key, case.value, kc0, vc0, case.slot_mapping,
                                           case.kv_dtype, case.cache_dtype)
    np.testing.assert_array_equal(to_numpy(kc), rk)
    np.testing.assert_array_equal(to_numpy(vc), rv)


def check_token_major(case, H, D, flash_blocks=None, seed=8):
    rng = np.random.default_rng(seed)
    shape = (case.num_slots, H, D)
    kc0 = random_bits(rng, shape, case.cache_dtype)
    vc0 = random_bits(rng, shape, case.cache_dtype)
    kc, vc = to_torch(kc0, case.cache_dtype), to_torch(vc0, case.cache_dtype)
    key, value = to_torch(case.key, case.kv_dtype), to_torch(case.value, case.kv_dtype)
    if flash_blocks:
        kf = kc.view(flash_blocks, -1, H, D)
        vf = vc.view(flash_blocks, -1, H, D)
        out = _ext.reshape_and_cache_flash(key, value, kf, vf, to_index(case.slot_mapping))
        assert out[0] is kf
    else:
        out = _ext.reshape_and_cache(key, value, kc, vc, to_index(case.slot_mapping))
        assert out[0] is kc
    torch.cuda.synchronize()
    rk, rv = orc.reshape_and_cache_token_major(case.key, case.value, kc0, vc0, case.slot_mapping,
                                               case.kv_dtype, case.cache_dtype)
    np.testing.assert_array_equal(to_numpy(kc), rk)
    np.testing.assert_array_equal(to_numpy(vc), rv)


def test_reference_fixture_geometry():
    # test_paged_attention_kernel.py:138-188: 4 KV heads, D 64, bs 16, 20
    # blocks, float32 K/V into a float16 cache, slots 0..24 and 32..81.
    rng = np.random.default_rng(11)
    key = rng.standard_normal((75, 4, 64), dtype=np.float32)
    value = rng.standard_normal((75, 4, 64), dtype=np.float32)
    slots = np.array(list(range(25)) + [32 + i for i in range(50)], dtype=np.int32)
    from pkv_cases import AppendCase
    case = AppendCase(key, value, slots, 20 * 16, 16, "float32", "float16")
    check_paged5d(case, 20, 4, 64)


@pytest.mark.parametrize("head_dim", [32, 128])
@pytest.mark.parametrize("block_size", [8, 16])
def test_reference_shape_sweep(head_dim, block_size):
    # test_paged_attention_kernel.py:248-266: 16 tokens, 2 KV heads, 4 blocks.
    rng = np.random.default_rng(head_dim * 100 + block_size)
    key = rng.standard_normal((16, 2, head_dim), dtype=np.float32)
    value = rng.standard_normal((16, 2, head_dim), dtype=np.float32)
    from pkv_cases import AppendCase
    case = AppendCase(key, value, np.arange(16, dtype=np.int32), 4 * block_size, block_size,
                      "float32", "float16")
    check_paged5d(case, 4, 2, head_dim)


PAIRS = [("bfloat16", "bfloat16"), ("float16", "float16"), ("float32", "float32"),
         ("float32", "float16"), ("float32", "bfloat16")]


@pytest.mark.parametrize("kv_dtype,cache_dtype", PAIRS)
@pytest.mark.parametrize("layout", ["paged5d", "token_major"])
def test_dtype_pairs(kv_dtype, cache_dtype, layout):
    case = make_append_case(21, N=300, H=4, D=128, num_slots=64 * 16, block_size=16,
                            kv_dtype=kv_dtype, cache_dtype=cache_dtype)
    if layout == "paged5d":
        check_paged5d(case, 64, 4, 128)
    else:
        check_token_major(case, 4, 128)


@pytest.mark.parametrize("block_size", [8, 16, 32])
@pytest.mark.parametrize("head_dim", [64, 80, 120, 256])
def test_paged5d_shapes(block_size, head_dim):
    case = make_append_case(31 + head_dim, N=100, H=2, D=head_dim, num_slots=32 * block_size,
                            block_size=block_size)
    check_paged5d(case, 32, 2, head_dim)


@pytest.mark.parametrize("H,D,cache_dtype", [(3, 128, "bfloat16"),   # 48 vectors: one token per workgroup
                                             (5, 128, "bfloat16"),   # 80 vectors: ragged lanes
                                             (32, 256, "bfloat16"),  # 1024 vectors: eight passes
                                             (2, 128, "float32"),    # 64 float32 vectors
                                             (7, 96, "float16")])    # 84 vectors
def test_token_major_row_lengths(H, D, cache_dtype):
    case = make_append_case(81 + H, N=70, H=H, D=D, num_slots=16 * 16, block_size=16,
                            kv_dtype="float32" if cache_dtype == "float32" else cache_dtype,
                            cache_dtype=cache_dtype)
    check_token_major(case, H, D)


def test_token_major_strided_source():
    # Source rows 2*H*D apart (a slice of a wider projection output).
    case = make_append_case(91, N=64, H=8, D=128, num_slots=32 * 16, block_size=16)
    rng = np.random.default_rng(4)
    kc0 = random_bits(rng, (case.num_slots, 8, 128), "bfloat16")
    vc0 = random_bits(rng, (case.num_slots, 8, 128), "bfloat16")
    rk, rv = orc.reshape_and_cache_token_major(case.key, case.value, kc0, vc0, case.slot_mapping,
                                               "bfloat16", "bfloat16")
    wide_k = torch.zeros((64, 16, 128), dtype=torch.bfloat16, device="cuda")
    wide_v = torch.zeros_like(wide_k)
    wide_k[:, :8] = to_torch(case.key, "bfloat16")
    wide_v[:, :8] = to_torch(case.value, "bfloat16")
    kc, vc = to_torch(kc0, "bfloat16"), to_torch(vc0, "bfloat16")
    _ext.reshape_and_cache(wide_k[:, :8], wide_v[:, :8], kc, vc, to_index(case.slot_mapping))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_numpy(kc), rk)
    np.testing.assert_array_equal(to_numpy(vc), rv)


def test_flash_layout_4d():
    case = make_append_case(41, N=200, H=8, D=64, num_slots=64 * 16, block_size=16)
    check_token_major(case, 8, 64, flash_blocks=64)


def test_strided_and_misaligned_sources():
    case = make_append_case(51, N=64, H=4, D=128, num_slots=32 * 16, block_size=16)
    x = X_OF["bfloat16"]
    rng = np.random.default_rng(3)
    kc0 = random_bits(rng, (32, 4, 128 // x, 16, x), "bfloat16")
    vc0 = random_bits(rng, (32, 4, 128, 16), "bfloat16")
    rk, rv = orc.reshape_and_cache_paged5d(case.key, case.value, kc0, vc0, case.slot_mapping,
                                           "bfloat16", "bfloat16")
    key, value = to_torch(case.key, "bfloat16"), to_torch(case.value, "bfloat16")
    # Row stride 2*H*D (a slice of a wider projection output).
    wide_k = torch.zeros((64, 8, 128), dtype=torch.bfloat16, device="cuda")
    wide_v = torch.zeros_like(wide_k)
    wide_k[:, :4] = key
    wide_v[:, :4] = value
    # Base address off by one element (2 bytes): the unaligned kernel path.
    flat_k = torch.zeros(64 * 4 * 128 + 1, dtype=torch.bfloat16, device="cuda")
    flat_v = torch.zeros_like(flat_k)
    flat_k[1:] = key.reshape(-1)
    flat_v[1:] = value.reshape(-1)
    for k_in, v_in in ((wide_k[:, :4], wide_v[:, :4]),
                       (flat_k[1:].view(64, 4, 128), flat_v[1:].view(64, 4, 128))):
        kc, vc = to_torch(kc0, "bfloat16"), to_torch(vc0, "bfloat16")
        _ext.reshape_and_cache(k_in, v_in, kc, vc, to_index(case.slot_mapping))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_numpy(kc), rk)
        np.testing.assert_array_equal(to_numpy(vc), rv)


def test_padding_only_and_empty():
    case = make_append_case(61, N=32, H=2, D=64, num_slots=16 * 16, block_size=16)
    case.slot_mapping[:] = -1
    check_paged5d(case, 16, 2, 64)
    check_token_major(case, 2, 64)
    empty = make_append_case(62, N=0, H=2, D=64, num_slots=16 * 16, block_size=16)
    check_paged5d(empty, 16, 2, 64)


def test_int64_slot_mapping_is_accepted():
    case = make_append_case(71, N=50, H=2, D=64, num_slots=16 * 16, block_size=16)
    rng = np.random.default_rng(5)
    kc0 = random_bits(rng, (16, 2, 8, 16, 8), "bfloat16")
    vc0 = random_bits(rng, (16, 2, 64, 16), "bfloat16")
    kc, vc = to_torch(kc0, "bfloat16"), to_torch(vc0, "bfloat16")
    _ext.reshape_and_cache(to_torch(case.key, "bfloat16"), to_torch(case.value, "bfloat16"), kc, vc,
                           to_index(case.slot_mapping, dtype=torch.int64))
    torch.cuda.synchronize()
    rk, rv = orc.reshape_and_cache_paged5d(case.key, case.value, kc0, vc0, case.slot_mapping,
                                           "bfloat16", "bfloat16")
    np.testing.assert_array_equal(to_numpy(kc), rk)
    np.testing.assert_array_equal(to_numpy(vc), rv)


@pytest.mark.parametrize("layout", ["token_major", "paged5d"])
def test_append_workload_full_size(layout):
    # 4096 new tokens, 8 KV heads, D 128, bf16, 65,536 slots in 4096 blocks of
    # 16, unique random slots, 5% padding; the whole pool is compared.
    case = make_append_case(1002, N=4096, H=8, D=128, num_slots=65536, block_size=16)
    if layout == "token_major":
        check_token_major(case, 8, 128)
    else:
        check_paged5d(case, 4096, 8, 128)


@pytest.mark.parametrize("kv_dtype,cache_dtype", [("bfloat16", "bfloat16"), ("float16", "float16"),
                                                  ("float32", "float32"), ("float32", "bfloat16")])
def test_large_append_of_slot_runs(kv_dtype, cache_dtype):
    # 4096 tokens x 8 heads x D 128 (16 MiB of cache written, 32 MiB for
    # float32 caches): neighbouring tokens write neighbouring bytes of the
    # same V rows and K chunks, so the stores of different wavefronts meet in
    # the same cache lines.
    case = make_run_append_case(31, N=4096, H=8, D=128, num_blocks=1024, block_size=16,
                                kv_dtype=kv_dtype, cache_dtype=cache_dtype)
    s = case.slot_mapping
    in_run = (s[1:] == s[:-1] + 1) & (s[:-1] >= 0)
    assert in_run.mean() > 0.5 and (~in_run).sum() > 100
    check_paged5d(case, 1024, 8, 128)


@pytest.mark.parametrize("block_size", [8, 16, 32])
@pytest.mark.parametrize("kv_dtype,cache_dtype", [("bfloat16", "bfloat16"), ("float32", "float16")])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_whole_block_runs(block_size, kv_dtype, cache_dtype, head_dim):
    # Whole blocks written by consecutive tokens take the one-wavefront-per-
    # (block, head) path; partial blocks, single slots and padding in the
    # same batch take the per-token path.
    H = 4
    case = make_run_append_case(40 + block_size, N=600, H=H, D=head_dim, num_blocks=160, block_size=block_size,
                                kv_dtype=kv_dtype, cache_dtype=cache_dtype)
    s = case.slot_mapping
    whole = sum(1 for i in range(0, len(s) - block_size + 1)
                if s[i] >= 0 and s[i] % block_size == 0
                and all(s[i + k] == s[i] + k for k in range(block_size)))
    assert whole >= 5
    check_paged5d(case, 160, H, head_dim)


@pytest.mark.parametrize("start", [0, 5, 16])
@pytest.mark.parametrize("N", [1, 15, 16, 17, 300, 1024])
def test_consecutive_slots(start, N):
    # The reference benchmark's slot mapping (slots start .. start+N-1, as a
    # prefill writes): whole blocks in the middle, partial blocks at the ends.
    case = make_append_case(N + start, N=N, H=8, D=128, num_slots=128 * 16, block_size=16, pad_frac=0.0)
    case = dataclasses.replace(case, slot_mapping=np.arange(start, start + N, dtype=np.int32))
    check_paged5d(case, 128, 8, 128)
