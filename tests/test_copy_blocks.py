"""Block copies on the CPU side: the oracle against the reference's
known-answer tests (tests/test_paged_attention_kernel.py:400-438) and against
plain NumPy indexing, the C-ABI's argument checks for pkv_copy_blocks (no
kernel is launched), and the Python wrappers' checks with the reference's
messages (mlx_cache.cpp:308-330, :352-360)."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from sglang_mlx_amd import _ext, _lib


def test_oracle_copy_blocks_reference_kat():
    # test_paged_attention_kernel.py:400-423: two layers of [4, 2, 3], pairs (0->2), (1->3).
    keys = [np.arange(24, dtype=np.float32).reshape(4, 2, 3) + layer * 100 for layer in range(2)]
    vals = [k + 1000 for k in keys]
    nk, nv = orc.copy_blocks(keys, vals, np.array([[0, 2], [1, 3]]))
    for layer in range(2):
        ek, ev = keys[layer].copy(), vals[layer].copy()
        ek[2], ek[3] = keys[layer][0], keys[layer][1]
        ev[2], ev[3] = vals[layer][0], vals[layer][1]
        np.testing.assert_array_equal(nk[layer], ek)
        np.testing.assert_array_equal(nv[layer], ev)
        np.testing.assert_array_equal(keys[layer], np.arange(24, dtype=np.float32).reshape(4, 2, 3) + layer * 100)


def test_oracle_swap_blocks_reference_kat():
    # test_paged_attention_kernel.py:425-438.
    src = np.arange(24, dtype=np.float32).reshape(4, 2, 3)
    dst = np.full((4, 2, 3), -1, dtype=np.float32)
    out = orc.swap_blocks(src, dst, np.array([[0, 2], [3, 1]]))
    expected = dst.copy()
    expected[2] = src[0]
    expected[1] = src[3]
    np.testing.assert_array_equal(out, expected)


def test_oracle_matches_fancy_indexing_and_skips_out_of_range():
    rng = np.random.default_rng(0)
    cache = rng.integers(0, 2 ** 16, size=(64, 4, 16, 16, 8), dtype=np.uint16)
    perm = rng.permutation(64)
    m = np.stack([perm[:20], perm[20:40]], axis=1)  # sources and destinations disjoint
    expected = cache.copy()
    expected[m[:, 1]] = cache[m[:, 0]]
    out = orc.swap_blocks(cache, cache, np.concatenate([m, [[70, 1], [2, -1]]]))
    np.testing.assert_array_equal(out, expected)


def call(**kw):
    a = dict(src=None, dst=None, planes=1, sb=8, db=8, bb=4096, mapping=None, pairs=1, stream=None)
    a.update(kw)
    lib = _lib.lib()
    st = lib.pkv_copy_blocks(a["src"], a["dst"], a["planes"], a["sb"], a["db"], a["bb"], a["mapping"], a["pairs"],
                             a["stream"])
    return st, lib.pkv_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(planes=-1), 1, "must be non-negative"),
    (dict(pairs=-2), 1, "must be non-negative"),
    (dict(bb=-16), 1, "must be non-negative"),
    (dict(sb=0), 1, "leading block dimension"),
    (dict(db=-3), 1, "leading block dimension"),
    (dict(), 1, "null buffer"),
])
def test_abi_rejections(kw, code, msg):
    st, err = call(**kw)
    assert st == code and msg in err, (st, err)


def test_abi_null_plane_pointer_is_rejected():
    arr = (ctypes.c_void_p * 2)(None, None)
    st, err = call(src=arr, dst=arr, planes=2, mapping=ctypes.c_void_p(16))
    assert st == _lib.PKV_ERR_INVALID and "null buffer" in err


@pytest.mark.parametrize("kw", [dict(planes=0), dict(pairs=0), dict(bb=0)])
def test_abi_empty_is_a_noop(kw):
    assert call(**kw)[0] == _lib.PKV_OK


def test_wrapper_checks_follow_the_reference_messages():
    k = torch.zeros((4, 2, 3))
    m = torch.tensor([[0, 1]])
    with pytest.raises(ValueError, match="key_caches and value_caches size mismatch"):
        _ext.copy_blocks([k, k], [k], m)
    with pytest.raises(ValueError, match=r"block_mapping must have shape \[num_pairs, 2\]"):
        _ext.copy_blocks([k], [k], torch.tensor([0, 1]))
    with pytest.raises(ValueError, match="key/value caches must have matching block counts"):
        _ext.copy_blocks([k], [torch.zeros((5, 2, 3))], m)
    with pytest.raises(ValueError, match="key/value cache block layouts must match"):
        _ext.copy_blocks([k], [torch.zeros((4, 2, 3), dtype=torch.float16)], m)
    with pytest.raises(ValueError, match="src and dst must have a leading block dimension"):
        _ext.swap_blocks(torch.zeros((0, 3)), k, m)
    with pytest.raises(ValueError, match="src and dst block layouts must match"):
        _ext.swap_blocks(k, torch.zeros((4, 7)), m)
    with pytest.raises(ValueError, match=r"block_mapping must have shape \[num_pairs, 2\]"):
        _ext.swap_blocks(k, k, torch.zeros((2, 3), dtype=torch.int64))
    with pytest.raises(TypeError):
        _ext.swap_blocks(k, np.zeros((4, 2, 3)), m)
    with pytest.raises(RuntimeError, match="GPU-only"):
        _ext.swap_blocks(k, k.clone(), m)
    with pytest.raises(RuntimeError, match="GPU-only"):
        _ext.copy_blocks([k], [k.clone()], m)
