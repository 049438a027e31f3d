"""The golden fixtures (tests/golden/*.npz, written by make_golden.py): the
oracle still reproduces every stored expectation, and the seeded generators
still reproduce every stored input.  CPU only."""

import glob
import os

import numpy as np
import pytest

from oracle import pagedkv_oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DECODE = sorted(glob.glob(os.path.join(GOLDEN, "decode_*.npz")))
APPEND = sorted(glob.glob(os.path.join(GOLDEN, "append_*.npz")))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fixtures_present():
    assert len(DECODE) == 3 and len(APPEND) == 3


@pytest.mark.parametrize("path", DECODE, ids=os.path.basename)
def test_oracle_reproduces_decode_fixture(path):
    f = load(path)
    alibi = f.get("alibi")
    args = (f["q"], f["k_cache"], f["v_cache"], f["block_tables"], f["context_lens"], int(f["num_kv_heads"]),
            float(f["scale"]), int(f["block_size"]), int(f["max_seq_len"]))
    got = orc.paged_attention(*args, alibi, str(f["q_dtype"]), str(f["cache_dtype"]))
    np.testing.assert_allclose(got, f["expected"], rtol=1e-13, atol=1e-15)
    for key in f:
        if key.startswith("expected_split_"):
            ps = int(key.rsplit("_", 1)[1])
            got = orc.paged_attention_split(*args, ps, alibi, str(f["q_dtype"]), str(f["cache_dtype"]))
            np.testing.assert_allclose(got, f[key], rtol=1e-13, atol=1e-15)
            np.testing.assert_allclose(f[key], f["expected"], rtol=1e-11, atol=1e-13)


@pytest.mark.parametrize("path", APPEND, ids=os.path.basename)
def test_oracle_reproduces_append_fixture(path):
    f = load(path)
    fn = orc.reshape_and_cache_paged5d if str(f["layout"]) == "paged5d" else orc.reshape_and_cache_token_major
    k, v = fn(f["key"], f["value"], f["key_cache"], f["value_cache"], f["slot_mapping"], str(f["kv_dtype"]),
              str(f["cache_dtype"]))
    np.testing.assert_array_equal(k, f["expected_key_cache"])
    np.testing.assert_array_equal(v, f["expected_value_cache"])
    assert (f["slot_mapping"] < 0).any()


def test_generators_reproduce_stored_inputs():
    from pkv_cases import make_append_case, make_decode_case
    f = load(os.path.join(GOLDEN, "decode_fp16_gqa4.npz"))
    c = make_decode_case(2001, B=3, Hq=8, Hkv=2, D=64, block_size=16, ctx_lo=1, ctx_hi=1,
                         context_lens=[1, 37, 200], cache_dtype="float16", num_blocks=20)
    np.testing.assert_array_equal(c.q, f["q"])
    np.testing.assert_array_equal(c.k_cache, f["k_cache"])
    np.testing.assert_array_equal(c.block_tables, f["block_tables"])
    f = load(os.path.join(GOLDEN, "append_token_major_bf16.npz"))
    a = make_append_case(2006, N=64, H=2, D=64, num_slots=128, block_size=16, kv_dtype="bfloat16")
    np.testing.assert_array_equal(a.key, f["key"])
    np.testing.assert_array_equal(a.slot_mapping, f["slot_mapping"])
