"""GPU kernels against the committed golden fixtures (tests/golden/*.npz):
append bit-exact over the whole cache, attention within the float16
(2e-3 abs / 1e-2 rel) or bfloat16 (1e-2 abs / 2e-2 rel) tolerance."""

import glob
import os

import numpy as np
import pytest
import torch

from pkv_cases import tolerance
from pkv_torch import to_f64, to_index, to_numpy, to_torch
from sglang_mlx_amd import kernels

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "decode_*.npz"))), ids=os.path.basename)
def test_decode_matches_fixture(path):
    f = load(path)
    qd, cd = str(f["q_dtype"]), str(f["cache_dtype"])
    alibi = torch.from_numpy(f["alibi"]).cuda() if "alibi" in f else None
    args = (to_torch(f["q"], qd), to_torch(f["k_cache"], cd), to_torch(f["v_cache"], cd), to_index(f["block_tables"]),
            to_index(f["context_lens"]), int(f["num_kv_heads"]), float(f["scale"]), int(f["block_size"]),
            int(f["max_seq_len"]), alibi)
    atol, rtol = tolerance(qd, cd)
    out = kernels.paged_attention_v1(*args)
    torch.cuda.synchronize()
    np.testing.assert_allclose(to_f64(out), f["expected"], atol=atol, rtol=rtol)
    for key in f:
        if key.startswith("expected_split_"):
            ps = int(key.rsplit("_", 1)[1])
            out = kernels.paged_attention_v2(*args, partition_size=ps)
            torch.cuda.synchronize()
            np.testing.assert_allclose(to_f64(out), f[key], atol=atol, rtol=rtol)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "append_*.npz"))), ids=os.path.basename)
def test_append_matches_fixture(path):
    f = load(path)
    kd, cd = str(f["kv_dtype"]), str(f["cache_dtype"])
    kc, vc = to_torch(f["key_cache"], cd), to_torch(f["value_cache"], cd)
    kernels.reshape_and_cache(to_torch(f["key"], kd), to_torch(f["value"], kd), kc, vc, to_index(f["slot_mapping"]))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_numpy(kc), f["expected_key_cache"])
    np.testing.assert_array_equal(to_numpy(vc), f["expected_value_cache"])
