"""The ctypes stub in INTEGRATION.md (the binding a maintainer of the
reference would add in place of bindings.cpp) is executed as written, with
only the library path made absolute.  On the CPU its argtypes/restype lists
must equal the package's own table, which tests/test_abi.py checks against
include/pagedkv.h; on the GPU its paged_attention_v1 and reshape_and_cache
must agree with the oracle (bf16 tolerance 1e-2 abs / 2e-2 rel; the append
bit-exact)."""

import os
import re

import numpy as np
import pytest

from sglang_mlx_amd import _lib
from test_abi import header_functions

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DOC = os.path.join(ROOT, "INTEGRATION.md")


def stub_namespace() -> dict:
    text = open(DOC).read()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    (code,) = [b for b in blocks if 'ctypes.CDLL("libpagedkv_gfx950.so")' in b]
    code = code.replace('ctypes.CDLL("libpagedkv_gfx950.so")', f"ctypes.CDLL({_lib.LIB_PATH!r})")
    ns: dict = {}
    exec(compile(code, "INTEGRATION.md", "exec"), ns)
    return ns


def test_stub_signatures_match_the_header():
    ns = stub_namespace()
    lib, decl = ns["lib"], header_functions()
    declared = [n for n in _lib.SIGNATURES if getattr(lib, n).argtypes is not None]
    assert {"pkv_paged_attention", "pkv_reshape_and_cache", "pkv_paged_attention_workspace_size"} <= set(declared)
    for name in declared:
        fn = getattr(lib, name)
        restype, argtypes = _lib.SIGNATURES[name]
        assert list(fn.argtypes) == list(argtypes), name
        assert len(fn.argtypes) == decl[name], name
        assert fn.restype == restype, name


def test_a_dropped_argument_is_caught():
    # The check above would have caught the earlier stub, which left out
    # k_scale and v_scale (28 argtypes for 30 parameters).
    short = list(_lib.SIGNATURES["pkv_paged_attention"][1])
    del short[-3:-1]
    assert len(short) == 28 != header_functions()["pkv_paged_attention"]


@pytest.mark.gpu
def test_stub_runs_against_the_oracle():
    import torch

    from oracle import pagedkv_oracle as orc
    from pkv_cases import decode_oracle, make_append_case, make_decode_case
    from pkv_torch import to_f64, to_index, to_numpy, to_torch

    ns = stub_namespace()
    c = make_decode_case(4242, B=5, Hq=16, Hkv=4, D=128, block_size=16, ctx_lo=1, ctx_hi=900,
                         cache_dtype="bfloat16")
    out = ns["paged_attention_v1"](to_torch(c.q, "bfloat16"), to_torch(c.k_cache, "bfloat16"),
                                   to_torch(c.v_cache, "bfloat16"), to_index(c.block_tables),
                                   to_index(c.context_lens), c.num_kv_heads, c.scale, c.block_size, c.max_seq_len)
    torch.cuda.synchronize()
    np.testing.assert_allclose(to_f64(out), decode_oracle(c), atol=1e-2, rtol=2e-2)

    a = make_append_case(4243, N=96, H=4, D=128, num_slots=64 * 16, block_size=16)
    kc0 = np.zeros((64, 4, 16, 16, 8), dtype=np.uint16)
    vc0 = np.zeros((64, 4, 128, 16), dtype=np.uint16)
    kc, vc = to_torch(kc0, "bfloat16"), to_torch(vc0, "bfloat16")
    ns["reshape_and_cache"](to_torch(a.key, "bfloat16"), to_torch(a.value, "bfloat16"), kc, vc,
                            to_index(a.slot_mapping))
    torch.cuda.synchronize()
    rk, rv = orc.reshape_and_cache_paged5d(a.key, a.value, kc0, vc0, a.slot_mapping, "bfloat16", "bfloat16")
    assert np.array_equal(to_numpy(kc), rk) and np.array_equal(to_numpy(vc), rv)
