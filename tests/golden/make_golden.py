"""Writes the golden fixtures of tests/golden/*.npz.

The reference ships no golden vectors (its tests draw unseeded random
inputs), so these fixtures are seeded inputs with the expected outputs of
the float64 oracle (oracle/pagedkv_oracle.py), itself pinned by
tests/test_oracle.py.  They freeze the oracle: tests/test_golden.py checks
that the oracle still reproduces them, and the GPU tests check the kernels
against them without recomputing anything.

16-bit floats are stored as uint16 bit patterns.  Run from the repository
root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from oracle import pagedkv_oracle as orc  # noqa: E402
from pkv_cases import make_append_case, make_decode_case  # noqa: E402


def decode_fixture(name, seed, partition_sizes=(), **kw):
    c = make_decode_case(seed, **kw)
    out = dict(q=c.q, k_cache=c.k_cache, v_cache=c.v_cache, block_tables=c.block_tables,
               context_lens=c.context_lens, num_kv_heads=c.num_kv_heads, scale=c.scale, block_size=c.block_size,
               max_seq_len=c.max_seq_len, q_dtype=c.q_dtype, cache_dtype=c.cache_dtype,
               expected=orc.paged_attention(c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens,
                                            c.num_kv_heads, c.scale, c.block_size, c.max_seq_len, c.alibi,
                                            c.q_dtype, c.cache_dtype))
    if c.alibi is not None:
        out["alibi"] = c.alibi
    for ps in partition_sizes:
        out[f"expected_split_{ps}"] = orc.paged_attention_split(
            c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens, c.num_kv_heads, c.scale, c.block_size,
            c.max_seq_len, ps, c.alibi, c.q_dtype, c.cache_dtype)
    np.savez_compressed(os.path.join(HERE, name), **out)


def append_fixture(name, seed, layout, nb, zero_cache=False, **kw):
    """Append case; the caches start from random bits (so untouched slots
    are checked too) or, like the reference's fixture, from zeros."""
    a = make_append_case(seed, **kw)
    H, D, bs = kw["H"], kw["D"], kw["block_size"]
    rng = np.random.default_rng(seed + 1)
    fill = (lambda shape: np.zeros(shape, np.float32)) if zero_cache else \
        (lambda shape: rng.standard_normal(shape, dtype=np.float32))
    if layout == "paged5d":
        x = 16 // (4 if a.cache_dtype == "float32" else 2)
        kc0 = orc.to_storage(fill((nb, H, D // x, bs, x)), a.cache_dtype)
        vc0 = orc.to_storage(fill((nb, H, D, bs)), a.cache_dtype)
        ek, ev = orc.reshape_and_cache_paged5d(a.key, a.value, kc0, vc0, a.slot_mapping, a.kv_dtype, a.cache_dtype)
    else:
        kc0 = orc.to_storage(fill((nb * bs, H, D)), a.cache_dtype)
        vc0 = orc.to_storage(fill((nb * bs, H, D)), a.cache_dtype)
        ek, ev = orc.reshape_and_cache_token_major(a.key, a.value, kc0, vc0, a.slot_mapping, a.kv_dtype,
                                                   a.cache_dtype)
    np.savez_compressed(os.path.join(HERE, name), key=a.key, value=a.value, slot_mapping=a.slot_mapping,
                        key_cache=kc0, value_cache=vc0, expected_key_cache=ek, expected_value_cache=ev,
                        kv_dtype=a.kv_dtype, cache_dtype=a.cache_dtype, layout=layout)


def main():
    decode_fixture("decode_fp16_gqa4.npz", 2001, B=3, Hq=8, Hkv=2, D=64, block_size=16, ctx_lo=1, ctx_hi=1,
                   context_lens=[1, 37, 200], cache_dtype="float16", num_blocks=20)
    decode_fixture("decode_bf16_gqa7_alibi_split.npz", 2002, partition_sizes=(64, 128), B=2, Hq=7, Hkv=1, D=128,
                   block_size=8, ctx_lo=1, ctx_hi=1, context_lens=[129, 300], cache_dtype="bfloat16", alibi=True)
    decode_fixture("decode_f32q_f16cache_edges.npz", 2003, B=4, Hq=4, Hkv=1, D=32, block_size=32, ctx_lo=1,
                   ctx_hi=1, context_lens=[0, 32, 33, 100], max_seq_len=64, cache_dtype="float16",
                   q_dtype="float32", max_blocks=4)
    append_fixture("append_paged5d_f32_to_f16.npz", 2004, "paged5d", 20, zero_cache=True, N=75, H=4, D=64,
                   num_slots=320, block_size=16, kv_dtype="float32", cache_dtype="float16")
    append_fixture("append_paged5d_bf16_bs8.npz", 2005, "paged5d", 16, N=100, H=1, D=128, num_slots=128,
                   block_size=8, kv_dtype="bfloat16")
    append_fixture("append_token_major_bf16.npz", 2006, "token_major", 8, N=64, H=2, D=64, num_slots=128,
                   block_size=16, kv_dtype="bfloat16")


if __name__ == "__main__":
    main()
