"""Argument checks of the drop-in API (sglang_mlx_amd.kernels / _ext) on CPU
tensors: the reference's checks and messages in the reference's order
(mlx_paged_attention.cpp:156-199), its KAT for the block-table capacity
(tests/test_paged_attention_kernel.py:380-398), TypeError for non-tensors
(bindings.cpp:15-19), and the GPU-only error once every check has passed
(the reference's eval_cpu throws, mlx_paged_attention.cpp:89-91).
"""

import pytest
import torch

from sglang_mlx_amd import kernels


def pa_args(**kw):
    a = dict(query=torch.zeros(2, 8, 64, dtype=torch.float16),
             key_cache=torch.zeros(6, 2, 8, 16, 8, dtype=torch.float16),
             value_cache=torch.zeros(6, 2, 64, 16, dtype=torch.float16),
             block_tables=torch.zeros(2, 4, dtype=torch.int32),
             context_lens=torch.ones(2, dtype=torch.int32),
             num_kv_heads=2, scale=0.125, block_size=16, max_seq_len=64, alibi_slopes=None)
    a.update(kw)
    return a


@pytest.mark.parametrize("kw,msg", [
    (dict(query=torch.zeros(2, 8, 64, 1, dtype=torch.float16)), "query must have shape"),
    (dict(value_cache=torch.zeros(6, 2, 64, dtype=torch.float16)), "must use paged attention layouts"),
    (dict(key_cache=torch.zeros(6, 2, 64, 16, 8, 1, dtype=torch.float16)), "must use paged attention layouts"),
    (dict(block_tables=torch.zeros(8, dtype=torch.int32)), "block_tables must be 2D"),
    (dict(context_lens=torch.ones(3, dtype=torch.int32)), "sequence counts differ"),
    (dict(num_kv_heads=3), "num_heads must be divisible by num_kv_heads"),
    (dict(num_kv_heads=0), "num_heads must be divisible by num_kv_heads"),
    (dict(num_kv_heads=4), "cache KV-head count does not match"),
    (dict(value_cache=torch.zeros(6, 2, 32, 16, dtype=torch.float16)), "cache head size does not match"),
    (dict(block_size=8), "cache block dimensions do not match block_size"),
    (dict(alibi_slopes=torch.zeros(4)), "alibi_slopes must have shape"),
    (dict(max_seq_len=0), "max_seq_len must be positive"),
    (dict(max_seq_len=65), "max_seq_len exceeds block table capacity"),
    (dict(query=torch.zeros(2, 8, 48, dtype=torch.float16), key_cache=torch.zeros(6, 2, 6, 16, 8, dtype=torch.float16),
          value_cache=torch.zeros(6, 2, 48, 16, dtype=torch.float16)), "Unsupported head_size/block_size"),
    (dict(key_cache=torch.zeros(6, 2, 16, 16, 4, dtype=torch.float16)), "16 / element size"),
    (dict(query=torch.zeros(2, 8, 64, dtype=torch.bfloat16)), "Unsupported query/cache dtype pair"),
])
def test_paged_attention_checks(kw, msg):
    with pytest.raises(ValueError, match=msg):
        kernels.paged_attention_v1(**pa_args(**kw))


def rows_args(**kw):
    # Token-row caches: MHATokenPool's [rows, Hkv, D] with a slot table (block size 1).
    a = pa_args(key_cache=torch.zeros(96, 2, 64, dtype=torch.float16),
                value_cache=torch.zeros(96, 2, 64, dtype=torch.float16), block_size=1,
                block_tables=torch.zeros(2, 64, dtype=torch.int32))
    a.update(kw)
    return a


@pytest.mark.parametrize("kw,msg", [
    (dict(num_kv_heads=4), "cache KV-head count does not match"),
    (dict(value_cache=torch.zeros(96, 2, 32, dtype=torch.float16)), "cache head size does not match"),
    (dict(value_cache=torch.zeros(90, 2, 64, dtype=torch.float16)), "cache block dimensions do not match"),
    (dict(block_size=16), "cache block dimensions do not match block_size"),
    (dict(key_cache=torch.zeros(6, 16, 2, 64, dtype=torch.float16),
          value_cache=torch.zeros(6, 16, 2, 64, dtype=torch.float16), block_size=8),
     "cache block dimensions do not match block_size"),
    (dict(key_cache=torch.zeros(6, 4, 2, 64, dtype=torch.float16),
          value_cache=torch.zeros(6, 4, 2, 64, dtype=torch.float16), block_size=4),
     "Unsupported head_size/block_size"),
    (dict(key_cache=torch.zeros(96, 2, 64, dtype=torch.float16)[:, :, :32].repeat(1, 1, 2)[::1]), None),
])
def test_token_row_layout_checks(kw, msg):
    if msg is None:
        with pytest.raises(RuntimeError, match="GPU-only"):
            kernels.paged_attention_v1(**rows_args(**kw))
        return
    with pytest.raises(ValueError, match=msg):
        kernels.paged_attention_v1(**rows_args(**kw))


def test_token_row_layout_rejects_strided_rows():
    k = torch.zeros(96, 2, 128, dtype=torch.float16)[:, :, :64]
    with pytest.raises(ValueError, match="rows must be contiguous"):
        kernels.paged_attention_v1(**rows_args(key_cache=k))
    # Flash layout whose blocks hold padding rows: block stride != block_size * row stride.
    padded = torch.zeros(6, 10, 2, 64, dtype=torch.float16)[:, :8]
    with pytest.raises(ValueError, match="rows must be contiguous"):
        kernels.paged_attention_v1(**rows_args(key_cache=padded, value_cache=padded.clone(), block_size=8))


def test_capacity_kat():
    # The reference KAT: one block of 16, max_seq_len 17.
    q = torch.zeros(1, 2, 32)
    kc = torch.zeros(2, 1, 4, 16, 8, dtype=torch.float16)
    vc = torch.zeros(2, 1, 32, 16, dtype=torch.float16)
    with pytest.raises(ValueError, match="block table capacity"):
        kernels.paged_attention_v1(q, kc, vc, torch.tensor([[0]], dtype=torch.int32),
                                   torch.tensor([1], dtype=torch.int32), 1, 1.0, 16, 17)


def test_non_tensor_arguments():
    with pytest.raises(TypeError, match="Expected torch.Tensor"):
        kernels.paged_attention_v1(**pa_args(query=[[0.0]]))
    with pytest.raises(TypeError):
        kernels.reshape_and_cache([0.0], torch.zeros(1), torch.zeros(1), torch.zeros(1), torch.zeros(1))


def test_valid_cpu_inputs_are_gpu_only():
    with pytest.raises(RuntimeError, match="GPU-only"):
        kernels.paged_attention_v1(**pa_args())
    with pytest.raises(RuntimeError, match="GPU-only"):
        kernels.paged_attention_v2(**pa_args(), partition_size=32)


def test_v2_partition_checks():
    with pytest.raises(ValueError, match="partition_size"):
        kernels.paged_attention_v2(**pa_args(), partition_size=24)
    with pytest.raises(ValueError, match="partition_size"):
        kernels.paged_attention_v2(**pa_args(), partition_size=8)


def rac_args(**kw):
    a = dict(key=torch.zeros(3, 2, 64, dtype=torch.bfloat16), value=torch.zeros(3, 2, 64, dtype=torch.bfloat16),
             key_cache=torch.zeros(4, 2, 8, 16, 8, dtype=torch.bfloat16),
             value_cache=torch.zeros(4, 2, 64, 16, dtype=torch.bfloat16),
             slot_mapping=torch.tensor([0, -1, 5], dtype=torch.int64))
    a.update(kw)
    return a


@pytest.mark.parametrize("kw,msg", [
    (dict(key=torch.zeros(3, 128, dtype=torch.bfloat16)), "key and value must have shape"),
    (dict(slot_mapping=torch.zeros(2, dtype=torch.int32)), "slot_mapping must have shape"),
    (dict(value_cache=torch.zeros(4, 2, 64, 16, dtype=torch.float16)), "dtypes differ"),
    (dict(key=torch.zeros(3, 2, 64, dtype=torch.float16), value=torch.zeros(3, 2, 64, dtype=torch.float16)),
     "Unsupported key/cache dtype pair"),
    (dict(key_cache=torch.zeros(4, 2, 8, 8, 8, dtype=torch.bfloat16)), "value_cache must have shape"),
    (dict(key_cache=torch.zeros(4, 2, 16, 16, 4, dtype=torch.bfloat16)), "key_cache must have shape"),
    (dict(key_cache=torch.zeros(64, 4, 64, dtype=torch.bfloat16),
          value_cache=torch.zeros(64, 4, 64, dtype=torch.bfloat16)), "token-major caches must have shape"),
    (dict(key_cache=torch.zeros(4, 2, 64, 16, dtype=torch.bfloat16)), "paged or token-major layout"),
    (dict(slot_mapping=torch.zeros(3, dtype=torch.float32)), "integer dtype"),
])
def test_reshape_and_cache_checks(kw, msg):
    with pytest.raises(ValueError, match=msg):
        kernels.reshape_and_cache(**rac_args(**kw))


def test_reshape_and_cache_gpu_only():
    with pytest.raises(RuntimeError, match="GPU-only"):
        kernels.reshape_and_cache(**rac_args())
    with pytest.raises(RuntimeError, match="GPU-only"):
        kernels.reshape_and_cache(**rac_args(key_cache=torch.zeros(64, 2, 64, dtype=torch.bfloat16),
                                             value_cache=torch.zeros(64, 2, 64, dtype=torch.bfloat16)))


def test_paged_cache_regions_must_be_contiguous():
    # A cache whose (block, head) regions are not one contiguous run would
    # need a whole-cache copy per call; it is rejected instead.
    kc = torch.zeros(6, 2, 16, 8, 8, dtype=torch.float16).transpose(2, 3)   # [6, 2, 8, 16, 8] view
    with pytest.raises(ValueError, match="key_cache must be contiguous within each"):
        kernels.paged_attention_v1(**pa_args(key_cache=kc))
    vc = torch.zeros(6, 2, 16, 64, dtype=torch.float16).transpose(2, 3)     # [6, 2, 64, 16] view
    with pytest.raises(ValueError, match="value_cache must be contiguous within each"):
        kernels.paged_attention_v1(**pa_args(value_cache=vc))
    # Block and head strides are free: a slice over blocks passes the checks.
    big_k = torch.zeros(12, 2, 8, 16, 8, dtype=torch.float16)
    big_v = torch.zeros(12, 2, 64, 16, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU-only"):
        kernels.paged_attention_v1(**pa_args(key_cache=big_k[::2], value_cache=big_v[::2]))


def test_fp8_token_major_append_needs_rows_of_eight():
    # Rows of num_kv_heads * head_size = 12 elements cannot be encoded in
    # groups of 8; 16 can (and then only the GPU is missing).
    key = torch.zeros(3, 1, 12)
    cache = torch.zeros(8, 1, 12, dtype=torch.uint8)
    with pytest.raises(ValueError, match="multiple of 8"):
        kernels.reshape_and_cache(key, key.clone(), cache, cache.clone(), torch.zeros(3, dtype=torch.int32),
                                  k_scale=1.0, v_scale=1.0)
    key = torch.zeros(3, 2, 8)
    cache = torch.zeros(8, 2, 8, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="GPU-only"):
        kernels.reshape_and_cache(key, key.clone(), cache, cache.clone(), torch.zeros(3, dtype=torch.int32))


def test_float32_caches():
    # (float32 query, float32 cache) is the reference's (float, float) pair:
    # accepted in the paged layout (x = 4), rejected for token rows.
    q = torch.zeros(2, 8, 64)
    kc = torch.zeros(6, 2, 16, 16, 4)
    vc = torch.zeros(6, 2, 64, 16)
    with pytest.raises(RuntimeError, match="GPU-only"):
        kernels.paged_attention_v1(**pa_args(query=q, key_cache=kc, value_cache=vc))
    with pytest.raises(ValueError, match="Unsupported query/cache dtype pair"):
        kernels.paged_attention_v1(**pa_args(query=q.half(), key_cache=kc, value_cache=vc))
    with pytest.raises(ValueError, match="float32 caches are read in the paged layout"):
        kernels.paged_attention_v1(**rows_args(query=q, key_cache=torch.zeros(96, 2, 64),
                                               value_cache=torch.zeros(96, 2, 64)))
