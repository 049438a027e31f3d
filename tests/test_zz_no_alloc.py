"""pkv_paged_attention_noalloc (the entry point that allocates nothing: its
split-K partials live in a static per-GPU device array) against
pkv_paged_attention with a caller workspace, both through the C-ABI.  The
two run the same kernels on the same inputs, so their outputs must be equal
bit for bit; each case makes two calls in a row, the second with smaller
sizes (the array keeps the first call's contents).  A request whose
workspace would exceed the array is refused before any HIP call."""

import ctypes

import numpy as np
import pytest
import torch

from pkv_cases import decode_oracle, make_decode_case, tolerance
from pkv_torch import to_f64, to_index, to_torch
from sglang_mlx_amd import _lib

pytestmark = pytest.mark.gpu

CODES = {"bfloat16": _lib.PKV_BF16, "float16": _lib.PKV_F16, "float32": _lib.PKV_F32}


def tensors(c):
    return (to_torch(c.q, c.q_dtype), to_torch(c.k_cache, c.cache_dtype), to_torch(c.v_cache, c.cache_dtype),
            to_index(c.block_tables), to_index(c.context_lens))


def call(c, t, partition_size, noalloc):
    q, kc, vc, bt, lens = t
    B, Hq, D = q.shape
    out = torch.full_like(q, float("nan"))
    lib = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    head = (out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), lens.data_ptr(), None,
            B, Hq, c.num_kv_heads, D, c.block_size, bt.shape[1], c.max_seq_len, kc.shape[0], c.scale, q.stride(0),
            kc.stride(0), kc.stride(1), vc.stride(0), vc.stride(1), _lib.PKV_LAYOUT_PAGED5D, partition_size)
    tail = (CODES[c.q_dtype], CODES[c.cache_dtype], 1.0, 1.0, stream)
    if noalloc:
        st = lib.pkv_paged_attention_noalloc(*head, *tail)
    else:
        n = lib.pkv_paged_attention_workspace_size(B, Hq, c.num_kv_heads, D, c.max_seq_len, partition_size)
        ws = torch.zeros(n, dtype=torch.uint8, device="cuda")  # counters zero before the first call
        st = lib.pkv_paged_attention(*head, ws.data_ptr(), n, *tail)
    _lib.check(st)
    return out


# (first call, second call with smaller sizes, partition size of each)
CASES = [
    # Qwen2-7B heads, long contexts, 512-token partitions: 2.3 MB of partials,
    # then 2 short sequences with 256-token partitions.
    (dict(seed=8101, B=4, Hq=28, Hkv=4, D=128, block_size=16, ctx_lo=8000, ctx_hi=20000), 512,
     dict(seed=8102, B=2, Hq=28, Hkv=4, D=128, block_size=16, ctx_lo=100, ctx_hi=3000), 256),
    # paged_attention_v1 semantics (the library's own partitioning) at
    # Llama-3-8B heads on 16 sequences, then 3.
    (dict(seed=8103, B=16, Hq=32, Hkv=8, D=128, block_size=16, ctx_lo=500, ctx_hi=4000), 0,
     dict(seed=8104, B=3, Hq=32, Hkv=8, D=128, block_size=16, ctx_lo=1, ctx_hi=900), 0),
    # float16, head size 64, 8-token blocks.
    (dict(seed=8105, B=6, Hq=16, Hkv=2, D=64, block_size=8, ctx_lo=2000, ctx_hi=6000, cache_dtype="float16"), 1024,
     dict(seed=8106, B=1, Hq=16, Hkv=2, D=64, block_size=8, ctx_lo=40, ctx_hi=40, cache_dtype="float16"), 16),
]


@pytest.mark.parametrize("first,ps1,second,ps2", CASES)
def test_noalloc_matches_workspace_entry_point(first, ps1, second, ps2):
    for kw, ps in ((first, ps1), (second, ps2)):
        c = make_decode_case(cache_dtype=kw.pop("cache_dtype", "bfloat16"), **kw)
        t = tensors(c)
        ref = call(c, t, ps, noalloc=False)
        got = call(c, t, ps, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        a, r = tolerance(c.q_dtype, c.cache_dtype)
        np.testing.assert_allclose(to_f64(got), decode_oracle(c, ps), atol=a, rtol=r)


def test_noalloc_refuses_more_than_its_scratch():
    # 256 sequences x 32 heads at 64K tokens in 4096-token partitions would
    # need 256 * 32 * 16 * (128 + 2) * 4 bytes (68 MB) of partials.
    lib = _lib.lib()
    B, Hq, Hkv, D, bs, msl = 256, 32, 8, 128, 16, 65536
    need = lib.pkv_paged_attention_workspace_size(B, Hq, Hkv, D, msl, 4096)
    assert need > _lib.PKV_NOALLOC_SCRATCH_BYTES
    q = torch.zeros((B, Hq, D), dtype=torch.bfloat16, device="cuda")
    out = torch.full_like(q, 7.0)
    kc = torch.zeros((2, Hkv, D // 8, bs, 8), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros((2, Hkv, D, bs), dtype=torch.bfloat16, device="cuda")
    bt = torch.zeros((B, msl // bs), dtype=torch.int32, device="cuda")
    lens = torch.full((B,), 100, dtype=torch.int32, device="cuda")
    st = lib.pkv_paged_attention_noalloc(
        out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), lens.data_ptr(), None,
        B, Hq, Hkv, D, bs, bt.shape[1], msl, 2, 1.0, q.stride(0), kc.stride(0), kc.stride(1), vc.stride(0),
        vc.stride(1), _lib.PKV_LAYOUT_PAGED5D, 4096, _lib.PKV_BF16, _lib.PKV_BF16, 1.0, 1.0,
        torch.cuda.current_stream().cuda_stream)
    assert st == _lib.PKV_ERR_UNSUPPORTED
    assert "static scratch" in lib.pkv_last_error().decode()
    torch.cuda.synchronize()
    assert (out == 7.0).all()   # nothing launched


CHILD = r'''
import math
import torch
from pkv_cases import make_decode_case
from pkv_torch import to_index, to_torch
from sglang_mlx_amd import _lib

lib = _lib.lib()
# B6 Qwen2-7B heads at 2K-9K tokens: nine partitions per row, merge kernel;
# B40 at <= 2K over two KV heads: four partitions, merged by the partition
# kernel with its self-resetting counters in the static array.
cases = [make_decode_case(8301, B=6, Hq=28, Hkv=4, D=128, block_size=16, ctx_lo=2000, ctx_hi=9000),
         make_decode_case(8302, B=40, Hq=8, Hkv=2, D=128, block_size=16, ctx_lo=1500, ctx_hi=2000)]
ts = [(to_torch(c.q, c.q_dtype), to_torch(c.k_cache, c.cache_dtype), to_torch(c.v_cache, c.cache_dtype),
       to_index(c.block_tables), to_index(c.context_lens)) for c in cases]


def call(c, t, out, stream):
    q, kc, vc, bt, lens = t
    B, Hq, D = q.shape
    return lib.pkv_paged_attention_noalloc(
        out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), lens.data_ptr(), None,
        B, Hq, c.num_kv_heads, D, c.block_size, bt.shape[1], c.max_seq_len, kc.shape[0], c.scale, q.stride(0),
        kc.stride(0), kc.stride(1), vc.stride(0), vc.stride(1), _lib.PKV_LAYOUT_PAGED5D, 0,
        _lib.PKV_BF16, _lib.PKV_BF16, 1.0, 1.0, stream)


torch.cuda.synchronize()
outs = [torch.full_like(t[0], float("nan")) for t in ts]
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):  # this process's first calls on the device are captured
    for c, t, o in zip(cases, ts, outs):
        assert call(c, t, o, torch.cuda.current_stream().cuda_stream) == 0, lib.pkv_last_error()
torch.cuda.synchronize()
for replay in range(4):
    for o in outs:
        o.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    for c, t, o in zip(cases, ts, outs):
        eager = torch.full_like(t[0], float("nan"))
        assert call(c, t, eager, torch.cuda.current_stream().cuda_stream) == 0, lib.pkv_last_error()
        torch.cuda.synchronize()
        assert torch.equal(o, eager), ("replay", replay)
        assert not torch.isnan(o.float()).any()
print("graph replays equal the eager calls")
'''


def test_noalloc_under_graph_capture_in_a_fresh_process():
    # The entry point that allocates nothing, captured in a HIP graph by a
    # process whose first call on the GPU is the captured one (the static
    # array's address is looked up inside the capture), replayed four times
    # with eager calls in between, each replay bit-equal to the eager call.
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([os.path.join(root, "sglang-mlx_amd"),
                                                       os.path.join(root, "tests"), root]))
    r = subprocess.run([sys.executable, "-c", CHILD], env=env, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "graph replays equal the eager calls" in r.stdout
