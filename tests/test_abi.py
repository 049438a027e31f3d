"""The C-ABI library: it loads, exports every entry point that
include/pagedkv.h declares with the argument count the ctypes table uses,
and rejects bad arguments with the documented status codes and messages
before any HIP call.  No kernel is launched (no call here reaches a launch),
so this runs without a GPU.
"""

import ctypes
import os
import re

import pytest

from sglang_mlx_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pagedkv.h")


def header_functions():
    """name -> parameter count of every function declared in the header."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"(?:const\s+char\s*\*|int|size_t)\s+(pkv_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return out


def test_library_is_built_and_loads():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"
    lib = _lib.lib()
    assert b"gfx950" in lib.pkv_version()


def test_every_declared_symbol_is_exported_with_matching_arity():
    decl = header_functions()
    assert set(decl) == set(_lib.SIGNATURES), (set(decl) ^ set(_lib.SIGNATURES))
    handle = ctypes.CDLL(_lib.LIB_PATH)
    for name, nparams in decl.items():
        getattr(handle, name)  # AttributeError if not exported
        assert len(_lib.SIGNATURES[name][1]) == nparams, name


def attn(noalloc=False, **kw):
    """pkv_paged_attention (or, with noalloc, pkv_paged_attention_noalloc,
    which takes no workspace arguments) with null buffers and valid
    defaults, overridden by kw."""
    a = dict(out=None, q=None, kc=None, vc=None, bt=None, ctx=None, alibi=None, B=2, Hq=8, Hkv=2, D=128, bs=16,
             max_blocks=4, max_seq_len=64, nb=10, scale=1.0, q_stride=1024, kbs=2 * 128 * 16, khs=128 * 16,
             vbs=2 * 128 * 16, vhs=128 * 16, layout=_lib.PKV_LAYOUT_PAGED5D, ps=0, ws=None, ws_bytes=0,
             qd=_lib.PKV_BF16, cd=_lib.PKV_BF16, k_scale=1.0, v_scale=1.0, stream=None)
    a.update(kw)
    lib = _lib.lib()
    if noalloc:
        del a["ws"], a["ws_bytes"]
        st = lib.pkv_paged_attention_noalloc(*a.values())
    else:
        st = lib.pkv_paged_attention(*a.values())
    return st, lib.pkv_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(Hq=6, Hkv=4), 1, "num_heads must be divisible by num_kv_heads"),
    (dict(Hkv=0), 1, "num_heads must be divisible by num_kv_heads"),
    (dict(max_seq_len=0), 1, "max_seq_len must be positive"),
    (dict(max_seq_len=65), 1, "max_seq_len exceeds block table capacity"),
    (dict(D=100), 2, "Unsupported head_size/block_size for paged_attention"),
    (dict(bs=64, max_blocks=1), 2, "Unsupported head_size/block_size for paged_attention"),
    (dict(qd=_lib.PKV_F16, cd=_lib.PKV_BF16), 2, "Unsupported query/cache dtype pair"),
    (dict(qd=_lib.PKV_BF16, cd=_lib.PKV_F32), 2, "Unsupported query/cache dtype pair"),
    (dict(qd=_lib.PKV_F32, cd=_lib.PKV_F32, layout=_lib.PKV_LAYOUT_TOKEN_MAJOR), 2,
     "float32 caches are read in the paged layout"),
    (dict(qd=_lib.PKV_F32, cd=_lib.PKV_F32), 1, "null buffer"),
    (dict(ps=24), 1, "partition_size must be a positive multiple of 16"),
    (dict(ps=8192), 1, "partition_size must be a positive multiple of 16"),
    (dict(bs=32, max_blocks=2, ps=16), 1, "partition_size must be a positive multiple of 16 and of block_size"),
    (dict(nb=0), 1, "num_blocks must be positive"),
    (dict(), 1, "null buffer"),
    (dict(qd=_lib.PKV_FP8_E4M3, cd=_lib.PKV_FP8_E4M3), 2, "Unsupported query/cache dtype pair"),
    (dict(cd=_lib.PKV_FP8_E4M3, D=120), 2, "FP8 caches are read in the paged layout"),
    (dict(cd=_lib.PKV_FP8_E4M3, layout=_lib.PKV_LAYOUT_TOKEN_MAJOR), 2, "FP8 caches are read in the paged layout"),
    (dict(cd=_lib.PKV_FP8_E4M3, k_scale=float("nan")), 1, "finite and nonzero"),
    (dict(cd=_lib.PKV_FP8_E4M3, v_scale=0.0), 1, "finite and nonzero"),
    (dict(cd=_lib.PKV_FP8_E4M3), 1, "null buffer"),
])
def test_paged_attention_rejections(kw, code, msg):
    st, err = attn(**kw)
    assert st == code and msg in err, (st, err)
    # The no-allocation entry point runs the same checks in the same order.
    st, err = attn(noalloc=True, **kw)
    assert st == code and msg in err, (st, err)


def test_noalloc_refuses_oversize_before_any_hip_call():
    # 256 sequences x 32 heads at 64K tokens in 4096-token partitions need
    # 68 MB of partials, more than the 32 MiB static scratch: refused by the
    # argument checks, so this runs without a GPU.
    import numpy as np
    buf = np.zeros(64, dtype=np.uint8)
    p = ctypes.c_void_p((buf.ctypes.data + 15) // 16 * 16)
    kw = dict(out=p, q=p, kc=p, vc=p, bt=p, ctx=p, B=256, Hq=32, Hkv=8, max_blocks=4096, max_seq_len=65536,
              q_stride=32 * 128, kbs=8 * 128 * 16, vbs=8 * 128 * 16, ps=4096)
    assert _lib.lib().pkv_paged_attention_workspace_size(256, 32, 8, 128, 65536, 4096) > \
        _lib.PKV_NOALLOC_SCRATCH_BYTES
    st, err = attn(noalloc=True, **kw)
    assert st == _lib.PKV_ERR_UNSUPPORTED and "static scratch" in err, (st, err)
    assert attn(noalloc=True, B=0)[0] == _lib.PKV_OK


def test_paged_attention_rejects_misaligned_output():
    import numpy as np
    buf = np.zeros(64, dtype=np.uint8)
    base = buf.ctypes.data
    good = (base + 15) // 16 * 16
    ptr = lambda a: ctypes.c_void_p(a)
    kw = dict(out=ptr(good + 8), q=ptr(good), kc=ptr(good), vc=ptr(good), bt=ptr(good), ctx=ptr(good),
              ws=ptr(good), ws_bytes=1 << 40)
    st, err = attn(**kw)
    assert st == _lib.PKV_ERR_INVALID and "out must be 16-byte aligned" in err, (st, err)


@pytest.mark.parametrize("kw,code,msg", [
    # Rows narrower than Hkv heads of D, or heads closer than D apart.
    (dict(kbs=16 * 255), 1, "rows that hold num_kv_heads heads"),
    (dict(vhs=64), 1, "rows that hold num_kv_heads heads"),
    (dict(kbs=16 * 256 + 1), 1, "rows that hold num_kv_heads heads"),
    # Row ids are 32-bit.
    (dict(nb=(1 << 31) // 16 + 1), 2, "at most 2^31 - 1 rows"),
    (dict(bs=1, max_seq_len=4, kbs=256, vbs=256, nb=1 << 31), 2, "at most 2^31 - 1 rows"),
    (dict(layout=2), 1, "Unknown cache layout"),
])
def test_token_row_rejections(kw, code, msg):
    # Token-row layout [nb, 16, Hkv=2, D=128]: block stride 16 rows of 256.
    import numpy as np
    buf = np.zeros(64, dtype=np.uint8)
    good = (buf.ctypes.data + 15) // 16 * 16
    ptr = ctypes.c_void_p(good)
    a = dict(out=ptr, q=ptr, kc=ptr, vc=ptr, bt=ptr, ctx=ptr, ws=ptr, ws_bytes=1 << 40,
             layout=_lib.PKV_LAYOUT_TOKEN_MAJOR, kbs=16 * 256, khs=128, vbs=16 * 256, vhs=128)
    a.update(kw)
    st, err = attn(**a)
    assert st == code and msg in err, (st, err)


def test_paged_attention_empty_batch_is_a_noop():
    assert attn(B=0)[0] == _lib.PKV_OK


def test_workspace_size_closed_form():
    lib = _lib.lib()
    align = lambda x: (x + 255) // 256 * 256
    C = _lib.PKV_COUNTER_BYTES  # the arrival counters at the start
    # v1 partitions: the largest of 4096, 2048, ... 256 tokens that still gives
    # 256 workgroups (seqs x units x partitions).
    # Llama-3-8B decode layer: 64 seqs x 8 KV heads at 4096 tokens -> one
    # 4096-token partition already gives 512 workgroups.
    parts = 1
    assert lib.pkv_paged_attention_workspace_size(64, 32, 8, 128, 4096, 0) == C + \
        align(64 * 32 * parts * 2 * 4) + align(64 * 32 * parts * 128 * 4)
    # One Qwen2-7B sequence at 32K (4 units): 512-token partitions, 64 of them.
    parts = 32768 // 512
    assert lib.pkv_paged_attention_workspace_size(1, 28, 4, 128, 32768, 0) == C + \
        align(28 * parts * 2 * 4) + align(28 * parts * 128 * 4)
    # Four sequences at 128K: 4096-token partitions.
    parts = 131072 // 4096
    assert lib.pkv_paged_attention_workspace_size(4, 28, 4, 128, 131072, 0) == C + \
        align(4 * 28 * parts * 2 * 4) + align(4 * 28 * parts * 128 * 4)
    # A short context never goes below 256-token partitions.
    assert lib.pkv_paged_attention_workspace_size(1, 8, 1, 64, 1000, 0) == C + \
        align(8 * 4 * 2 * 4) + align(8 * 4 * 64 * 4)
    # Explicit split-K partitions: runs of them per workgroup, as many as
    # keep v1's grid (here 4096 tokens, so 8 of 512 and 1 of 4096) ...
    assert lib.pkv_paged_attention_workspace_size(4, 28, 4, 128, 131072, 512) == C + \
        align(4 * 28 * 32 * 2 * 4) + align(4 * 28 * 32 * 128 * 4)
    assert lib.pkv_paged_attention_workspace_size(4, 28, 4, 128, 131072, 4096) == C + \
        align(4 * 28 * 32 * 2 * 4) + align(4 * 28 * 32 * 128 * 4)
    # ... and whole partitions: 10 of 400 tokens (4000) where v1 takes 4096.
    assert lib.pkv_paged_attention_workspace_size(4, 28, 4, 128, 65536, 400) == C + \
        align(4 * 28 * 17 * 2 * 4) + align(4 * 28 * 17 * 128 * 4)
    # One sequence at 32K: v1 takes 512, so 512-token partitions are not grouped.
    assert lib.pkv_paged_attention_workspace_size(1, 28, 4, 128, 32768, 512) == C + \
        align(28 * 64 * 2 * 4) + align(28 * 64 * 128 * 4)
    assert lib.pkv_paged_attention_workspace_size(4, 28, 4, 128, 100, 24) == 0
    assert lib.pkv_paged_attention_workspace_size(4, 28, 3, 128, 100, 0) == 0
    assert lib.pkv_paged_attention_workspace_size(4, 28, 4, 128, 100, 8192) == 0


def rac(**kw):
    a = dict(key=None, value=None, kc=None, vc=None, slots=None, N=4, H=8, D=128, ks=1024, vs=1024,
             layout=_lib.PKV_LAYOUT_PAGED5D, bs=16, x=8, num_slots=1024, kvd=_lib.PKV_BF16, cd=_lib.PKV_BF16,
             k_scale=1.0, v_scale=1.0, stream=None)
    a.update(kw)
    lib = _lib.lib()
    st = lib.pkv_reshape_and_cache(*a.values())
    return st, lib.pkv_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(N=-1), 1, "num_tokens must be non-negative"),
    (dict(H=0), 1, "num_kv_heads and head_size must be positive"),
    (dict(kvd=_lib.PKV_F16, cd=_lib.PKV_BF16), 2, "Unsupported key/cache dtype pair"),
    (dict(kvd=7), 1, "Unsupported dtype"),
    (dict(layout=5), 1, "Unknown cache layout"),
    (dict(num_slots=0), 1, "num_slots must be in"),
    (dict(ks=100), 1, "row stride"),
    (dict(x=4), 1, "16 / sizeof(cache element)"),
    (dict(num_slots=1000), 1, "multiple of block_size"),
    (dict(), 1, "null buffer"),
    (dict(kvd=_lib.PKV_FP8_E4M3, cd=_lib.PKV_FP8_E4M3, x=16), 1, "Unsupported dtype"),
    (dict(cd=_lib.PKV_FP8_E4M3, x=8), 1, "16 / sizeof(cache element)"),
    (dict(cd=_lib.PKV_FP8_E4M3, x=16, D=120), 1, "head_size must be a multiple of x"),
    (dict(cd=_lib.PKV_FP8_E4M3, x=16, k_scale=0.0), 1, "finite and nonzero"),
    (dict(cd=_lib.PKV_FP8_E4M3, x=16, v_scale=float("inf")), 1, "finite and nonzero"),
    (dict(cd=_lib.PKV_FP8_E4M3, x=16), 1, "null buffer"),
    # FP8 token-major rows are encoded 8 elements at a time: H * D = 12 and
    # 4 would leave elements unwritten, so they are rejected.
    (dict(cd=_lib.PKV_FP8_E4M3, kvd=_lib.PKV_F32, layout=_lib.PKV_LAYOUT_TOKEN_MAJOR, H=1, D=12, ks=12, vs=12),
     2, "multiple of 8"),
    (dict(cd=_lib.PKV_FP8_E4M3, layout=_lib.PKV_LAYOUT_TOKEN_MAJOR, H=1, D=4, ks=8, vs=8, N=0), 2, "multiple of 8"),
    (dict(cd=_lib.PKV_FP8_E4M3, layout=_lib.PKV_LAYOUT_TOKEN_MAJOR, H=3, D=8, ks=24, vs=24), 1, "null buffer"),
])
def test_reshape_and_cache_rejections(kw, code, msg):
    st, err = rac(**kw)
    assert st == code and msg in err, (st, err)


def test_reshape_and_cache_empty_is_a_noop():
    assert rac(N=0)[0] == _lib.PKV_OK
    assert rac(N=0, layout=_lib.PKV_LAYOUT_TOKEN_MAJOR)[0] == _lib.PKV_OK


def test_status_translation():
    lib = _lib.lib()
    rac(H=0)
    with pytest.raises(ValueError, match="num_kv_heads and head_size must be positive"):
        _lib.check(_lib.PKV_ERR_INVALID)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.PKV_ERR_HIP)
    _lib.check(_lib.PKV_OK)
    assert lib.pkv_max_shared_memory_per_block(0, None) == _lib.PKV_ERR_INVALID


def test_convert_fp8_rejections():
    import numpy as np
    lib = _lib.lib()
    buf = np.zeros(256, dtype=np.uint8)
    base = (buf.ctypes.data + 15) // 16 * 16
    p = lambda off: ctypes.c_void_p(base + off)
    cases = [
        ((p(0), p(128), -1, 1.0, 0, 3), 1, "num_elements must be non-negative"),
        ((p(0), p(128), 8, 1.0, 4, 3), 2, "Unsupported dtype pair"),
        ((p(0), p(128), 8, 1.0, 0, -1), 2, "Unsupported dtype pair"),
        ((None, p(128), 8, 1.0, 0, 3), 1, "null buffer"),
        ((p(0), p(129), 8, 1.0, 0, 3), 1, "not aligned"),         # float32 source at an odd address
        ((p(0), p(4), 8, 1.0, 0, 0), 1, "overlap"),
        ((p(0), p(0), 8, 1.0, 0, 3), 1, "overlap"),               # in place needs equal element sizes
    ]
    for args, code, msg in cases:
        st = lib.pkv_convert_fp8(*args, None)
        err = lib.pkv_last_error().decode()
        assert st == code and msg in err, (args, st, err)
    assert lib.pkv_convert_fp8(p(0), p(128), 0, 1.0, 0, 3, None) == _lib.PKV_OK   # empty: no launch



def test_counter_region_constant_matches_header():
    import re
    from pathlib import Path
    text = (Path(__file__).resolve().parents[1] / "include" / "pagedkv.h").read_text()
    m = re.search(r"#define PKV_COUNTER_BYTES (\d+)", text)
    assert m and int(m.group(1)) == _lib.PKV_COUNTER_BYTES
