"""ctypes loader for libpagedkv_gfx950.so (C ABI declared in include/pagedkv.h).

The shared library is the only compute path of this package.  If it has not
been built, ``lib()`` raises ImportError -- there is no fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libpagedkv_gfx950.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

# Status codes and enums (include/pagedkv.h).
PKV_OK = 0
PKV_ERR_INVALID = 1
PKV_ERR_UNSUPPORTED = 2
PKV_ERR_HIP = 3

PKV_F32, PKV_F16, PKV_BF16, PKV_FP8_E4M3 = 0, 1, 2, 3
PKV_LAYOUT_PAGED5D, PKV_LAYOUT_TOKEN_MAJOR = 0, 1
PKV_NOALLOC_SCRATCH_BYTES = 32 << 20  # static scratch of pkv_paged_attention_noalloc, per GPU
PKV_COUNTER_BYTES = 65536  # arrival counters at the start of every decode workspace (zero between calls)

_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_size = ctypes.c_size_t
_f32 = ctypes.c_float



class CascadePlanC(ctypes.Structure):
    """pkv_cascade_plan (include/pagedkv.h): device pointers and sizes of a
    shared-prefix plan."""

    _fields_ = [
        ("prefix_lens", _c_void_p),
        ("members", _c_void_p),
        ("tiles", _c_void_p),
        ("parts", _c_void_p),
        ("num_members", _i32),
        ("num_tiles", _i32),
        ("num_parts", _i32),
        ("chunk_tokens", _i32),
        ("max_chunks", _i32),
        ("part_tokens", _i32),
        ("max_parts", _i32),
    ]


# name -> (restype, argtypes); the tests check this table against the header.
SIGNATURES = {
    "pkv_version": (ctypes.c_char_p, []),
    "pkv_last_error": (ctypes.c_char_p, []),
    "pkv_reshape_and_cache": (ctypes.c_int, [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # key, value, kc, vc, slots
        _i64, _i32, _i32,                                          # num_tokens, Hkv, D
        _i64, _i64,                                                # key/value stride
        _i32, _i32, _i32,                                          # layout, block_size, x
        _i64, _i32, _i32,                                          # num_slots, kv/cache dtype
        _f32, _f32,                                                # k_scale, v_scale (FP8 caches)
        _c_void_p,                                                 # stream
    ]),
    "pkv_paged_attention_workspace_size": (_size, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "pkv_paged_attention": (ctypes.c_int, [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p,              # out, q, kc, vc
        _c_void_p, _c_void_p, _c_void_p,                          # block_tables, ctx, alibi
        _i32, _i32, _i32, _i32, _i32,                             # B, Hq, Hkv, D, bs
        _i32, _i32, _i64,                                         # max_blocks, max_seq_len, nb
        _f32, _i64,                                               # scale, q_stride
        _i64, _i64, _i64, _i64,                                   # k/v block & head strides
        _i32, _i32,                                               # layout, partition_size
        _c_void_p, _size,                                         # workspace, bytes
        _i32, _i32,                                               # q dtype, cache dtype
        _f32, _f32, _c_void_p,                                    # k_scale, v_scale (FP8), stream
    ]),
    "pkv_paged_attention_cascade_workspace_size": (_size, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "pkv_paged_attention_cascade": (ctypes.c_int, [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p,              # out, q, kc, vc
        _c_void_p, _c_void_p, _c_void_p,                          # block_tables, ctx, alibi
        ctypes.POINTER(CascadePlanC),                             # plan
        _i32, _i32, _i32, _i32, _i32,                             # B, Hq, Hkv, D, bs
        _i32, _i32, _i64,                                         # max_blocks, max_seq_len, nb
        _f32, _i64,                                               # scale, q_stride
        _i64, _i64, _i64, _i64,                                   # k/v block & head strides
        _c_void_p, _size,                                         # workspace, bytes
        _i32, _i32,                                               # q dtype, cache dtype
        _f32, _f32, _c_void_p,                                    # k_scale, v_scale (FP8), stream
    ]),
    "pkv_paged_attention_noalloc": (ctypes.c_int, [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p,              # out, q, kc, vc
        _c_void_p, _c_void_p, _c_void_p,                          # block_tables, ctx, alibi
        _i32, _i32, _i32, _i32, _i32,                             # B, Hq, Hkv, D, bs
        _i32, _i32, _i64,                                         # max_blocks, max_seq_len, nb
        _f32, _i64,                                               # scale, q_stride
        _i64, _i64, _i64, _i64,                                   # k/v block & head strides
        _i32, _i32,                                               # layout, partition_size
        _i32, _i32,                                               # q dtype, cache dtype
        _f32, _f32, _c_void_p,                                    # k_scale, v_scale (FP8), stream
    ]),
    "pkv_copy_blocks": (ctypes.c_int, [
        ctypes.POINTER(_c_void_p), ctypes.POINTER(_c_void_p), _i32,  # src/dst planes, count
        _i64, _i64, _i64,                                            # src/dst blocks, block bytes
        _c_void_p, _i64, _c_void_p]),                                # mapping, pairs, stream
    "pkv_convert_fp8": (ctypes.c_int, [
        _c_void_p, _c_void_p, _i64, _f32,                            # dst, src, n, scale
        _i32, _i32, _c_void_p]),                                     # src/dst dtype, stream
    "pkv_max_shared_memory_per_block": (ctypes.c_int, [_i32, ctypes.POINTER(_i64)]),
    "pkv_get_device_attribute": (ctypes.c_int, [_i32, _i32, ctypes.POINTER(_i64)]),
}

_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; ImportError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is not built; run `make -C sglang-mlx_amd/csrc -j8` "
                    "(or __graft_entry__.build())")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def check(status: int) -> None:
    """Translate a non-zero status into the reference's Python exception types."""
    if status == PKV_OK:
        return
    msg = lib().pkv_last_error().decode("utf-8", "replace")
    if status in (PKV_ERR_INVALID, PKV_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(msg)
