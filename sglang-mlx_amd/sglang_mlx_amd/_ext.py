"""Boundary module: the functions of the reference's ``sglang_mlx._ext``
(bindings.cpp:37-134) over PyTorch-ROCm tensors, backed by the gfx950 C ABI.

Argument checks mirror the reference host ops (mlx_paged_attention.cpp:156-199)
with the same messages and exception types and run before anything touches a
GPU, so they behave the same on CPU tensors.  Kernels launch asynchronously
on the current HIP stream of the tensors' device, as MLX's lazy evaluation
does on its GPU stream.

Deliberate differences from the reference, all on inputs it cannot serve:
  * no LDS ceiling on max_seq_len (the decode kernel streams the softmax, so
    the threadgroup-memory check of mlx_paged_attention.cpp:192-199 can never
    fail);
  * key_cache's last dimension must equal 16 / element size (the reference
    kernel hard-codes it without checking, paged_attention_kernels.metal:80);
  * reshape_and_cache validates shapes (the reference checks none,
    mlx_cache.cpp:256-278) and also accepts the token-major MHATokenPool
    buffers [num_slots, Hkv, D];
  * ``paged_attention_v2`` adds split-K decode, absent from the reference.
"""

from __future__ import annotations

import ctypes
import math
import threading

import torch

from . import _lib

_DTYPE_CODE = {torch.float32: _lib.PKV_F32, torch.float16: _lib.PKV_F16, torch.bfloat16: _lib.PKV_BF16}
_ELEM_BYTES = {torch.float32: 4, torch.float16: 2, torch.bfloat16: 2, torch.uint8: 1}
# uint8 tensors hold FP8 E4M3 codes (the reference's uchar, float8.metal).
_FP8_DTYPE_CODE = {**_DTYPE_CODE, torch.uint8: _lib.PKV_FP8_E4M3}
_HEAD_SIZES = (32, 64, 80, 96, 112, 120, 128, 192, 256)
_BLOCK_SIZES = (8, 16, 32)


def _tensor(x, allow_none: bool = False):
    if x is None and allow_none:
        return None
    if not isinstance(x, torch.Tensor):
        raise TypeError("Expected torch.Tensor")
    return x


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError("Unsupported dtype") from None


def _on_gpu(op: str, *tensors) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if t is not None and (t.device.type != "cuda" or t.device != dev):
            raise RuntimeError(f"{op} is GPU-only")
    if dev.type != "cuda":
        raise RuntimeError(f"{op} is GPU-only")
    return dev


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _check_index(t: torch.Tensor) -> None:
    if t.dtype.is_floating_point or t.dtype.is_complex or t.dtype == torch.bool:
        raise ValueError("index tensors must have an integer dtype")


def _as_i32(t: torch.Tensor) -> torch.Tensor:
    """32-bit index buffer (the kernels read int32; uint32 keeps its bits)."""
    _check_index(t)
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


# ---------------------------------------------------------------------------
# Decode scratch, one buffer per (device, stream).  Its first
# PKV_COUNTER_BYTES are arrival counters that start at zero (a new buffer is
# zero-filled) and that every call leaves at zero; the rest is read only
# where the same launch wrote it.  So calls ordered on one stream share it
# whatever their shapes.
# ---------------------------------------------------------------------------
_ws_lock = threading.Lock()
_ws_cache: dict = {}


def _decode_scratch(dev: torch.device, stream: int, scratch_bytes: int) -> torch.Tensor:
    key = (dev.index, stream)
    with _ws_lock:
        scratch = _ws_cache.get(key)
        if scratch is None or scratch.numel() < scratch_bytes:
            scratch = torch.zeros(max(scratch_bytes, 1 << 17), dtype=torch.uint8, device=dev)
            _ws_cache[key] = scratch
        return scratch


def _cache_layout(key_cache, value_cache) -> int:
    """PKV_LAYOUT_PAGED5D for K [nb, Hkv, D/x, bs, x] / V [nb, Hkv, D, bs]
    (the reference's layout), PKV_LAYOUT_TOKEN_MAJOR for token rows: K and V
    [rows, Hkv, D] (MHATokenPool; block size 1) or [nb, bs, Hkv, D]."""
    if key_cache.dim() == 5 and value_cache.dim() == 4:
        return _lib.PKV_LAYOUT_PAGED5D
    if key_cache.dim() in (3, 4) and value_cache.dim() == key_cache.dim():
        return _lib.PKV_LAYOUT_TOKEN_MAJOR
    raise ValueError("key_cache/value_cache must use paged attention layouts")


def _check_paged_attention(query, key_cache, value_cache, block_tables, context_lens,
                           num_kv_heads, block_size, max_seq_len, alibi_slopes):
    """Checks of mlx_paged_attention.cpp:156-188, same order and messages;
    token-row caches (an extension) get the same checks on their own dims."""
    if query.dim() != 3:
        raise ValueError("query must have shape [num_seqs, num_heads, head_size]")
    layout = _cache_layout(key_cache, value_cache)
    rows = layout == _lib.PKV_LAYOUT_TOKEN_MAJOR
    if block_tables.dim() != 2 or context_lens.dim() != 1:
        raise ValueError("block_tables must be 2D and context_lens must be 1D")
    if query.shape[0] != block_tables.shape[0] or query.shape[0] != context_lens.shape[0]:
        raise ValueError("query, block_tables, and context_lens sequence counts differ")
    if num_kv_heads <= 0 or query.shape[1] % num_kv_heads != 0:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    if rows:
        cache_bs = key_cache.shape[1] if key_cache.dim() == 4 else 1
        if key_cache.shape[-2] != num_kv_heads or value_cache.shape[-2] != num_kv_heads:
            raise ValueError("cache KV-head count does not match num_kv_heads")
        if key_cache.shape[-1] != query.shape[2] or value_cache.shape[-1] != query.shape[2]:
            raise ValueError("cache head size does not match query head size")
        if key_cache.shape[:-2] != value_cache.shape[:-2] or cache_bs != block_size:
            raise ValueError("cache block dimensions do not match block_size")
    else:
        if key_cache.shape[1] != num_kv_heads or value_cache.shape[1] != num_kv_heads:
            raise ValueError("cache KV-head count does not match num_kv_heads")
        if key_cache.shape[2] * key_cache.shape[4] != query.shape[2] or value_cache.shape[2] != query.shape[2]:
            raise ValueError("cache head size does not match query head size")
        if (key_cache.shape[0] != value_cache.shape[0] or key_cache.shape[3] != block_size
                or value_cache.shape[3] != block_size):
            raise ValueError("cache block dimensions do not match block_size")
    if alibi_slopes is not None and (alibi_slopes.dim() != 1 or alibi_slopes.shape[0] != query.shape[1]):
        raise ValueError("alibi_slopes must have shape [num_heads]")
    if max_seq_len <= 0:
        raise ValueError("max_seq_len must be positive")
    if max_seq_len > block_tables.shape[1] * block_size:
        raise ValueError("max_seq_len exceeds block table capacity")
    if query.shape[2] not in _HEAD_SIZES or not (block_size in _BLOCK_SIZES or (rows and block_size == 1)):
        raise ValueError("Unsupported head_size/block_size for paged_attention")
    # Checks the reference leaves to the kernel.
    qc = _dtype_code(query)
    try:
        cc = _FP8_DTYPE_CODE[key_cache.dtype]
    except KeyError:
        raise ValueError("Unsupported dtype") from None
    if value_cache.dtype != key_cache.dtype:
        raise ValueError("key_cache and value_cache dtypes differ")
    if not rows and key_cache.shape[4] != 16 // _ELEM_BYTES[key_cache.dtype]:
        raise ValueError("key_cache last dimension must be 16 / element size of the cache dtype")
    fp8 = cc == _lib.PKV_FP8_E4M3
    if not (qc == cc or qc == _lib.PKV_F32 or fp8):
        raise ValueError(
            f"Unsupported query/cache dtype pair for paged_attention: {query.dtype}/{key_cache.dtype}")
    if cc == _lib.PKV_F32 and rows:
        raise ValueError("float32 caches are read in the paged layout")
    if fp8 and (rows or query.shape[2] % 16):
        raise ValueError("FP8 caches are read in the paged layout with head_size a multiple of 16")
    if not rows:
        # The kernels take any block and head strides but read each (block,
        # head) region as one contiguous run; a cache that is not is
        # rejected rather than silently copied whole on every call.
        x = key_cache.shape[4]
        if key_cache.stride()[2:] != (block_size * x, x, 1):
            raise ValueError("key_cache must be contiguous within each (block, head) region [head_size/x, "
                             "block_size, x]")
        if value_cache.stride()[2:] != (block_size, 1):
            raise ValueError("value_cache must be contiguous within each (block, head) region [head_size, "
                             "block_size]")
    if rows:
        # Rows must be [Hkv, D]-contiguous, and the rows of a block evenly
        # spaced (block stride = block_size * row stride).
        H, D = key_cache.shape[-2], key_cache.shape[-1]
        for name, c in (("key_cache", key_cache), ("value_cache", value_cache)):
            if c.stride()[-2:] != (D, 1) or (c.dim() == 4 and (c.stride(1) < H * D
                                                                or c.stride(0) != c.shape[1] * c.stride(1))):
                raise ValueError(f"{name} rows must be contiguous [num_kv_heads, head_size]")
    return qc, cc, layout


def _plan_struct(plan, B: int, dev: torch.device):
    """The ctypes pkv_cascade_plan of a CascadePlan (checked: int32 tensors
    on the query's device, contiguous, with the shapes the header states)."""
    arrays = {}
    for name, shape in (("prefix_lens", (B,)), ("members", None), ("tiles", None), ("parts", None)):
        t = getattr(plan, name)
        if not isinstance(t, torch.Tensor) or t.dtype != torch.int32 or t.device != dev or not t.is_contiguous():
            raise ValueError(f"cascade plan: {name} must be a contiguous int32 tensor on {dev}")
        if shape is not None and tuple(t.shape) != shape:
            raise ValueError(f"cascade plan: {name} must have shape {list(shape)}")
        arrays[name] = t
    tiles, parts = arrays["tiles"], arrays["parts"]
    if tiles.dim() != 2 or tiles.shape[1] != 4:
        raise ValueError("cascade plan: tiles must have shape [num_tiles, 4]")
    if parts.dim() != 2 or parts.shape[1] != 2:
        raise ValueError("cascade plan: parts must have shape [num_parts, 2]")
    if arrays["members"].dim() != 1:
        raise ValueError("cascade plan: members must be 1-D")
    ptr = lambda t: t.data_ptr() if t.numel() else None  # noqa: E731
    return _lib.CascadePlanC(ptr(arrays["prefix_lens"]), ptr(arrays["members"]), ptr(tiles), ptr(parts),
                             arrays["members"].numel(), tiles.shape[0], parts.shape[0], int(plan.chunk_tokens),
                             int(plan.max_chunks), int(plan.part_tokens), int(plan.max_parts))


def _paged_attention(op, query, key_cache, value_cache, block_tables, context_lens, num_kv_heads,
                     scale, block_size, max_seq_len, alibi_slopes, partition_size, k_scale=1.0, v_scale=1.0,
                     plan=None):
    for t in (query, key_cache, value_cache, block_tables, context_lens):
        _tensor(t)
    _tensor(alibi_slopes, allow_none=True)
    num_kv_heads, block_size, max_seq_len = int(num_kv_heads), int(block_size), int(max_seq_len)
    qc, cc, layout = _check_paged_attention(query, key_cache, value_cache, block_tables, context_lens,
                                            num_kv_heads, block_size, max_seq_len, alibi_slopes)
    k_scale, v_scale = float(k_scale), float(v_scale)
    if cc == _lib.PKV_FP8_E4M3 and not all(math.isfinite(v) and v != 0.0 for v in (k_scale, v_scale)):
        raise ValueError("k_scale and v_scale must be finite and nonzero for FP8 caches")
    _check_index(block_tables)
    _check_index(context_lens)
    dev = _on_gpu(op, query, key_cache, value_cache, block_tables, context_lens, alibi_slopes)
    B, Hq, D = query.shape
    if query.stride(2) != 1 or query.stride(1) != D or (query.stride(0) * _ELEM_BYTES[query.dtype]) % 16:
        query = query.contiguous()
    bt = _as_i32(block_tables)
    lens = _as_i32(context_lens)
    alibi = None if alibi_slopes is None else alibi_slopes.to(torch.float32).contiguous()
    out = torch.empty((B, Hq, D), dtype=query.dtype, device=dev)
    if B == 0:
        return out
    lib = _lib.lib()
    if plan is not None:
        if layout != _lib.PKV_LAYOUT_PAGED5D:
            raise ValueError("paged_attention_cascade reads the paged 5-D layout")
        cplan = _plan_struct(plan, B, dev)
        with torch.cuda.device(dev):
            stream = _stream(dev)
            need = lib.pkv_paged_attention_cascade_workspace_size(B, Hq, num_kv_heads, D, max_seq_len,
                                                                  int(plan.max_chunks), int(plan.max_parts))
            if need == 0:
                raise ValueError("cascade plan: invalid sizes (max_chunks and max_parts must be in [1, 65536])")
            ws = _decode_scratch(dev, stream, need)
            st = lib.pkv_paged_attention_cascade(
                out.data_ptr(), query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
                bt.data_ptr(), lens.data_ptr(), None if alibi is None else alibi.data_ptr(), ctypes.byref(cplan),
                B, Hq, num_kv_heads, D, block_size, bt.shape[1], max_seq_len, key_cache.shape[0],
                float(scale), query.stride(0), key_cache.stride(0), key_cache.stride(1),
                value_cache.stride(0), value_cache.stride(1), ws.data_ptr(), ws.numel(), qc, cc, k_scale,
                v_scale, stream)
        _lib.check(st)
        return out
    with torch.cuda.device(dev):
        stream = _stream(dev)
        need = lib.pkv_paged_attention_workspace_size(B, Hq, num_kv_heads, D, max_seq_len,
                                                      partition_size)
        if need == 0:
            _lib.check(_lib.PKV_ERR_INVALID)
        ws = _decode_scratch(dev, stream, need)
        st = lib.pkv_paged_attention(
            out.data_ptr(), query.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
            bt.data_ptr(), lens.data_ptr(), None if alibi is None else alibi.data_ptr(),
            B, Hq, num_kv_heads, D, block_size, bt.shape[1], max_seq_len, key_cache.shape[0],
            float(scale), query.stride(0), key_cache.stride(0), key_cache.stride(-2 if layout else 1),
            value_cache.stride(0), value_cache.stride(-2 if layout else 1), layout, partition_size,
            ws.data_ptr(), ws.numel(), qc, cc, k_scale, v_scale, stream)
    _lib.check(st)
    return out


def paged_attention_v1(query, key_cache, value_cache, block_tables, seq_lens, num_kv_heads,
                       scale, block_size, max_seq_len, alibi_slopes=None, k_scale=1.0, v_scale=1.0):
    """Single-softmax paged decode attention (bindings.cpp:44-65).

    Returns a new tensor shaped and typed like ``query``
    (mlx_paged_attention.cpp:212).  uint8 caches hold FP8 E4M3 codes, read
    as decode(code) * k_scale / v_scale.
    """
    return _paged_attention("PagedAttentionV1", query, key_cache, value_cache, block_tables, seq_lens,
                            num_kv_heads, scale, block_size, max_seq_len, alibi_slopes, 0, k_scale, v_scale)


def paged_attention_v2(query, key_cache, value_cache, block_tables, seq_lens, num_kv_heads,
                       scale, block_size, max_seq_len, alibi_slopes=None, partition_size=512, k_scale=1.0,
                       v_scale=1.0):
    """Split-K paged decode: softmax per partition of ``partition_size``
    tokens, merged across partitions by log-sum-exp.  Same arguments and
    result as ``paged_attention_v1`` plus ``partition_size``.  A workgroup
    takes a run of consecutive partitions (as many as keep one workgroup per
    CU) and merges them as it streams; the merge kernel combines the runs by
    the same rule, so the result is the same softmax either way."""
    partition_size = int(partition_size)
    if partition_size <= 0 or partition_size % 16 or partition_size % int(block_size) or partition_size > 4096:
        raise ValueError("partition_size must be a positive multiple of 16 and of block_size, at most 4096")
    return _paged_attention("PagedAttentionV2", query, key_cache, value_cache, block_tables, seq_lens,
                            num_kv_heads, scale, block_size, max_seq_len, alibi_slopes, partition_size,
                            k_scale, v_scale)


def paged_attention_cascade(query, key_cache, value_cache, block_tables, seq_lens, num_kv_heads,
                            scale, block_size, max_seq_len, plan, alibi_slopes=None, k_scale=1.0,
                            v_scale=1.0):
    """paged_attention_v1 with radix-shared prefixes computed once per
    group: ``plan`` (srt.mem_cache.build_cascade_plan) lists the sequences
    whose block tables begin with the same blocks.  A prefix pass attends
    every member's query rows to the shared tokens at once; a tail pass
    streams each sequence's remaining tokens and folds the prefix state in.
    Same arguments and result as ``paged_attention_v1`` (paged 5-D caches);
    shapes the cascade kernels do not cover run the one-pass decode."""
    return _paged_attention("PagedAttentionCascade", query, key_cache, value_cache, block_tables, seq_lens,
                            num_kv_heads, scale, block_size, max_seq_len, alibi_slopes, 0, k_scale, v_scale,
                            plan=plan)


def _reshape_and_cache(op, key, value, key_cache, value_cache, slot_mapping, flash: bool,
                       k_scale: float = 1.0, v_scale: float = 1.0):
    for t in (key, value, key_cache, value_cache, slot_mapping):
        _tensor(t)
    if key.dim() != 3 or value.shape != key.shape:
        raise ValueError("key and value must have shape [num_tokens, num_kv_heads, head_size]")
    if slot_mapping.dim() != 1 or slot_mapping.shape[0] != key.shape[0]:
        raise ValueError("slot_mapping must have shape [num_tokens]")
    N, H, D = key.shape
    if value_cache.dtype != key_cache.dtype:
        raise ValueError("key_cache and value_cache dtypes differ")
    kvc = _dtype_code(key)
    try:
        cc = _FP8_DTYPE_CODE[key_cache.dtype]
    except KeyError:
        raise ValueError("Unsupported dtype") from None
    if value.dtype != key.dtype:
        raise ValueError("key and value dtypes differ")
    fp8 = cc == _lib.PKV_FP8_E4M3
    if not (kvc == cc or kvc == _lib.PKV_F32 or fp8):
        raise ValueError(f"Unsupported key/cache dtype pair: {key.dtype} -> {key_cache.dtype}")
    k_scale, v_scale = float(k_scale), float(v_scale)
    if fp8 and not all(math.isfinite(v) and v != 0.0 for v in (k_scale, v_scale)):
        raise ValueError("k_scale and v_scale must be finite and nonzero for FP8 caches")
    x = 16 // _ELEM_BYTES[key_cache.dtype]
    if not flash and key_cache.dim() == 5:
        layout = _lib.PKV_LAYOUT_PAGED5D
        nb, bs = key_cache.shape[0], key_cache.shape[3]
        if tuple(key_cache.shape) != (nb, H, D // x, bs, x) or D % x:
            raise ValueError("key_cache must have shape [num_blocks, num_kv_heads, head_size/x, block_size, x]")
        if tuple(value_cache.shape) != (nb, H, D, bs):
            raise ValueError("value_cache must have shape [num_blocks, num_kv_heads, head_size, block_size]")
        num_slots = nb * bs
    elif key_cache.dim() in ((3, 4) if flash else (3,)):
        layout = _lib.PKV_LAYOUT_TOKEN_MAJOR
        if tuple(key_cache.shape[-2:]) != (H, D) or value_cache.shape != key_cache.shape:
            raise ValueError("token-major caches must have shape [..., num_kv_heads, head_size]")
        num_slots = key_cache.numel() // (H * D) if H * D else 0
        bs = key_cache.shape[1] if key_cache.dim() == 4 else 1
        if fp8 and (H * D) % 8:
            raise ValueError("FP8 token-major caches need num_kv_heads * head_size to be a multiple of 8")
    else:
        raise ValueError("key_cache/value_cache must use a paged or token-major layout")
    if not key_cache.is_contiguous() or not value_cache.is_contiguous():
        raise ValueError("key_cache and value_cache must be contiguous (they are updated in place)")
    _check_index(slot_mapping)
    dev = _on_gpu(op, key, value, key_cache, value_cache, slot_mapping)
    # Rows must be [Hkv, D]-contiguous at a stride of at least Hkv * D; a
    # single row's stride is meaningless (views of one token may carry any).
    if key.stride()[1:] != (D, 1) or (N > 1 and key.stride(0) < H * D):
        key = key.contiguous()
    if value.stride()[1:] != (D, 1) or (N > 1 and value.stride(0) < H * D):
        value = value.contiguous()
    key_stride = key.stride(0) if N > 1 else H * D
    value_stride = value.stride(0) if N > 1 else H * D
    slots = _as_i32(slot_mapping)
    if N == 0:
        return [key_cache, value_cache]
    lib = _lib.lib()
    with torch.cuda.device(dev):
        st = lib.pkv_reshape_and_cache(
            key.data_ptr(), value.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
            slots.data_ptr(), N, H, D, key_stride, value_stride, layout, bs, x, num_slots,
            kvc, cc, k_scale, v_scale, _stream(dev))
    _lib.check(st)
    return [key_cache, value_cache]


def reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, k_scale: float = 1.0,
                      v_scale: float = 1.0):
    """Scatter new tokens into the cache in place; returns [key_cache, value_cache].

    Paged 5-D caches follow mlx_cache.cpp:256-278; 3-D [num_slots, Hkv, D]
    caches (MHATokenPool buffers) use the token-major kernel.  uint8 caches
    hold FP8 E4M3 codes of key / k_scale and value / v_scale (x = 16).
    """
    return _reshape_and_cache("ReshapeAndCache", key, value, key_cache, value_cache, slot_mapping, False,
                              k_scale, v_scale)


def reshape_and_cache_flash(key, value, key_cache, value_cache, slot_mapping, k_scale: float = 1.0,
                            v_scale: float = 1.0):
    """Scatter into [num_blocks, block_size, Hkv, D] caches (mlx_cache.cpp:280-300)."""
    return _reshape_and_cache("ReshapeAndCacheFlash", key, value, key_cache, value_cache, slot_mapping,
                              True, k_scale, v_scale)


def _block_mapping(block_mapping) -> torch.Tensor:
    _tensor(block_mapping)
    if block_mapping.dim() != 2 or block_mapping.shape[1] != 2:
        raise ValueError("block_mapping must have shape [num_pairs, 2]")
    _check_index(block_mapping)
    return block_mapping


def _copy_planes(src_planes, dst_planes, src_blocks, dst_blocks, block_bytes, mapping, dev):
    """One pkv_copy_blocks call over planes that share block counts and size."""
    import ctypes
    n = len(src_planes)
    if n == 0 or mapping.shape[0] == 0:
        return
    m = mapping.to(device=dev, dtype=torch.int64).contiguous()
    src_arr = (ctypes.c_void_p * n)(*[t.data_ptr() for t in src_planes])
    dst_arr = (ctypes.c_void_p * n)(*[t.data_ptr() for t in dst_planes])
    with torch.cuda.device(dev):
        st = _lib.lib().pkv_copy_blocks(src_arr, dst_arr, n, src_blocks, dst_blocks, block_bytes, m.data_ptr(),
                                        m.shape[0], _stream(dev))
    _lib.check(st)


def copy_blocks(key_caches, value_caches, block_mapping):
    """Copy whole blocks src -> dst inside every layer's K and V cache, in
    place (mlx_cache.cpp:302-346, copy_blocks.metal:9-39); returns the two
    lists.  Checks and messages follow mlx_cache.cpp:308-330.  Pairs are
    copied concurrently (a block that is both a source and a destination in
    one call gives an unspecified result, as in the reference); pairs with
    out-of-range block ids are skipped."""
    key_caches, value_caches = list(key_caches), list(value_caches)
    if len(key_caches) != len(value_caches):
        raise ValueError("key_caches and value_caches size mismatch")
    mapping = _block_mapping(block_mapping)
    groups = []  # runs of layers with the same (device, blocks, block bytes)
    for kc, vc in zip(key_caches, value_caches):
        _tensor(kc)
        _tensor(vc)
        if kc.dim() == 0 or vc.dim() == 0 or kc.shape[0] == 0 or vc.shape[0] == 0 or kc.shape[0] != vc.shape[0]:
            raise ValueError("key/value caches must have matching block counts")
        if kc.dtype != vc.dtype or kc.numel() // kc.shape[0] != vc.numel() // vc.shape[0]:
            raise ValueError("key/value cache block layouts must match")
        if not kc.is_contiguous() or not vc.is_contiguous():
            raise ValueError("key/value caches must be contiguous (they are updated in place)")
        dev = _on_gpu("CopyBlocksLayer", kc, vc)
        key = (dev, kc.shape[0], kc.numel() // kc.shape[0] * kc.element_size())
        if groups and groups[-1][0] == key:
            groups[-1][1].extend((kc, vc))
        else:
            groups.append((key, [kc, vc]))
    for (dev, nb, block_bytes), planes in groups:
        _copy_planes(planes, planes, nb, nb, block_bytes, mapping, dev)
    return key_caches, value_caches


def swap_blocks(src, dst, block_mapping):
    """dst[m[:, 1]] = src[m[:, 0]] block by block (mlx_cache.cpp:348-370,
    copy_blocks.metal:55-70); updates and returns dst.  Between two tensors on
    one GPU this is the copy kernel.  With one side in host memory (the
    offload use) the blocks travel through one pinned staging buffer in a
    single copy on the current stream:
      host -> GPU: the host gathers the source blocks into pinned memory, one
        asynchronous copy moves them to a device buffer, and the copy kernel
        scatters them into dst (nothing waits);
      GPU -> host: the copy kernel gathers the source blocks into a device
        buffer, one copy moves them into pinned memory, and after the stream
        has reached it the host scatters them into dst (the call returns
        with dst updated).
    Pairs with out-of-range block ids are skipped.  Tensors on two different
    GPUs are rejected (this path runs one process per GPU)."""
    _tensor(src)
    _tensor(dst)
    if src.dim() == 0 or dst.dim() == 0 or src.shape[0] == 0 or dst.shape[0] == 0:
        raise ValueError("src and dst must have a leading block dimension")
    if src.dtype != dst.dtype or src.numel() // src.shape[0] != dst.numel() // dst.shape[0]:
        raise ValueError("src and dst block layouts must match")
    mapping = _block_mapping(block_mapping)
    if not src.is_contiguous() or not dst.is_contiguous():
        raise ValueError("src and dst must be contiguous")
    if src.device.type == "cuda" and dst.device == src.device:
        _copy_planes([src], [dst], src.shape[0], dst.shape[0], src.numel() // src.shape[0] * src.element_size(),
                     mapping, src.device)
        return dst
    if src.device.type != "cuda" and dst.device.type != "cuda":
        raise RuntimeError("SwapBlocks is GPU-only")
    if src.device.type == "cuda" and dst.device.type == "cuda":
        raise RuntimeError("SwapBlocks between two GPUs is not supported")
    m = mapping.to("cpu", torch.int64)
    keep = (m[:, 0] >= 0) & (m[:, 0] < src.shape[0]) & (m[:, 1] >= 0) & (m[:, 1] < dst.shape[0])
    m = m[keep]
    n = m.shape[0]
    if n == 0:
        return dst
    block_shape = tuple(src.shape[1:])
    block_bytes = src.numel() // src.shape[0] * src.element_size()
    dev = dst.device if dst.device.type == "cuda" else src.device
    staging = torch.empty((n,) + block_shape, dtype=src.dtype, pin_memory=True)
    dev_buf = torch.empty((n,) + block_shape, dtype=src.dtype, device=dev)
    order = torch.arange(n, dtype=torch.int64)
    if dst.device.type == "cuda":
        torch.index_select(src, 0, m[:, 0], out=staging)
        with torch.cuda.device(dev):
            dev_buf.copy_(staging, non_blocking=True)
        # Row i of the device buffer -> block m[i, 1] of dst.
        _copy_planes([dev_buf], [dst], n, dst.shape[0], block_bytes, torch.stack([order, m[:, 1]], 1), dev)
    else:
        _copy_planes([src], [dev_buf], src.shape[0], n, block_bytes, torch.stack([m[:, 0], order], 1), dev)
        with torch.cuda.device(dev):
            staging.copy_(dev_buf, non_blocking=True)
            torch.cuda.current_stream(dev).synchronize()
        dst[m[:, 1]] = staging
    return dst


def get_device_attribute(attribute, device_id=0):
    """hipDeviceGetAttribute(attribute, device_id)."""
    import ctypes
    v = ctypes.c_int64(0)
    _lib.check(_lib.lib().pkv_get_device_attribute(int(attribute), int(device_id), ctypes.byref(v)))
    return v.value


def get_max_shared_memory_per_block_device_attribute(device_id=0):
    """LDS bytes per workgroup (mlx_device.cpp:16-20)."""
    import ctypes
    v = ctypes.c_int64(0)
    _lib.check(_lib.lib().pkv_max_shared_memory_per_block(int(device_id), ctypes.byref(v)))
    return v.value


def convert_fp8(dst, src, scale: float = 1.0):
    """Element-wise conversion with a scale (convert_fp8.metal:13-80) between
    float32, float16, bfloat16 and uint8 tensors of FP8 E4M3 codes: decode
    then multiply into wider types, divide then encode into codes, multiply
    between wider types.  Writes dst in place and returns it."""
    _tensor(dst)
    _tensor(src)
    if dst.dtype not in _FP8_DTYPE_CODE or src.dtype not in _FP8_DTYPE_CODE:
        raise ValueError(f"Unsupported dtype pair for convert_fp8: {src.dtype} -> {dst.dtype}")
    if dst.numel() != src.numel():
        raise ValueError("dst and src must have the same number of elements")
    if not dst.is_contiguous():
        raise ValueError("dst must be contiguous (it is written in place)")
    dev = _on_gpu("ConvertFp8", dst, src)
    if not src.is_contiguous():
        src = src.contiguous()
    n = src.numel()
    if n == 0:
        return dst
    with torch.cuda.device(dev):
        st = _lib.lib().pkv_convert_fp8(dst.data_ptr(), src.data_ptr(), n, float(scale),
                                        _FP8_DTYPE_CODE[src.dtype], _FP8_DTYPE_CODE[dst.dtype], _stream(dev))
    _lib.check(st)
    return dst

