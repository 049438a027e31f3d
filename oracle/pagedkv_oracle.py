"""CPU oracle for the paged-KV hot path -- TEST INFRASTRUCTURE ONLY.

This module restates the reference's algorithms in NumPy so that tests,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` can
check the HIP kernels.  Nothing in the product package imports it; the
product path fails loudly when its HIP library is missing instead of falling
back to anything here.

Representation: 16-bit caches are carried as ``uint16`` bit arrays together
with a dtype name (``"float16"`` / ``"bfloat16"``); float32 data as
``float32``.  The append functions work on those raw arrays (bit-exact); the
attention functions decode to float64 and compute in float64.

Functions and the reference code they restate (paths relative to the
reference repository):

- ``f32_to_bf16_bits``     paged_attention/metal/utils.metal:21-35
- ``convert_elements``     paged_attention/metal/cache/reshape_and_cache.metal:9-12
- ``reshape_and_cache_paged5d``
                           reshape_and_cache.metal:35-69;
                           tests/test_paged_attention_kernel.py:33-65
- ``reshape_and_cache_token_major``
                           reshape_and_cache.metal:115-136;
                           sglang_mlx/srt/mem_cache/memory_pool.py:117-137
- ``paged_attention``      paged_attention/metal/attention/paged_attention_kernels.metal:37-168;
                           tests/test_paged_attention_kernel.py:68-120
- ``paged_attention_split``  (no reference code: split-K is absent from the
                           reference, README.md:11-19) log-sum-exp merge of
                           per-partition (max, sum, output).
- ``gather_kv``            the per-token gather of test_paged_attention_kernel.py:93-105
- ``copy_blocks``, ``swap_blocks``
                           paged_attention/metal/cache/copy_blocks.metal:9-39, :55-70;
                           paged_attention/mlx_cache.cpp:302-370
- ``fp8_e4m3_decode``      paged_attention/metal/float8.metal:13-38
- ``fp8_e4m3_encode``      paged_attention/metal/float8.metal:72-124 (including
                           its behaviour for 256 <= |x| < 2^14 and near 2^-6, kept
                           as is; +-inf where its shifts are undefined)
- ``convert_fp8``          paged_attention/metal/convert_fp8.metal:13-47

FP8 codes are ``uint8`` arrays (the reference's ``uchar``), format E4M3 with
bias 7 in which exponent 15 is +-inf (mantissa 0) or NaN.

Pinning (tests/test_oracle_*.py, tests/test_fp8_oracle.py): the FP8 decode
table against torch's float8_e4m3fn on the 240 codes both formats share and
known values elsewhere; the encoder by round trips over every finite code,
torch's round-to-nearest-even in the normal range, brute-force nearest search
in the subnormal range and explicit cases of its overflow and wrap-around
behaviour; bf16/fp16 rounding against torch's
conversions; the append against the element loop of the reference's own test
and read-back invariants; attention against torch's float64
scaled_dot_product_attention, closed forms (single token, equal keys,
one-hot logits, ALiBi geometric weights) and the reference's zero-output
cases; split-K against the unpartitioned oracle.
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# Element conversions (bit level)
# ---------------------------------------------------------------------------

DTYPES = ("float32", "float16", "bfloat16")


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits: round to nearest even, every NaN -> 0x7FC0.

    Restates float_to_bfloat_bits, paged_attention/metal/utils.metal:21-35.
    """
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    return np.where(nan, 0x7FC0, r).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """bfloat16 bits -> float32 (upper half of the float word), utils.metal:37-40."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return np.asarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> IEEE binary16 bits, round to nearest even (NumPy's cast)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def to_storage(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float data to the storage representation of ``dtype``."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "float32":
        return x.copy()
    if dtype == "float16":
        return f32_to_f16_bits(x)
    if dtype == "bfloat16":
        return f32_to_bf16_bits(x)
    raise ValueError(dtype)


def decode(bits: np.ndarray, dtype: str) -> np.ndarray:
    """Storage representation -> float64 values."""
    if dtype == FP8:
        return fp8_e4m3_decode(bits).astype(np.float64)
    if dtype == "float32":
        return np.asarray(bits, dtype=np.float32).astype(np.float64)
    if dtype == "float16":
        return f16_bits_to_f32(bits).astype(np.float64)
    if dtype == "bfloat16":
        return bf16_bits_to_f32(bits).astype(np.float64)
    raise ValueError(dtype)


def convert_elements(src: np.ndarray, src_dtype: str, dst_dtype: str, scale: float = 1.0) -> np.ndarray:
    """static_cast<CACHE_T>(KV_T), reshape_and_cache.metal:9-12.

    Equal types copy the bits; float32 -> float16/bfloat16 rounds to nearest
    even.  The reference instantiates exactly these pairs
    (reshape_and_cache.metal:91-95).  An FP8 cache (which the reference's
    append does not have) stores encode(float(x) / scale), the quantisation
    of convert_fp8.metal:33-35.
    """
    if dst_dtype == FP8:
        return fp8_e4m3_encode(decode(src, src_dtype).astype(np.float32) / np.float32(scale))
    if src_dtype == dst_dtype:
        return np.array(src, copy=True)
    if src_dtype != "float32":
        raise ValueError(f"unsupported conversion {src_dtype} -> {dst_dtype}")
    return to_storage(src, dst_dtype)


# ---------------------------------------------------------------------------
# Append
# ---------------------------------------------------------------------------


def reshape_and_cache_paged5d(key, value, key_cache, value_cache, slot_mapping,
                              kv_dtype: str, cache_dtype: str, k_scale: float = 1.0, v_scale: float = 1.0):
    """Scatter new tokens into the paged 5-D layout; returns new caches.

    key/value: [N, H, D] storage arrays.  key_cache [nb, H, D/x, bs, x],
    value_cache [nb, H, D, bs].  Token i goes to block slot//bs, offset
    slot%bs; slots < 0 are skipped (reshape_and_cache.metal:35-69).
    Implemented with vectorised fancy indexing; the reference test's element
    loop (test_paged_attention_kernel.py:46-63) is the independent check.
    """
    kc = np.array(key_cache, copy=True)
    vc = np.array(value_cache, copy=True)
    nb, H, dx, bs, x = kc.shape
    D = dx * x
    slots = np.asarray(slot_mapping).astype(np.int64)
    keep = slots >= 0
    tok = np.nonzero(keep)[0]
    if tok.size == 0:
        return kc, vc
    s = slots[keep]
    blk, off = s // bs, s % bs
    k = convert_elements(np.asarray(key)[tok], kv_dtype, cache_dtype, k_scale)  # [n, H, D]
    v = convert_elements(np.asarray(value)[tok], kv_dtype, cache_dtype, v_scale)
    # Two tokens naming one slot race on the GPU (the reference does not
    # order them either); the oracle lets the later token win.
    order = np.arange(tok.size)
    _, last = np.unique(s[::-1], return_index=True)
    sel = order[::-1][last]
    blk, off, k, v = blk[sel], off[sel], k[sel], v[sel]
    d = np.arange(D)
    kc[blk[:, None, None], np.arange(H)[None, :, None], (d // x)[None, None, :],
       off[:, None, None], (d % x)[None, None, :]] = k
    vc[blk[:, None, None], np.arange(H)[None, :, None], d[None, None, :],
       off[:, None, None]] = v
    return kc, vc


def reshape_and_cache_token_major(key, value, key_cache, value_cache, slot_mapping,
                                  kv_dtype: str, cache_dtype: str, k_scale: float = 1.0, v_scale: float = 1.0):
    """Scatter into [num_slots, H, D] (MHATokenPool / flash layout).

    reshape_and_cache.metal:115-136 with slot = block*bs + offset, which is
    the MHATokenPool buffer indexing of memory_pool.py:117-137.
    """
    kc = np.array(key_cache, copy=True)
    vc = np.array(value_cache, copy=True)
    shape = kc.shape
    kc = kc.reshape(-1, shape[-2], shape[-1])
    vc = vc.reshape(-1, shape[-2], shape[-1])
    slots = np.asarray(slot_mapping).astype(np.int64)
    tok = np.nonzero(slots >= 0)[0]
    if tok.size:
        s = slots[tok]
        _, last = np.unique(s[::-1], return_index=True)
        sel = np.arange(tok.size)[::-1][last]
        kc[s[sel]] = convert_elements(np.asarray(key)[tok[sel]], kv_dtype, cache_dtype, k_scale)
        vc[s[sel]] = convert_elements(np.asarray(value)[tok[sel]], kv_dtype, cache_dtype, v_scale)
    return kc.reshape(shape), vc.reshape(shape)


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------


def gather_kv(kc64: np.ndarray, vc64: np.ndarray, block_row: np.ndarray, ctx: int):
    """Logical tokens 0..ctx-1 of one sequence -> (K, V) as [ctx, H, D].

    kc64 [nb, H, D/x, bs, x] and vc64 [nb, H, D, bs] hold decoded values.
    Token t lives in block block_row[t // bs] at offset t % bs
    (test_paged_attention_kernel.py:93-105).
    """
    nb, H, dx, bs, x = kc64.shape
    t = np.arange(ctx)
    blk = np.asarray(block_row, dtype=np.int64)[t // bs]
    off = t % bs
    k = kc64[blk, :, :, off, :].reshape(ctx, H, dx * x)  # [ctx, H, D/x, x] -> [ctx, H, D]
    v = vc64[blk, :, :, off]                              # [ctx, H, D]
    return k, v


def _softmax_attend(qh: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
                    bias: np.ndarray | None):
    """One sequence, all heads: qh [Hq, D]; k, v [T, Hkv, D] -> [Hq, D].

    Query head h reads KV head h // (Hq/Hkv) (paged_attention_kernels.metal:57-58);
    scale, then ALiBi (:95-97), max-subtracted exp, denominator
    (sum + 1e-6) (:144), weighted V sum (:146-160).
    """
    Hq, D = qh.shape
    Hkv = k.shape[1]
    qg = qh.reshape(Hkv, Hq // Hkv, D)
    logits = np.einsum("kgd,tkd->kgt", qg, k) * scale
    if bias is not None:
        logits = logits + bias.reshape(Hkv, Hq // Hkv, -1)
    m = logits.max(axis=2, keepdims=True)
    p = np.exp(logits - m)
    inv = 1.0 / (p.sum(axis=2, keepdims=True) + 1e-6)
    return np.einsum("kgt,tkd->kgd", p * inv, v).reshape(Hq, D)


def alibi_bias(slopes: np.ndarray, ctx: int) -> np.ndarray:
    """slope[h] * (t - ctx + 1), paged_attention_kernels.metal:97."""
    t = np.arange(ctx)
    return np.asarray(slopes, dtype=np.float64)[:, None] * (t - ctx + 1)[None, :]


def paged_attention(q, key_cache, value_cache, block_tables, context_lens, num_kv_heads: int,
                    scale: float, block_size: int, max_seq_len: int, alibi_slopes=None,
                    q_dtype: str = "float32", cache_dtype: str = "float32",
                    k_scale: float = 1.0, v_scale: float = 1.0) -> np.ndarray:
    """paged_attention_v1 in float64 -> [B, Hq, D] float64.

    Follows paged_attention_kernels.metal:37-168: zero output when
    ctx == 0 or ctx > max_seq_len (:44-50, context read as uint32),
    GQA map h // (Hq/Hkv) (:57-58), fp32-exact inputs, denominator
    sum + 1e-6 (:144).  ``block_size`` is implied by the cache shape and
    only cross-checked.  FP8 caches (an extension; the reference's decode
    reads 16/32-bit caches only) are read as decode(code) * k_scale and
    decode(code) * v_scale, the dequantisation of convert_fp8.metal:27-29.
    """
    q64 = decode(q, q_dtype)
    kc64 = decode(key_cache, cache_dtype)
    vc64 = decode(value_cache, cache_dtype)
    if cache_dtype == FP8:
        kc64 = kc64 * k_scale
        vc64 = vc64 * v_scale
    assert kc64.shape[3] == block_size
    B, Hq, D = q64.shape
    assert Hq % num_kv_heads == 0
    out = np.zeros((B, Hq, D), dtype=np.float64)
    lens = np.asarray(context_lens).astype(np.int64) & 0xFFFFFFFF
    for s in range(B):
        ctx = int(lens[s])
        if ctx == 0 or ctx > max_seq_len:
            continue
        k, v = gather_kv(kc64, vc64, block_tables[s], ctx)
        bias = None if alibi_slopes is None else alibi_bias(alibi_slopes, ctx)
        out[s] = _softmax_attend(q64[s], k, v, scale, bias)
    return out


def partition_stats(qh, k, v, scale, bias, lo: int, hi: int):
    """(max, sum, normalised output) of tokens [lo, hi) for all heads."""
    Hq, D = qh.shape
    Hkv = k.shape[1]
    qg = qh.reshape(Hkv, Hq // Hkv, D)
    logits = np.einsum("kgd,tkd->kgt", qg, k[lo:hi]).reshape(Hq, hi - lo) * scale
    if bias is not None:
        logits = logits + bias[:, lo:hi]
    m = logits.max(axis=1)
    p = np.exp(logits - m[:, None])
    s = p.sum(axis=1)
    o = np.einsum("kgt,tkd->kgd", p.reshape(Hkv, Hq // Hkv, -1), v[lo:hi]).reshape(Hq, D) / s[:, None]
    return m, s, o


def lse_merge(ms: np.ndarray, ss: np.ndarray, os_: np.ndarray) -> np.ndarray:
    """Merge partitions: M = max m_p, S = sum s_p e^(m_p-M),
    O = sum o_p s_p e^(m_p-M) / (S + 1e-6).  ms, ss [P, H]; os_ [P, H, D]."""
    M = ms.max(axis=0)
    w = ss * np.exp(ms - M[None, :])
    return np.einsum("ph,phd->hd", w, os_) / (w.sum(axis=0) + 1e-6)[:, None]


def paged_attention_split(q, key_cache, value_cache, block_tables, context_lens,
                          num_kv_heads: int, scale: float, block_size: int, max_seq_len: int,
                          partition_size: int, alibi_slopes=None, q_dtype: str = "float32",
                          cache_dtype: str = "float32") -> np.ndarray:
    """Split-K decode: partitions of ``partition_size`` tokens, LSE-merged.

    Same edge semantics as ``paged_attention``; equal to it up to float64
    rounding (the merge is an algebraic identity).
    """
    q64 = decode(q, q_dtype)
    kc64 = decode(key_cache, cache_dtype)
    vc64 = decode(value_cache, cache_dtype)
    B, Hq, D = q64.shape
    out = np.zeros((B, Hq, D), dtype=np.float64)
    lens = np.asarray(context_lens).astype(np.int64) & 0xFFFFFFFF
    for s in range(B):
        ctx = int(lens[s])
        if ctx == 0 or ctx > max_seq_len:
            continue
        k, v = gather_kv(kc64, vc64, block_tables[s], ctx)
        bias = None if alibi_slopes is None else alibi_bias(alibi_slopes, ctx)
        parts = [partition_stats(q64[s], k, v, scale, bias, lo, min(lo + partition_size, ctx))
                 for lo in range(0, ctx, partition_size)]
        out[s] = lse_merge(np.stack([p[0] for p in parts]), np.stack([p[1] for p in parts]),
                           np.stack([p[2] for p in parts]))
    return out


# ---------------------------------------------------------------------------
# Layout helpers for tests: token-major <-> paged 5-D
# ---------------------------------------------------------------------------


def token_major_to_paged5d(kt: np.ndarray, vt: np.ndarray, block_size: int, x: int):
    """[num_slots, H, D] (slot = block*bs + off) -> paged 5-D K and V."""
    S, H, D = kt.shape
    nb = S // block_size
    k5 = kt.reshape(nb, block_size, H, D // x, x).transpose(0, 2, 3, 1, 4).copy()
    v4 = vt.reshape(nb, block_size, H, D).transpose(0, 2, 3, 1).copy()
    return k5, v4


# ---------------------------------------------------------------------------
# Block copies (paged_attention/metal/cache/copy_blocks.metal:9-39, :55-70;
# mlx_cache.cpp:302-370): for every (src, dst) pair, block dst of the
# destination receives block src of the source, as bytes.  The reference runs
# the pairs concurrently, so a mapping whose sources and destinations overlap
# has no defined result; the restatement applies pairs in order and its tests
# use mappings without such overlaps.  Out-of-range pairs are skipped here (the
# reference does not check them).
# ---------------------------------------------------------------------------
def copy_blocks(key_caches, value_caches, block_mapping):
    """Per layer: K[dst] = K[src], V[dst] = V[src] (copy_blocks.metal:9-39)."""
    out_k, out_v = [], []
    m = np.asarray(block_mapping, dtype=np.int64).reshape(-1, 2)
    for kc, vc in zip(key_caches, value_caches):
        k, v = np.array(kc, copy=True), np.array(vc, copy=True)
        for s, d in m:
            if 0 <= s < k.shape[0] and 0 <= d < k.shape[0]:
                k[d] = kc[s]
                v[d] = vc[s]
        out_k.append(k)
        out_v.append(v)
    return out_k, out_v


def swap_blocks(src, dst, block_mapping):
    """dst[d] = src[s] for every pair (copy_blocks.metal:55-70)."""
    out = np.array(dst, copy=True)
    for s, d in np.asarray(block_mapping, dtype=np.int64).reshape(-1, 2):
        if 0 <= s < src.shape[0] and 0 <= d < out.shape[0]:
            out[d] = src[s]
    return out


# ---------------------------------------------------------------------------
# FP8 E4M3 (paged_attention/metal/float8.metal, convert_fp8.metal)
# ---------------------------------------------------------------------------


def fp8_e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """E4M3 codes -> float32 values (fp8_e4m3_to_float, float8.metal:13-38).

    Bias 7; exponent 0 is zero or subnormal (mantissa/8 * 2^-6); exponent 15
    is +-inf for mantissa 0 and NaN otherwise (not E4M3FN) -- the reference
    returns an unsigned NAN there whatever the sign bit (:29-30); the rest is
    (1 + mantissa/8) * 2^(exponent - 7).
    """
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    s = c >> 7
    e = (c >> 3) & 0xF
    m = c & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(np.minimum(e, 14) - 7.0))
    val = np.where(s == 1, -mag, mag).astype(np.float32)
    inf = np.where(s == 1, -np.inf, np.inf).astype(np.float32)
    nan = np.full(c.shape, 0x7FC00000, dtype=np.uint32).view(np.float32)
    return np.where(e == 15, np.where(m == 0, inf, nan), val).astype(np.float32)


def fp8_e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> E4M3 codes, detail::fp32_to_fp8<4, 3, 7> (float8.metal:72-120).

    Step by step as the reference:
    * |x| inf or NaN: exponent 15, mantissa (NaN ? 1 : 0) (:80-83).
    * Biased exponent e8 = e + 7 in [1, 14]: round the 23-bit mantissa to 3
      bits to nearest even (:91-97); a carry moves to e8 + 1, and past 14 the
      result is inf (:98-103).
    * Otherwise (e8 < 1 -- and also e8 > 14, which the reference lets fall
      through to this branch): e8 < -2 gives +-0 (:108-109); else the 24-bit
      significand is shifted right by (1 - e8) + 20 with round-half-up and
      only its low 3 bits are kept (:111-118).  So a value that rounds up to
      2^-6 encodes as +-0, and 256 <= |x| < 2^14 lands on small codes
      (256 -> +0).
    * From |x| >= 2^14 (e8 >= 21) the reference's shift counts leave [0, 31]
      (``1u << (rshift - 1)`` with rshift <= 0), which is undefined; this
      restatement defines the result there as +-inf, the value of the
      reference's own overflow branch.
    """
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.int64)
    s = (u >> 31) & 1
    a = u & 0x7FFFFFFF
    special = a >= 0x7F800000
    e8 = ((a >> 23) & 0xFF) - 127 + 7
    m = a & 0x7FFFFF
    # normal path
    shift = 20
    mant = m >> shift
    lsb = mant & 1
    rnd = (m >> (shift - 1)) & 1
    sticky = (m & ((1 << (shift - 1)) - 1)) != 0
    mant = mant + (rnd & (sticky | lsb))
    carry = (mant >> 3) != 0
    e_n = np.where(carry, e8 + 1, e8)
    mant_n = np.where(carry, 0, mant)
    normal_code = np.where(e_n > 14, (s << 7) | (15 << 3), (s << 7) | (e_n << 3) | (mant_n & 7))
    is_normal = (e8 >= 1) & (e8 <= 14)
    # subnormal / underflow path (also reached for e8 > 14)
    rshift = np.clip((1 - e8) + 20, 0, 63)
    full = 0x800000 | m
    rounded = (full + (np.int64(1) << np.maximum(rshift - 1, 0))) >> rshift
    sub_code = np.where((e8 < -2) | (rounded == 0), s << 7, (s << 7) | (rounded & 7))
    code = np.where(is_normal, normal_code, sub_code)
    code = np.where(e8 >= 21, (s << 7) | (15 << 3), code)
    code = np.where(special, (s << 7) | (15 << 3) | (a != 0x7F800000), code)
    return code.astype(np.uint8)


FP8 = "fp8_e4m3"


def convert_fp8(src: np.ndarray, src_dtype: str, dst_dtype: str, scale: float) -> np.ndarray:
    """convert_fp8_kernel<SRC_T, DST_T> (convert_fp8.metal:13-47), element-wise.

    ``src``/result are storage arrays (uint8 codes for ``FP8``, uint16 bits for
    float16/bfloat16, float32 values).  fp8 -> T: decode * scale (float32),
    then rounded to T; T -> fp8: encode(float(x) / scale); fp8 -> fp8:
    encode(decode * scale); T -> U: float(x) * scale rounded to U.  The
    reference instantiates the 16 pairs of convert_fp8.metal:58-80.
    """
    sc = np.float32(scale)
    if src_dtype == FP8:
        v = fp8_e4m3_decode(src) * sc
    else:
        v = decode(src, src_dtype).astype(np.float32)
        v = v / sc if dst_dtype == FP8 else v * sc
    v = np.asarray(v, dtype=np.float32)
    if dst_dtype == FP8:
        return fp8_e4m3_encode(v)
    return to_storage(v, dst_dtype)

