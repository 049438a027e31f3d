"""Paged-attention kernel API for MI355X -- drop-in for the reference's
``sglang_mlx.metal_kernels`` (metal_kernels.py:1-96) over PyTorch-ROCm
tensors.

Operations:
    paged_attention_v1   single-softmax paged decode attention
    paged_attention_v2   split-K paged decode with a log-sum-exp merge
    paged_attention_cascade  decode with radix-shared prefixes computed once
                         per group of sequences (a host-built plan)
    reshape_and_cache    scatter new KV tokens into the cache (in place)
    copy_blocks          block copies inside the caches
    swap_blocks          block copies between two buffers
    convert_fp8          element-wise conversion with a scale, FP8 E4M3 codes
                         as uint8 tensors

Tensors live on a HIP device; kernels run asynchronously on the current
stream of that device.
"""

from __future__ import annotations

import torch

from . import _ext


def paged_attention_v1(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    num_kv_heads: int,
    scale: float,
    block_size: int,
    max_seq_len: int,
    alibi_slopes: torch.Tensor | None = None,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> torch.Tensor:
    """Single-pass paged attention (metal_kernels.py:20-61).

    Args:
        query: [num_seqs, num_heads, head_size]
        key_cache: [num_blocks, num_kv_heads, head_size/x, block_size, x]
        value_cache: [num_blocks, num_kv_heads, head_size, block_size]
        block_tables: [num_seqs, max_num_blocks_per_seq] (32-bit ids)
        context_lens: [num_seqs]
        num_kv_heads: Number of KV heads
        scale: Attention scaling factor
        block_size: Number of tokens per block
        max_seq_len: Maximum sequence length
        alibi_slopes: Optional ALiBi slopes [num_heads]
        k_scale, v_scale: for uint8 (FP8 E4M3) caches, K = decode(code) *
            k_scale and V = decode(code) * v_scale; ignored otherwise

    Returns:
        Output tensor [num_seqs, num_heads, head_size], dtype of query.
    """
    return _ext.paged_attention_v1(query, key_cache, value_cache, block_tables, context_lens,
                                   num_kv_heads, scale, block_size, max_seq_len, alibi_slopes, k_scale, v_scale)


def paged_attention_v2(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    num_kv_heads: int,
    scale: float,
    block_size: int,
    max_seq_len: int,
    alibi_slopes: torch.Tensor | None = None,
    partition_size: int = 512,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> torch.Tensor:
    """Split-K paged attention for long contexts: each partition of
    ``partition_size`` tokens yields (max, sum, output); partitions are merged
    by log-sum-exp.  Same arguments and result as ``paged_attention_v1``."""
    return _ext.paged_attention_v2(query, key_cache, value_cache, block_tables, context_lens,
                                   num_kv_heads, scale, block_size, max_seq_len, alibi_slopes,
                                   partition_size, k_scale, v_scale)


def paged_attention_cascade(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    num_kv_heads: int,
    scale: float,
    block_size: int,
    max_seq_len: int,
    plan,
    alibi_slopes: torch.Tensor | None = None,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> torch.Tensor:
    """Paged attention with radix-shared prefixes computed once per group of
    sequences (``plan``: srt.mem_cache.build_cascade_plan over the same block
    tables).  Same arguments and result as ``paged_attention_v1`` (paged 5-D
    caches), to within floating-point rounding."""
    return _ext.paged_attention_cascade(query, key_cache, value_cache, block_tables, context_lens, num_kv_heads,
                                        scale, block_size, max_seq_len, plan, alibi_slopes, k_scale, v_scale)


def reshape_and_cache(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> list[torch.Tensor]:
    """Scatter-write new KV tokens into the cache (metal_kernels.py:64-74).

    key/value: [num_tokens, num_kv_heads, head_size]; slot_mapping:
    [num_tokens], -1 = padding (skipped).  The caches are updated in place
    and returned as [key_cache, value_cache].  Paged 5-D caches and 3-D
    MHATokenPool buffers [num_slots, num_kv_heads, head_size] are accepted.
    uint8 caches hold FP8 E4M3 codes (the reference's format) of
    key / k_scale and value / v_scale; the paged layout then has x = 16.
    """
    return _ext.reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, k_scale, v_scale)


def copy_blocks(
    key_caches: list[torch.Tensor],
    value_caches: list[torch.Tensor],
    block_mapping: torch.Tensor,
) -> tuple[list[torch.Tensor], list[torch.Tensor]]:
    """Copy blocks within the caches (metal_kernels.py:77-85)."""
    return _ext.copy_blocks(key_caches, value_caches, block_mapping)


def swap_blocks(src: torch.Tensor, dst: torch.Tensor, block_mapping: torch.Tensor) -> torch.Tensor:
    """Blit blocks between two buffers (metal_kernels.py:88-96)."""
    return _ext.swap_blocks(src, dst, block_mapping)


def convert_fp8(dst: torch.Tensor, src: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """Element-wise precision conversion with a scale (the reference's
    convert_fp8_kernel, convert_fp8.metal:13-80).  uint8 tensors hold FP8
    E4M3 codes in the reference's format (bias 7, exponent 15 = inf / NaN).
    fp8 -> T: decode * scale; T -> fp8: encode(x / scale); fp8 -> fp8:
    encode(decode * scale); T -> U: x * scale.  dst is written in place and
    returned."""
    return _ext.convert_fp8(dst, src, scale)

