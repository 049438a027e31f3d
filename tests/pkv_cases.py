"""Seeded input generators shared by the tests, the golden-fixture script,
smoke() and bench.py.

All inputs are drawn with numpy.random.default_rng(seed) (PCG64) as float32
N(0, 1) and rounded to the storage dtype with the oracle's converters, so the
same seed gives the same bits everywhere.  Arrays are NumPy storage arrays:
uint16 bit patterns for float16/bfloat16, float32 otherwise.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from oracle import pagedkv_oracle as orc

X_OF = {"float32": 4, "float16": 8, "bfloat16": 8}


@dataclass
class DecodeCase:
    q: np.ndarray                 # [B, Hq, D] storage of q_dtype
    k_cache: np.ndarray           # [nb, Hkv, D/x, bs, x]
    v_cache: np.ndarray           # [nb, Hkv, D, bs]
    block_tables: np.ndarray      # [B, max_blocks] int32 (-1 past the context)
    context_lens: np.ndarray      # [B] int32
    num_kv_heads: int
    scale: float
    block_size: int
    max_seq_len: int
    q_dtype: str
    cache_dtype: str
    alibi: np.ndarray | None = None
    meta: dict = field(default_factory=dict)


def normal(rng, shape, dtype: str) -> np.ndarray:
    return orc.to_storage(rng.standard_normal(shape, dtype=np.float32), dtype)


def make_decode_case(seed: int, B: int, Hq: int, Hkv: int, D: int, block_size: int,
                     ctx_lo: int, ctx_hi: int, cache_dtype: str = "bfloat16",
                     q_dtype: str | None = None, pool_factor: float = 1.1,
                     num_blocks: int | None = None, shared_prefix_blocks: int = 0,
                     max_seq_len: int | None = None, alibi: bool = False,
                     context_lens=None, max_blocks: int | None = None) -> DecodeCase:
    """Random paged decode input.

    Block 0 is the padding block and never appears in a table.  Private
    blocks are a seeded permutation of the pool (no block in two tables);
    with ``shared_prefix_blocks`` every table starts with the same ids.
    """
    q_dtype = q_dtype or cache_dtype
    rng = np.random.default_rng(seed)
    if context_lens is None:
        ctx = rng.integers(ctx_lo, ctx_hi + 1, size=B).astype(np.int64)
    else:
        ctx = np.asarray(context_lens, dtype=np.int64)
    nblk = -(-ctx // block_size)
    shared = shared_prefix_blocks
    private = np.maximum(nblk - shared, 0)
    need = int(private.sum()) + shared
    nb = num_blocks or (int(math.ceil(need * pool_factor)) + 1)
    assert nb >= need + 1, "pool too small"
    perm = rng.permutation(np.arange(1, nb))
    shared_ids = perm[:shared]
    priv_ids = perm[shared:shared + int(private.sum())]
    msl = max_seq_len if max_seq_len is not None else int(max(1, ctx.max()))
    mb = max_blocks or int(max(1, nblk.max(), -(-msl // block_size)))
    bt = np.full((B, mb), -1, dtype=np.int32)
    pos = 0
    for s in range(B):
        row = np.concatenate([shared_ids[:min(shared, nblk[s])], priv_ids[pos:pos + private[s]]])
        pos += private[s]
        bt[s, :len(row)] = row
    x = X_OF[cache_dtype]
    kc = normal(rng, (nb, Hkv, D // x, block_size, x), cache_dtype)
    vc = normal(rng, (nb, Hkv, D, block_size), cache_dtype)
    q = normal(rng, (B, Hq, D), q_dtype)
    slopes = None
    if alibi:
        slopes = (2.0 ** (-8.0 * np.arange(1, Hq + 1) / Hq)).astype(np.float32)
    return DecodeCase(q, kc, vc, bt, ctx.astype(np.int32), Hkv, 1.0 / math.sqrt(D), block_size, msl,
                      q_dtype, cache_dtype, slopes,
                      meta=dict(seed=seed, B=B, Hq=Hq, Hkv=Hkv, D=D, nb=nb))


def decode_oracle(c: DecodeCase, partition_size: int = 0) -> np.ndarray:
    if partition_size:
        return orc.paged_attention_split(c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens,
                                         c.num_kv_heads, c.scale, c.block_size, c.max_seq_len,
                                         partition_size, c.alibi, c.q_dtype, c.cache_dtype)
    return orc.paged_attention(c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens,
                               c.num_kv_heads, c.scale, c.block_size, c.max_seq_len, c.alibi,
                               c.q_dtype, c.cache_dtype)


@dataclass
class AppendCase:
    key: np.ndarray               # [N, H, D] storage of kv_dtype
    value: np.ndarray
    slot_mapping: np.ndarray      # [N] int32, -1 = padding
    num_slots: int
    block_size: int
    kv_dtype: str
    cache_dtype: str


def make_append_case(seed: int, N: int, H: int, D: int, num_slots: int, block_size: int,
                     kv_dtype: str = "bfloat16", cache_dtype: str | None = None,
                     pad_frac: float = 0.05, reserve_slot0: bool = True) -> AppendCase:
    """Unique random slots (slot 0 reserved as padding), ``pad_frac`` of the
    tokens set to -1."""
    cache_dtype = cache_dtype or kv_dtype
    rng = np.random.default_rng(seed)
    lo = 1 if reserve_slot0 else 0
    slots = rng.choice(num_slots - lo, size=N, replace=False).astype(np.int64) + lo
    npad = int(round(pad_frac * N))
    if npad:
        slots[rng.choice(N, size=npad, replace=False)] = -1
    key = normal(rng, (N, H, D), kv_dtype)
    value = normal(rng, (N, H, D), kv_dtype)
    return AppendCase(key, value, slots.astype(np.int32), num_slots, block_size, kv_dtype, cache_dtype)


def run_slots(rng, N: int, num_blocks: int, block_size: int, pad_frac: float = 0.03) -> np.ndarray:
    """N unique slots laid out as a prefill and its neighbours write them:
    blocks in a shuffled order, each taken whole (a run of block_size
    consecutive slots, half the blocks), as a run over part of the block
    (a quarter) or as one slot (a quarter); then pad_frac of the tokens set
    to -1.  Needs num_blocks large enough to hold N tokens (~10 per block)."""
    slots: list[int] = []
    for b in rng.permutation(num_blocks):
        if len(slots) >= N:
            break
        kind = int(rng.integers(0, 4))
        base = int(b) * block_size
        if kind < 2:
            slots.extend(range(base, base + block_size))
        elif kind == 2:
            lo = int(rng.integers(0, block_size))
            slots.extend(range(base + lo, base + int(rng.integers(lo + 1, block_size + 1))))
        else:
            slots.append(base + int(rng.integers(0, block_size)))
    if len(slots) < N:
        raise ValueError("too few blocks for N tokens")
    out = np.asarray(slots[:N], dtype=np.int64)
    npad = int(round(pad_frac * N))
    if npad:
        out[rng.choice(N, size=npad, replace=False)] = -1
    return out.astype(np.int32)


def make_run_append_case(seed: int, N: int, H: int, D: int, num_blocks: int, block_size: int,
                         kv_dtype: str = "bfloat16", cache_dtype: str | None = None) -> AppendCase:
    """An append whose slots come in runs (run_slots)."""
    cache_dtype = cache_dtype or kv_dtype
    rng = np.random.default_rng(seed)
    slots = run_slots(rng, N, num_blocks, block_size)
    key = normal(rng, (N, H, D), kv_dtype)
    value = normal(rng, (N, H, D), kv_dtype)
    return AppendCase(key, value, slots, num_blocks * block_size, block_size, kv_dtype, cache_dtype)


def tolerance(q_dtype: str, cache_dtype: str) -> tuple[float, float]:
    """(atol, rtol) of the attention outputs: 2e-3/1e-2 for float16,
    1e-2/2e-2 for bfloat16 (the coarser of query and cache type decides)."""
    if "bfloat16" in (q_dtype, cache_dtype):
        return 1e-2, 2e-2
    return 2e-3, 1e-2
