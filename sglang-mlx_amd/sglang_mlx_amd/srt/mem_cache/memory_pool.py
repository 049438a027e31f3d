"""KV memory pool: slot allocator, per-layer K/V buffers in HBM and the
per-request cache adapter (sglang_mlx/srt/mem_cache/memory_pool.py:27-269).

* TokenPoolAllocator -- LIFO free stack of slot ids 1..pool_size (slot 0
  is the padding slot and is never handed out).  A fresh pool hands out
  descending runs: alloc(3) on a pool of 10 returns [3, 2, 1]; freed slots
  are reused first (memory_pool.py:27-68).
* MHATokenPool -- one device allocation per K and V holding every layer,
  [num_layers, pool_size + 1, Hkv, D]; ``k_buffer[l]`` / ``v_buffer[l]`` are
  the per-layer [pool_size + 1, Hkv, D] views of memory_pool.py:102-108.
  ``store`` scatters new tokens with the HIP append kernel (token-major
  layout, one 16-byte vector per lane); ``fetch`` gathers slots back into
  [1, Hkv, T, D].
* PooledKVCache -- the per-request, per-layer adapter with the mlx-lm cache
  protocol (set_indices / offset / update_and_fetch / state / make_mask).
* Decode without the gather (the TODOs of memory_pool.py:110-115 and
  :175-177): ``MHATokenPool.decode`` runs the paged decode kernel on the
  pool's token rows with one slot table row per request (block size 1), and
  ``decode_batch`` does so for a batch of PooledKVCache views.
"""

from __future__ import annotations

import numpy as np
import torch

from ... import _ext


class TokenPoolAllocator:
    """Free list of pool slots.  Slot 0 is reserved padding."""

    def __init__(self, pool_size: int):
        if pool_size <= 0:
            raise ValueError(f"pool_size must be positive, got {pool_size}")
        self._pool_size = pool_size
        self.clear()

    def clear(self) -> None:
        """Every slot free again, in the initial order."""
        self._stack = np.arange(self._pool_size, 0, -1, dtype=np.int64)
        self._top = self._pool_size

    def alloc(self, n: int) -> list[int]:
        """The ``n`` most recently freed slots (a fresh pool: n, n-1, ..., 1),
        in stack order.  MemoryError if fewer than ``n`` are free."""
        if n <= 0:
            return []
        if n > self._top:
            raise MemoryError(f"Cannot allocate {n} slots: only {self._top} available")
        out = self._stack[self._top - n:self._top].tolist()
        self._top -= n
        return out

    def free(self, indices) -> None:
        """Push slots back; the next alloc returns the last of them first."""
        idx = np.asarray(list(indices), dtype=np.int64)
        end = self._top + idx.size
        if end > self._stack.size:
            grown = np.empty(max(end, 2 * self._stack.size), dtype=np.int64)
            grown[:self._top] = self._stack[:self._top]
            self._stack = grown
        self._stack[self._top:end] = idx
        self._top = end

    @property
    def available_size(self) -> int:
        return self._top


class MHATokenPool:
    """Pre-allocated K/V buffers for all layers, token-major."""

    def __init__(self, pool_size: int, num_layers: int, n_kv_heads: int, head_dim: int,
                 dtype: torch.dtype = torch.float16, device="cuda"):
        self.pool_size = pool_size
        self.num_layers = num_layers
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = torch.device(device)
        shape = (num_layers, pool_size + 1, n_kv_heads, head_dim)
        self._k = torch.zeros(shape, dtype=dtype, device=self.device)
        self._v = torch.zeros(shape, dtype=dtype, device=self.device)
        self.k_buffer = [self._k[i] for i in range(num_layers)]
        self.v_buffer = [self._v[i] for i in range(num_layers)]

    def _slots(self, indices) -> torch.Tensor:
        if isinstance(indices, torch.Tensor):
            return indices.to(device=self.device, dtype=torch.int32)
        return torch.tensor(list(indices), dtype=torch.int32, device=self.device)

    def store(self, layer_idx: int, indices, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Write ``keys`` / ``values`` of shape [1, Hkv, S, D] (mlx-lm order)
        into slots ``indices`` (length S) of layer ``layer_idx``."""
        k = keys[0].transpose(0, 1)   # [S, Hkv, D]
        v = values[0].transpose(0, 1)
        if k.shape[0] == 0:
            return
        _ext.reshape_and_cache(k.to(self.dtype) if k.dtype not in (self.dtype, torch.float32) else k,
                               v.to(self.dtype) if v.dtype not in (self.dtype, torch.float32) else v,
                               self.k_buffer[layer_idx], self.v_buffer[layer_idx], self._slots(indices))

    def fetch(self, layer_idx: int, indices) -> tuple[torch.Tensor, torch.Tensor]:
        """Gather slots ``indices`` of layer ``layer_idx`` as [1, Hkv, T, D]."""
        idx = self._slots(indices).to(torch.int64)
        k = self.k_buffer[layer_idx].index_select(0, idx).transpose(0, 1).unsqueeze(0)
        v = self.v_buffer[layer_idx].index_select(0, idx).transpose(0, 1).unsqueeze(0)
        return k, v

    def decode(self, layer_idx: int, q: torch.Tensor, slot_lists, scale: float,
               alibi_slopes: torch.Tensor | None = None) -> torch.Tensor:
        """Decode attention of one query token per request over layer
        ``layer_idx``: q [B, Hq, D]; slot_lists[i] lists request i's context
        slots in order.  Returns [B, Hq, D] like q.  The kernel reads the
        token rows in place (slot tables, block size 1); nothing is
        gathered."""
        B = q.shape[0]
        if len(slot_lists) != B:
            raise ValueError("one slot list per query row is required")
        width = max((len(s) for s in slot_lists), default=0) or 1
        table = np.full((B, width), -1, dtype=np.int32)
        lens = np.zeros(B, dtype=np.int32)
        for i, slots in enumerate(slot_lists):
            table[i, :len(slots)] = np.asarray(list(slots), dtype=np.int32)
            lens[i] = len(slots)
        bt = torch.from_numpy(table).to(self.device, non_blocking=True)
        ctx = torch.from_numpy(lens).to(self.device, non_blocking=True)
        return _ext.paged_attention_v1(q, self.k_buffer[layer_idx], self.v_buffer[layer_idx], bt, ctx,
                                       self.n_kv_heads, scale, 1, width, alibi_slopes)


class PooledKVCache:
    """One request's view of one layer of the pool (mlx-lm cache protocol)."""

    def __init__(self, pool: MHATokenPool, layer_idx: int):
        self._pool = pool
        self._layer_idx = layer_idx
        self._prefix_indices: list[int] = []
        self._new_indices: list[int] = []
        self._store_offset = 0

    def set_indices(self, prefix_indices, new_indices) -> None:
        """Slots already holding this request's prefix, and slots reserved
        for the tokens the next forward passes compute."""
        self._prefix_indices = list(prefix_indices)
        self._new_indices = list(new_indices)
        self._store_offset = 0

    @property
    def offset(self) -> int:
        """Position of the first new token (its RoPE offset)."""
        return len(self._prefix_indices)

    def _live(self) -> list[int]:
        return self._prefix_indices + self._new_indices[:self._store_offset]

    @property
    def slot_indices(self) -> list[int]:
        """Slots of every token of the request so far (prefix, then stored)."""
        return self._live()

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Store the next keys.shape[2] new tokens, then return every token of
        the request so far as [1, Hkv, T, D]."""
        n = keys.shape[2]
        dest = self._new_indices[self._store_offset:self._store_offset + n]
        self._store_offset += n
        self._pool.store(self._layer_idx, dest, keys, values)
        return self._pool.fetch(self._layer_idx, self._live())

    @property
    def state(self):
        live = self._live()
        if not live:
            return None, None
        return self._pool.fetch(self._layer_idx, live)

    def make_mask(self, N: int, return_array: bool = False, window_size: int | None = None):
        """Attention mask for N new queries after ``offset`` cached tokens:
        None for a single query; a boolean [N, offset + N] tensor (query i
        sees key j iff j <= offset + i and, with a window w,
        j > offset + i - w) when ``return_array`` is set or the window cuts
        into the keys; "causal" otherwise.  The cases the reference's tests
        fix (tests/test_memory_pool.py:276-343) are reproduced; which of
        "causal" and an all-causal array mlx-lm returns for a window that
        cuts nothing is not fixed by them."""
        if N == 1:
            return None
        if not return_array and (window_size is None or self.offset + N <= window_size):
            return "causal"
        q = torch.arange(self.offset, self.offset + N).unsqueeze(1)
        k = torch.arange(self.offset + N).unsqueeze(0)
        mask = k <= q
        if window_size is not None:
            mask &= k > q - window_size
        return mask


def decode_batch(caches: list[PooledKVCache], q: torch.Tensor, scale: float,
                 alibi_slopes: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention for a batch of requests that share one pool layer:
    row i of q [B, Hq, D] attends over every token caches[i] holds (call it
    after the step's update_and_fetch / store).  Continuous batching without
    the per-request gather (memory_pool.py:175-177)."""
    if not caches:
        raise ValueError("decode_batch needs at least one cache")
    pool, layer = caches[0]._pool, caches[0]._layer_idx
    if any(c._pool is not pool or c._layer_idx != layer for c in caches):
        raise ValueError("decode_batch caches must view the same pool layer")
    return pool.decode(layer, q, [c.slot_indices for c in caches], scale, alibi_slopes)
