"""CPU baseline: torch-CPU restatement of the reference's gather + SDPA decode.

TEST INFRASTRUCTURE ONLY -- used by the ``cpu_baseline`` leg of bench.py
and by tests/test_cpu_baseline.py, which checks it against the float64
oracle.  Nothing in the product package imports it.

The reference decodes without its paged kernel: each layer scatters the new
token into the token-major MHATokenPool buffers, gathers every token of the
sequence back into a contiguous [1, Hkv, T, D] copy
(sglang_mlx/srt/mem_cache/memory_pool.py:139-159, called from
PooledKVCache.update_and_fetch, :206-234) and hands that copy to MLX's
scaled_dot_product_attention, one sequence at a time (the runner's batch is
1, sglang_mlx/model_runner.py:278).  tests/bench_paged_vs_gather.py:81-103
times the same gather + SDPA.  MLX is not installed (and has no ROCm
backend), so this restatement runs the same steps with torch on the host:

  1. slots of logical token t: block_table[t // bs] * bs + t % bs
     (token-major pool, slot = block * bs + offset);
  2. index_select those rows of the [num_slots, Hkv, D] K and V buffers,
     transpose to [1, Hkv, T, D];
  3. torch.nn.functional.scaled_dot_product_attention(q[1, Hq, 1, D], k, v,
     scale, enable_gqa=True).

tests/bench_paged_vs_gather.py:86-92 starts one step earlier: its gather
first relays the paged 5-D caches out as token-major [nb * bs, Hkv, D]
(a transpose + copy of the whole cache) and then indexes them.
gather_sdpa_decode_paged5d does the same, so that the relayout is inside
whatever is timed.

scatter_append_paged5d is the append (reshape_and_cache) restated the same
way: each token's K and V rows written in place into the paged 5-D caches
at block slot // bs, offset slot % bs, slots < 0 skipped
(reshape_and_cache.metal:35-69), with torch indexing on the host.

The 1e-6 in the reference kernel's softmax denominator is a kernel detail
(paged_attention_kernels.metal:144), absent from SDPA, so results differ
from the oracle by a relative 1e-6 plus SDPA's own rounding.
"""

from __future__ import annotations

import os
import time

import torch
import torch.nn.functional as F


def host_threads() -> int:
    """Threads the baseline may use: the process's CPU affinity, capped by
    OMP_NUM_THREADS when that is set (a shared host may set it to this job's
    CPU share)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def token_slots(block_row: torch.Tensor, ctx: int, block_size: int) -> torch.Tensor:
    """Pool slots of logical tokens 0..ctx-1 (int64)."""
    t = torch.arange(ctx, dtype=torch.int64)
    return block_row.to(torch.int64)[t // block_size] * block_size + t % block_size


def gather_sdpa_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                       block_tables: torch.Tensor, context_lens: torch.Tensor, block_size: int,
                       scale: float, seqs=None) -> torch.Tensor:
    """One decode layer, sequence by sequence, on CPU tensors.

    q [B, Hq, D]; k_pool / v_pool [num_slots, Hkv, D] (token-major);
    block_tables [B, max_blocks]; context_lens [B].  Returns [B, Hq, D] in
    q's dtype (rows of sequences outside ``seqs`` or with ctx 0 are zero).
    """
    B, Hq, D = q.shape
    out = torch.zeros_like(q)
    for s in (range(B) if seqs is None else seqs):
        ctx = int(context_lens[s])
        if ctx <= 0:
            continue
        idx = token_slots(block_tables[s], ctx, block_size)
        k = k_pool.index_select(0, idx).transpose(0, 1).unsqueeze(0)  # [1, Hkv, T, D]
        v = v_pool.index_select(0, idx).transpose(0, 1).unsqueeze(0)
        o = F.scaled_dot_product_attention(q[s].reshape(1, Hq, 1, D), k, v, scale=scale,
                                           enable_gqa=True)
        out[s] = o.reshape(Hq, D)
    return out


def paged5d_to_token_major(key_cache: torch.Tensor, value_cache: torch.Tensor):
    """The paged 5-D caches K [nb, Hkv, D/x, bs, x] and V [nb, Hkv, D, bs]
    as token-major [nb * bs, Hkv, D] copies (slot = block * bs + offset),
    the relayout of tests/bench_paged_vs_gather.py:86-92."""
    nb, hkv, dx, bs, x = key_cache.shape
    k = key_cache.permute(0, 3, 1, 2, 4).reshape(nb * bs, hkv, dx * x)
    v = value_cache.permute(0, 3, 1, 2).reshape(nb * bs, hkv, dx * x)
    return k, v


def gather_sdpa_decode_paged5d(q, key_cache, value_cache, block_tables, context_lens, block_size, scale,
                               seqs=None):
    """gather_sdpa_decode from the paged 5-D caches: relayout to token-major
    first, as the reference's benchmark does, then gather + SDPA."""
    k_pool, v_pool = paged5d_to_token_major(key_cache, value_cache)
    return gather_sdpa_decode(q, k_pool, v_pool, block_tables, context_lens, block_size, scale, seqs)


def scatter_append_paged5d(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                           value_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """In place: key / value [N, H, D] into key_cache [nb, H, D/x, bs, x] and
    value_cache [nb, H, D, bs] (same dtype), token i at slot_mapping[i]."""
    nb, H, dx, bs, x = key_cache.shape
    slots = slot_mapping.to(torch.int64)
    keep = slots >= 0
    s = slots[keep]
    blk, off = s // bs, s % bs
    k = key[keep].reshape(-1, H, dx, x)
    v = value[keep]
    key_cache.permute(0, 3, 1, 2, 4)[blk, off] = k      # [n, H, D/x, x] at (block, offset)
    value_cache.permute(0, 3, 1, 2)[blk, off] = v       # [n, H, D] at (block, offset)


def time_calls(fn, budget_s: float = 1.0, min_iters: int = 5) -> dict:
    """Median wall time of fn() over >= min_iters runs (after one warm-up),
    stopping once ``budget_s`` of timed work is done, on host_threads()
    threads."""
    threads = host_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        fn()
        times = []
        t_all = time.perf_counter()
        while len(times) < min_iters or time.perf_counter() - t_all < budget_s:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
            if len(times) >= 10000:
                break
        times.sort()
        return dict(median_s=times[len(times) // 2], iters=len(times), threads=threads, cpu=cpu_model())
    finally:
        torch.set_num_threads(prev)


def time_decode(q, k_pool, v_pool, block_tables, context_lens, block_size, scale,
                budget_s: float = 10.0, min_iters: int = 5, seqs=None, fn=None) -> dict:
    """Median wall time of ``fn`` (gather_sdpa_decode by default; its
    k_pool / v_pool are then token-major pools, for
    gather_sdpa_decode_paged5d the paged 5-D caches) over >= min_iters runs
    (after one warm-up), stopping once ``budget_s`` of timed work is done."""
    fn = fn or gather_sdpa_decode
    threads = host_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        fn(q, k_pool, v_pool, block_tables, context_lens, block_size, scale, seqs)
        times = []
        t_all = time.perf_counter()
        while len(times) < min_iters or time.perf_counter() - t_all < budget_s:
            t0 = time.perf_counter()
            fn(q, k_pool, v_pool, block_tables, context_lens, block_size, scale, seqs)
            times.append(time.perf_counter() - t0)
            if len(times) >= 1000:
                break
        times.sort()
        return dict(median_s=times[len(times) // 2], iters=len(times), threads=threads,
                    cpu=cpu_model())
    finally:
        torch.set_num_threads(prev)
