#!/usr/bin/env python3
"""Benchmark of the MI355X paged-KV hot path (one GPU).

Default workload: one paged decode-attention layer at Llama-3-8B shape --
64 sequences, 32 query heads over 8 KV heads (GQA 4), head_dim 128,
block_size 16, context lengths uniform in [512, 4096], bf16 query and KV,
block tables a seeded random permutation over a pool of 1.1x the blocks
needed (block 0 is the padding block).  One step = one
``paged_attention_v1`` call over the batch.  Independent per-layer KV pools
(4 by default, 2.7 GB in all) are used in turn, as consecutive layers of a
model would be, so neither L2 nor the 256 MiB Infinity Cache serves a step
from the previous one.

Printed: ONE JSON line with the driver's fields plus
  roofline      the decode kernel's algorithmic HBM bytes per launch divided
                by its mean launch time (a HIP event pair around the timed
                region's back-to-back launches, on the stream the kernels
                run on, divided by the steps), against the 8 TB/s peak;
                ``traffic`` is the measured HBM bytes per launch from the
                committed rocprofv3 counter summary when present;
  append        the slot-mapped append at 4096 tokens / 8 KV heads / D 128 /
                bf16 into 65,536 slots with 5% padding, timed as a HIP graph
                of back-to-back launches over rotating sources and pools, for
                the token-major (MHATokenPool) and paged 5-D layouts;
  split_k       long-context decode (Qwen2-7B shape, B 1 and 4, contexts of
                32K/64K/128K tokens) through paged_attention_v1 and
                paged_attention_v2 with 512-token partitions, HIP graphs;
  radix_shared  256 sequences sharing a 2048-token prefix (128 blocks) plus
                64..512 private tokens, with 10% private-block churn through
                the block allocator and the append kernel between steps;
                bandwidth over unique bytes (prefix once) and logical bytes;
  radix_shared_fp8  the same over FP8 E4M3 caches (appends quantise with
                k_scale / v_scale);
  token_rows    the decode layer on token-row caches: MHATokenPool's
                [rows, Hkv, D] buffer through slot tables (block size 1) and
                the flash layout [blocks, 16, Hkv, D];
  fp8_kv        the decode layer over FP8 E4M3 caches (half the KV bytes);
  batch_sweep   the decode layer at batch 8 .. 128;
  ref_decode_b1 the reference's own decode benchmark (batch 1, fp16, seq
                1024 / 4096 / 8192), with its CPU gather + SDPA beside it;
  ref_append    the reference's own append benchmark (fp16, N = 1 .. 1024
                tokens), with a CPU scatter beside it;
  cpu_baseline  the reference's gather + SDPA decode restated in torch on
                this host's cores, on the same inputs (full batch, one layer).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-append] [--no-splitk] [--no-radix]
                       [--no-rows] [--no-fp8] [--no-sweep] [--no-ref] [--only LEG]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sglang-mlx_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

METRIC = "paged decode µs/step + HBM GB/s (% peak), bs64 ctx≤4k Llama-3-8B shape"
PEAK_GBS = 8000.0  # MI355X HBM3E, published peak
DECODE_KERNEL = "paged_decode_persist_kernel<BF16, BF16, 128, 16>"
APPEND_KERNEL = "rac_token_major_wave_kernel<BF16, BF16, 2>"


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=4, help="independent KV pools used in turn")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-append", action="store_true", help="skip the append measurement")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of timed CPU baseline work")
    ap.add_argument("--no-splitk", action="store_true", help="skip the long-context split-K measurement")
    ap.add_argument("--no-radix", action="store_true", help="skip the radix-shared decode measurement")
    ap.add_argument("--no-rows", action="store_true", help="skip the token-row (MHATokenPool) decode measurement")
    ap.add_argument("--no-fp8", action="store_true", help="skip the FP8-cache decode measurement")
    ap.add_argument("--no-sweep", action="store_true", help="skip the batch-size sweep of the decode layer")
    ap.add_argument("--no-ref", action="store_true",
                    help="skip the reference's own benchmark configurations (B1 fp16 decode, fp16 append counts)")
    ap.add_argument("--lib", help="load libpagedkv_gfx950.so from this path instead of the package's (a build of the "
                                  "same sources with other compile-time settings, e.g. make EXTRA_HIPFLAGS=... "
                                  "OUTDIR=...), for A/B profiles")
    ap.add_argument("--only", choices=["decode", "append", "copy", "splitk", "radix", "radix_fp8", "rows", "fp8", "sweep",
                                       "ref_decode", "ref_append"],
                    help="run one leg and print its own short JSON line (for counter collection under "
                         "rocprofv3 --pmc): the decode layer, the token-major append, or a plain 1 GiB device "
                         "copy whose FETCH_SIZE / WRITE_SIZE calibrate the counters")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# Inputs
# ---------------------------------------------------------------------------


def decode_inputs(seed: int, B: int, Hq: int, Hkv: int, D: int, bs: int, ctx_lo: int, ctx_hi: int,
                  layers: int, dev):
    """Seeded decode-layer inputs generated on the device."""
    rng = np.random.default_rng(seed)
    ctx = rng.integers(ctx_lo, ctx_hi + 1, size=B).astype(np.int64)
    nblk = -(-ctx // bs)
    need = int(nblk.sum())
    nb = int(math.ceil(need * 1.1)) + 1
    perm = rng.permutation(np.arange(1, nb))
    max_blocks = -(-ctx_hi // bs)
    bt = np.full((B, max_blocks), -1, dtype=np.int32)
    pos = 0
    for s in range(B):
        bt[s, :nblk[s]] = perm[pos:pos + nblk[s]]
        pos += nblk[s]
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn((B, Hq, D), generator=g, device=dev).to(torch.bfloat16)
    pools = []
    for _ in range(layers):
        kc = torch.randn((nb, Hkv, D // 8, bs, 8), generator=g, device=dev).to(torch.bfloat16)
        vc = torch.randn((nb, Hkv, D, bs), generator=g, device=dev).to(torch.bfloat16)
        pools.append((kc, vc))
    return dict(q=q, pools=pools, bt=torch.from_numpy(bt).to(dev), ctx=torch.from_numpy(ctx.astype(np.int32)).to(dev),
                ctx_np=ctx, nb=nb, B=B, Hq=Hq, Hkv=Hkv, D=D, bs=bs, max_seq_len=ctx_hi)


def decode_bytes(ctx: np.ndarray, B: int, Hq: int, Hkv: int, D: int, bs: int, s_kv=2, s_q=2, s_o=2) -> int:
    """Algorithmic HBM bytes of one decode launch: every context token's K and
    V read once per KV head, the queries read and outputs written once, the
    used block-table entries and context lengths read once."""
    return int(ctx.sum() * Hkv * D * 2 * s_kv + B * Hq * D * (s_q + s_o) + (-(-ctx // bs)).sum() * 4 + B * 4)


# ---------------------------------------------------------------------------
# Timing helpers
# ---------------------------------------------------------------------------


def timed_launches(fn, steps: int, warmup: int):
    """Run fn(i) warmup times, then the timed region: steps back-to-back
    calls between a synchronize and a HIP event pair on the current stream
    (the stream the kernels run on) at each end.  Returns (wall seconds,
    event-timed seconds) of the timed region."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a.record()
    for i in range(steps):
        fn(i)
    b.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, a.elapsed_time(b) * 1e-3


_SLEEP_CYCLES_PER_US = None


def queue_ahead(us: float = 80.0):
    """Queue about `us` microseconds of GPU spinning (torch.cuda._sleep) so that
    an event recorded next fires only after the host has also queued the
    launch that follows it: a single launch's event window then holds the
    kernel, not the host's argument checks and launch call."""
    global _SLEEP_CYCLES_PER_US
    if _SLEEP_CYCLES_PER_US is None:
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        torch.cuda._sleep(1_000_000)
        b.record()
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_US = 1_000_000 / max(a.elapsed_time(b) * 1e3, 1.0)
    torch.cuda._sleep(int(us * _SLEEP_CYCLES_PER_US))


def per_launch_ms(fn, launches: int, offset: int = 0):
    """Device time of single launches: a HIP event pair around each of
    `launches` calls, each queued behind a GPU spin (queue_ahead) so that the
    window holds the kernel alone."""
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(launches)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(launches)]
    torch.cuda.synchronize()
    for i in range(launches):
        queue_ahead()
        starts[i].record()
        fn(offset + i)
        ends[i].record()
    torch.cuda.synchronize()
    return sorted(s.elapsed_time(e) for s, e in zip(starts, ends))


def graph_launch_ms(fn, launches: int, replays: int = 5):
    """Mean device time of one launch: capture `launches` calls fn(i) in one
    HIP graph, replay it and divide the event-timed replay by `launches`."""
    for i in range(3):
        fn(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(launches):
            fn(i)
    graph.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(replays):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        torch.cuda.synchronize()
        per.append(a.elapsed_time(b) / launches)
    per.sort()
    return per[len(per) // 2]


def read_traffic(name: str):
    """(HBM bytes per launch, kernel average in us) from a committed
    rocprofv3 counter summary (profiles/<name>: lines
    'traffic_bytes_per_launch: <int>' and 'kernel_avg_us: <float>'), else
    (None, None)."""
    path = os.path.join(ROOT, "profiles", name)
    traffic = avg = None
    try:
        with open(path) as f:
            for line in f:
                m = re.match(r"\s*traffic_bytes_per_launch:\s*([0-9.eE+]+)", line)
                if m:
                    traffic = int(float(m.group(1)))
                m = re.match(r"\s*kernel_avg_us:\s*([0-9.eE+]+)", line)
                if m:
                    avg = float(m.group(1))
    except OSError:
        pass
    return traffic, avg


# ---------------------------------------------------------------------------
# Legs
# ---------------------------------------------------------------------------


def bench_decode(args, dev, kernels):
    inp = decode_inputs(1003, B=64, Hq=32, Hkv=8, D=128, bs=16, ctx_lo=512, ctx_hi=4096,
                        layers=args.layers, dev=dev)
    B, Hq, Hkv, D, bs = inp["B"], inp["Hq"], inp["Hkv"], inp["D"], inp["bs"]
    scale = 1.0 / math.sqrt(D)
    outs = [None] * len(inp["pools"])

    def step(i):
        li = i % len(inp["pools"])
        kc, vc = inp["pools"][li]
        outs[li] = kernels.paged_attention_v1(inp["q"], kc, vc, inp["bt"], inp["ctx"], Hkv, scale, bs,
                                              inp["max_seq_len"])

    wall, dev_s = timed_launches(step, args.steps, args.warmup)
    nbytes = decode_bytes(inp["ctx_np"], B, Hq, Hkv, D, bs)
    ms_step = wall * 1e3 / args.steps
    mean_ms = dev_s * 1e3 / args.steps  # back-to-back launches: kernel time plus launch gaps
    achieved = nbytes / (mean_ms * 1e-3) / 1e9
    single = per_launch_ms(step, min(args.steps, 40))
    res = dict(inp=inp, scale=scale, out0=outs[0], nbytes=nbytes, ms_step=ms_step, mean_ms=mean_ms,
               median_single_ms=single[len(single) // 2], achieved=achieved)
    return res


def bench_rows(dev, kernels, layers: int = 4, steps: int = 100, warmup: int = 10):
    """The Llama-3-8B decode layer of bench_decode (same sequences and context
    lengths) on token-row caches: MHATokenPool's [rows, 8, 128] buffer read
    through one slot per token (block size 1; slots a seeded permutation of a
    pool of 1.1x the tokens), and the flash layout [blocks, 16, 8, 128] through
    the same block tables shape as the paged leg.  Layer pools rotated."""
    B, Hq, Hkv, D = 64, 32, 8, 128
    rng = np.random.default_rng(1003)
    ctx = rng.integers(512, 4096 + 1, size=B).astype(np.int64)
    g = torch.Generator(device=dev)
    g.manual_seed(1003)
    q = torch.randn((B, Hq, D), generator=g, device=dev).to(torch.bfloat16)
    lens = torch.from_numpy(ctx.astype(np.int32)).to(dev)
    scale = 1.0 / math.sqrt(D)
    out = {}
    for bs in (1, 16):
        nblk = -(-ctx // bs)
        nb = int(math.ceil(int(nblk.sum()) * 1.1)) + 1
        perm = rng.permutation(np.arange(1, nb))
        bt = np.full((B, -(-4096 // bs)), -1, dtype=np.int32)
        pos = 0
        for s in range(B):
            bt[s, :nblk[s]] = perm[pos:pos + nblk[s]]
            pos += nblk[s]
        shape = (nb, Hkv, D) if bs == 1 else (nb, bs, Hkv, D)
        pools = [(torch.randn(shape, generator=g, device=dev).to(torch.bfloat16),
                  torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)) for _ in range(layers)]
        btd = torch.from_numpy(bt).to(dev)

        def step(i, pools=pools, btd=btd, bs=bs):
            kc, vc = pools[i % len(pools)]
            kernels.paged_attention_v1(q, kc, vc, btd, lens, Hkv, scale, bs, 4096)

        _, dev_s = timed_launches(step, steps, warmup)
        us = dev_s * 1e6 / steps
        nbytes = decode_bytes(ctx, B, Hq, Hkv, D, bs)
        gbs = nbytes / (us * 1e-6) / 1e9
        out["slot_table_bs1" if bs == 1 else "flash_bs16"] = dict(
            us=round(us, 2), bytes_per_launch=nbytes, gbs=round(gbs, 1), frac=round(gbs / PEAK_GBS, 4))
        del pools
        torch.cuda.empty_cache()
    out["kernel"] = "paged_decode_persist_kernel<BF16, BF16, 128, 0> (token-row mode)"
    out["timing"] = f"HIP events around {steps} back-to-back launches after {warmup} warm-up launches"
    return out


def bench_fp8(dev, kernels, layers: int = 4, steps: int = 100, warmup: int = 10):
    """The Llama-3-8B decode layer of bench_decode (same sequences, context
    lengths and block tables) over FP8 E4M3 caches (paged 5-D, x = 16) with
    k_scale / v_scale: half the KV bytes.  Layer pools rotated."""
    B, Hq, Hkv, D, bs = 64, 32, 8, 128, 16
    rng = np.random.default_rng(1003)
    ctx = rng.integers(512, 4096 + 1, size=B).astype(np.int64)
    nblk = -(-ctx // bs)
    nb = int(math.ceil(int(nblk.sum()) * 1.1)) + 1
    perm = rng.permutation(np.arange(1, nb))
    bt = np.full((B, -(-4096 // bs)), -1, dtype=np.int32)
    pos = 0
    for s in range(B):
        bt[s, :nblk[s]] = perm[pos:pos + nblk[s]]
        pos += nblk[s]
    g = torch.Generator(device=dev)
    g.manual_seed(1003)
    q = torch.randn((B, Hq, D), generator=g, device=dev).to(torch.bfloat16)
    k_scale, v_scale = 0.05, 0.02
    pools = []
    for _ in range(layers):
        kc = torch.empty((nb, Hkv, D // 16, bs, 16), dtype=torch.uint8, device=dev)
        vc = torch.empty((nb, Hkv, D, bs), dtype=torch.uint8, device=dev)
        kernels.convert_fp8(kc, torch.randn(kc.shape, generator=g, device=dev) * 1.5, k_scale * 20.0)
        kernels.convert_fp8(vc, torch.randn(vc.shape, generator=g, device=dev) * 0.5, v_scale * 20.0)
        pools.append((kc, vc))
    btd = torch.from_numpy(bt).to(dev)
    lens = torch.from_numpy(ctx.astype(np.int32)).to(dev)
    scale = 1.0 / math.sqrt(D)

    def step(i):
        kc, vc = pools[i % layers]
        kernels.paged_attention_v1(q, kc, vc, btd, lens, Hkv, scale, bs, 4096, k_scale=k_scale, v_scale=v_scale)

    _, dev_s = timed_launches(step, steps, warmup)
    us = dev_s * 1e6 / steps
    nbytes = decode_bytes(ctx, B, Hq, Hkv, D, bs, s_kv=1)
    gbs = nbytes / (us * 1e-6) / 1e9
    out = dict(us=round(us, 2), bytes_per_launch=nbytes, gbs=round(gbs, 1), frac=round(gbs / PEAK_GBS, 4),
               kernel="paged_decode_persist_kernel<BF16, FP8, 128, 16>",
               cache="E4M3 (reference format), x = 16, k_scale 0.05, v_scale 0.02",
               timing=f"HIP events around {steps} back-to-back launches after {warmup} warm-up launches")
    del pools
    torch.cuda.empty_cache()
    return out


def bench_batch_sweep(dev, kernels, batches=(8, 16, 32, 48, 63, 64, 96, 128), launches: int = 24):
    """The Llama-3-8B decode layer (32 q / 8 kv heads, D128, bs16, ctx
    U[512, 4096], bf16) through paged_attention_v1 at several batch sizes,
    each a HIP graph of `launches` calls over layer pools rotated to exceed
    the Infinity Cache (median of 5 replays)."""
    Hq, Hkv, D, bs = 32, 8, 128, 16
    scale = 1.0 / math.sqrt(D)
    rows = []
    for B in batches:
        pool_bytes = int(B * 2304 * Hkv * D * 2 * 2 * 1.1)
        layers = max(2, -(-800_000_000 // pool_bytes))
        inp = decode_inputs(1003, B=B, Hq=Hq, Hkv=Hkv, D=D, bs=bs, ctx_lo=512, ctx_hi=4096, layers=layers, dev=dev)
        nbytes = decode_bytes(inp["ctx_np"], B, Hq, Hkv, D, bs)

        def step(i):
            kc, vc = inp["pools"][i % layers]
            return kernels.paged_attention_v1(inp["q"], kc, vc, inp["bt"], inp["ctx"], Hkv, scale, bs, 4096)

        ms = graph_launch_ms(step, launches)
        gbs = nbytes / (ms * 1e-3) / 1e9
        rows.append(dict(batch=B, us=round(ms * 1e3, 2), bytes_per_launch=nbytes, gbs=round(gbs, 1),
                         frac=round(gbs / PEAK_GBS, 4), max_ctx=int(inp["ctx_np"].max())))
        del inp
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return dict(workload="llama3-8b paged decode layer at several batch sizes: 32 q / 8 kv heads, D128, bs16, "
                         "ctx U[512,4096] (seed 1003), bf16", rows=rows,
                method=f"HIP graph of {launches} calls over rotated pools (> 800 MB), median of 5 replays")


def bench_append(dev, kernels, sources: int = 24, pools: int = 4, launches: int = 96):
    """Append workload: 4096 tokens, 8 KV heads, D 128, bf16, 65,536 slots
    (4096 blocks of 16), unique random slots (slot 0 reserved), 5% = -1."""
    N, H, D, S, bs = 4096, 8, 128, 65536, 16
    rng = np.random.default_rng(1002)
    g = torch.Generator(device=dev)
    g.manual_seed(1002)
    srcs, maps, nvalid = [], [], []
    for _ in range(sources):
        slots = rng.choice(S - 1, size=N, replace=False).astype(np.int64) + 1
        slots[rng.choice(N, size=int(round(0.05 * N)), replace=False)] = -1
        nvalid.append(int((slots >= 0).sum()))
        maps.append(torch.from_numpy(slots.astype(np.int32)).to(dev))
        srcs.append((torch.randn((N, H, D), generator=g, device=dev).to(torch.bfloat16),
                     torch.randn((N, H, D), generator=g, device=dev).to(torch.bfloat16)))
    nv = sum(nvalid) / len(nvalid)
    nbytes = int(2 * nv * H * D * 2 + 2 * nv * H * D * 2 + N * 4)
    out = {}
    for layout in ("token_major", "paged5d"):
        if layout == "token_major":
            caches = [(torch.zeros((S, H, D), dtype=torch.bfloat16, device=dev),
                       torch.zeros((S, H, D), dtype=torch.bfloat16, device=dev)) for _ in range(pools)]
        else:
            caches = [(torch.zeros((S // bs, H, D // 8, bs, 8), dtype=torch.bfloat16, device=dev),
                       torch.zeros((S // bs, H, D, bs), dtype=torch.bfloat16, device=dev)) for _ in range(pools)]

        def launch(i):
            k, v = srcs[i % sources]
            kc, vc = caches[i % pools]
            kernels.reshape_and_cache(k, v, kc, vc, maps[i % sources])

        ms = graph_launch_ms(launch, launches)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[layout] = dict(us_per_launch=round(ms * 1e3, 3), achieved_gbs=round(gbs, 1),
                           frac=round(gbs / PEAK_GBS, 4))
        del caches
    torch.cuda.synchronize()
    out["bytes_per_launch"] = nbytes
    out["workload"] = ("reshape_and_cache: 4096 tokens, 8 kv heads, D128, bf16, 65536 slots "
                       "(4096 blocks of 16), unique random slots, 5% padding")
    out["kernel"] = APPEND_KERNEL
    out["method"] = f"HIP graph of {launches} launches over {sources} sources x {pools} pools, median of 5 replays"
    return out


def bench_splitk(dev, kernels, launches: int = 24):
    """Long-context split-K decode: Qwen2-7B shape (28 q / 4 kv heads, D128,
    bs16, bf16), B in {1, 4}, every context 32K / 64K / 128K tokens.  Each
    configuration rotates enough KV pools to exceed 600 MB (more than the
    Infinity Cache); paged_attention_v1 (the build's own partition choice) and
    paged_attention_v2 with 512-token partitions are timed as HIP graphs of
    `launches` calls (median of 5 replays)."""
    out = []
    Hq, Hkv, D, bs = 28, 4, 128, 16
    scale = 1.0 / math.sqrt(D)
    for B in (1, 4):
        for ctx in (32768, 65536, 131072):
            pool_bytes = int(B * ctx * Hkv * D * 2 * 2 * 1.1)
            layers = max(2, -(-600_000_000 // pool_bytes))
            inp = decode_inputs(1004, B=B, Hq=Hq, Hkv=Hkv, D=D, bs=bs, ctx_lo=ctx, ctx_hi=ctx, layers=layers,
                                dev=dev)
            nbytes = decode_bytes(inp["ctx_np"], B, Hq, Hkv, D, bs)
            row = dict(batch=B, ctx=ctx, bytes_per_launch=nbytes, kv_pools_rotated=layers)
            for mode in ("v1", "v2_p512"):
                def step(i, mode=mode):
                    kc, vc = inp["pools"][i % layers]
                    args = (inp["q"], kc, vc, inp["bt"], inp["ctx"], Hkv, scale, bs, inp["max_seq_len"])
                    if mode == "v1":
                        return kernels.paged_attention_v1(*args)
                    return kernels.paged_attention_v2(*args, partition_size=512)

                ms = graph_launch_ms(step, launches)
                gbs = nbytes / (ms * 1e-3) / 1e9
                row[mode] = dict(us=round(ms * 1e3, 2), achieved_gbs=round(gbs, 1), frac=round(gbs / PEAK_GBS, 4))
            out.append(row)
            del inp
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
    return dict(workload="qwen2-7b split-K decode: 28 q / 4 kv heads, D128, bs16, bf16, B in {1,4}, "
                         "ctx in {32K, 64K, 128K}", configs=out,
                method=f"HIP graph of {launches} calls over rotated pools, median of 5 replays")


# GPU spin queued before each radix window.  After a churn step the GPU is
# idle, and queueing four calls takes the host longer than the 80 us that a
# single launch needs: with 80 us the first window after a churn held ~8 us
# per launch of host time between the kernels.
RADIX_SPIN_US = 400.0


def bench_radix(dev, kernels, steps: int = 40, warmup: int = 5, layers: int = 4, fp8: bool = False):
    """Radix-shared decode (tests/pkv_workloads.py): 256 sequences (Llama-3-8B
    heads: 32 q / 8 kv, D128, bs16, bf16) whose block tables all start with
    the same 128 blocks (a 2048-token shared prefix) followed by 64..512
    private tokens.  Between steps 10% of the private blocks are evicted and
    re-allocated through the block allocator (freed in a shuffled order, so
    blocks change hands), their K/V rewritten with the append kernel, and
    the tables rebuilt.  Each step then decodes every one of `layers`
    independent layer pools (each with its own prefix blocks) back to back,
    as a model's layers would run; a HIP event pair around those launches,
    divided by `layers`, is the step's time per launch.  fp8: the caches
    hold FP8 E4M3 codes (k_scale 0.05, v_scale 0.02), written by the FP8
    append and read by the FP8 decode."""
    from pkv_workloads import B, BS, D, HKV, HQ, SHARED_BLOCKS, RadixSharedWorkload

    w = RadixSharedWorkload(dev, kernels, layers=layers, fp8=fp8)
    # Each mode decodes right after a churn step of its own (the order of
    # the two modes alternates from step to step), then decodes the same
    # step once more.  The first decode after the appends pays for whatever
    # the appends leave in the caches, as a serving step would; the second
    # is the decode alone.  (With the appends' whole-block runs written as
    # whole lines the two measure the same.)
    times = {(m, k): [] for m in ("cascade", "v1") for k in ("first", "second")}

    def launches(mode, info):
        for layer in range(layers):
            if mode == "cascade":
                w.decode_cascade(layer, info["bt_dev"], info["ctx_dev"], info["plan"])
            else:
                w.decode(layer, info["bt_dev"], info["ctx_dev"])

    for it in range(warmup + steps):
        for mode in (("cascade", "v1") if it % 2 == 0 else ("v1", "cascade")):
            info = w.churn()
            for k in ("first", "second"):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                # The host queues four calls (argument checks and, for the
                # cascade, the plan's arrays) while the GPU spins: long
                # enough that the window holds the kernels, not the host.
                queue_ahead(RADIX_SPIN_US)
                a.record()
                launches(mode, info)
                b.record()
                if it >= warmup:
                    times[(mode, k)].append((a, b))
    torch.cuda.synchronize()
    meds = {}
    for key, ev in times.items():
        us = sorted(a.elapsed_time(b) * 1e3 / layers for a, b in ev)
        meds[key] = us[len(us) // 2]
    med = meds[("cascade", "first")]
    ctx_np = np.array([t.num_tokens for t in w.tables], dtype=np.int64)
    s_kv = 1 if fp8 else 2
    logical = decode_bytes(ctx_np, B, HQ, HKV, D, BS, s_kv=s_kv)
    unique = logical - (B - 1) * SHARED_BLOCKS * BS * HKV * D * 2 * s_kv
    cache = "FP8 E4M3 caches (k_scale 0.05, v_scale 0.02), bf16 query" if fp8 else "bf16"
    v1 = meds[("v1", "first")]
    return dict(workload="radix-shared decode: B256, 32 q / 8 kv heads, D128, bs16, " + cache + ", 128 shared "
                         "blocks (2048 tokens) + U[64,512] private tokens, 10% private-block evict/realloc churn "
                         "per step (blocks change hands)",
                path="paged_attention_cascade (prefix pass + tail pass, plan built on the host from the churned "
                     "tables)",
                us_per_launch=round(med, 2), unique_bytes_per_launch=int(unique), logical_bytes_per_launch=int(logical),
                unique_gbs=round(unique / (med * 1e-6) / 1e9, 1),
                unique_frac=round(unique / (med * 1e-6) / 1e9 / PEAK_GBS, 4),
                effective_gbs=round(logical / (med * 1e-6) / 1e9, 1), kv_pools_rotated=layers,
                us_per_launch_second=round(meds[("cascade", "second")], 2),
                v1=dict(path="paged_attention_v1 (grouped persistent kernel, no plan)", us_per_launch=round(v1, 2),
                        unique_frac=round(unique / (v1 * 1e-6) / 1e9 / PEAK_GBS, 4),
                        us_per_launch_second=round(meds[("v1", "second")], 2)),
                method=(f"median over {steps} steps of a HIP event pair around {layers} back-to-back decode calls "
                        f"(one per layer pool), divided by {layers}; each mode right after a churn step of its own "
                        f"(churn, append and the plan's host build outside the events; the two modes' order "
                        f"alternates), us_per_launch; then the same step decoded again, us_per_launch_second"))


def bench_ref_decode(dev, kernels, seq_lens=(1024, 4096, 8192), cpu_budget_s: float = 1.0):
    """The reference's own decode benchmark configuration
    (tests/bench_paged_vs_gather.py:9-45,120-123): batch 1, float16, 32 query
    / 8 KV heads, D 128, block_size 16, a pool of seq/16 + 10 blocks, the
    block table 0 .. seq/16 - 1, caches filled through reshape_and_cache
    with slots 0 .. seq-1 from uniform [0, 1) keys and values, a uniform
    query; seq in {1024, 4096, 8192}.  Per seq: paged_attention_v1's device
    time per call as a HIP graph of back-to-back calls on the one cache (as
    the reference reuses it: L2 and the Infinity Cache hold it) and on
    caches rotated past the Infinity Cache (HBM-bound, the % of 8 TB/s
    quoted), and the CPU baseline: the reference's gather + SDPA on the same
    inputs, torch on this host's cores."""
    from oracle import cpu_baseline as cb

    Hq, Hkv, D, bs, x = 32, 8, 128, 16, 8
    scale = 1.0 / math.sqrt(D)
    g = torch.Generator(device=dev)
    g.manual_seed(1006)
    rows = []
    for seq in seq_lens:
        nb = -(-seq // bs) + 10
        pool_bytes = nb * bs * Hkv * D * 2 * 2
        npools = max(2, -(-700_000_000 // pool_bytes))
        q = torch.rand((1, Hq, D), generator=g, device=dev).to(torch.float16)
        slots = torch.arange(seq, dtype=torch.int32, device=dev)
        pools = []
        for i in range(npools):
            kc = torch.zeros((nb, Hkv, D // x, bs, x), dtype=torch.float16, device=dev)
            vc = torch.zeros((nb, Hkv, D, bs), dtype=torch.float16, device=dev)
            ks = torch.rand((seq, Hkv, D), generator=g, device=dev).to(torch.float16)
            vs = torch.rand((seq, Hkv, D), generator=g, device=dev).to(torch.float16)
            kernels.reshape_and_cache(ks, vs, kc, vc, slots)
            pools.append((kc, vc))
        bt = torch.arange(seq // bs, dtype=torch.int32, device=dev).reshape(1, -1)
        ctx = torch.tensor([seq], dtype=torch.int32, device=dev)
        nbytes = decode_bytes(np.array([seq]), 1, Hq, Hkv, D, bs)

        def call(i, rotate):
            kc, vc = pools[i % npools] if rotate else pools[0]
            return kernels.paged_attention_v1(q, kc, vc, bt, ctx, Hkv, scale, bs, seq)

        hot = graph_launch_ms(lambda i: call(i, False), 100)
        cold = graph_launch_ms(lambda i: call(i, True), npools)
        gbs = nbytes / (cold * 1e-3) / 1e9
        kc0, vc0 = pools[0]
        qc, k5, v5, btc, ctxc = q.cpu(), kc0.cpu(), vc0.cpu(), bt.cpu(), ctx.cpu()
        t = cb.time_decode(qc, k5, v5, btc, ctxc, bs, scale, budget_s=cpu_budget_s,
                           fn=cb.gather_sdpa_decode_paged5d)
        ref = cb.gather_sdpa_decode_paged5d(qc, k5, v5, btc, ctxc, bs, scale)
        diff = (call(0, False).float().cpu() - ref.float()).abs().max().item()
        rows.append(dict(seq_len=seq, bytes_per_call=nbytes, us_same_cache=round(hot * 1e3, 2),
                         us=round(cold * 1e3, 2), gbs=round(gbs, 1), frac=round(gbs / PEAK_GBS, 4),
                         caches_rotated=npools,
                         cpu_baseline=dict(us=round(t["median_s"] * 1e6, 1),
                                           gbs=round(nbytes / t["median_s"] / 1e9, 2), cores=t["threads"],
                                           kind="port", iters=t["iters"]),
                         max_abs_diff_vs_cpu=round(diff, 5)))
        del pools
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return dict(workload="reference decode benchmark: B1, fp16, 32 q / 8 kv heads, D128, bs16, contiguous "
                         "blocks, seq in {1024, 4096, 8192}", rows=rows,
                method="HIP graph of back-to-back calls (median of 5 replays): us_same_cache on one cache, us "
                       "over caches rotated past 700 MB; CPU: gather + SDPA (relayout included), torch CPU, "
                       "median over a 1 s sample")


def bench_ref_append(dev, kernels, counts=(1, 8, 16, 64, 128, 256, 512, 1024), cpu_budget_s: float = 0.5):
    """The reference's own append benchmark configuration
    (tests/bench_reshape_and_cache.py:29-37,60-89): float16, 8 KV heads,
    D 128, block_size 16, a pool of ceil(N/16) + 1 blocks, slots 0 .. N-1,
    uniform [0, 1) keys and values, N in {1, 8, 16, 64, 128, 256, 512,
    1024}.  Per N: device time per launch as a HIP graph of 100 launches,
    the host-synchronous call latency the reference measures (call then
    synchronise, median of 100 after 20 warm-ups), % of 8 TB/s on the
    algorithmic bytes (K and V read and written, the slot ids read), the
    reference's own write bandwidth (K and V bytes written / device time),
    and the CPU baseline: the same scatter with torch on this host's
    cores."""
    from oracle import cpu_baseline as cb

    H, D, bs, x = 8, 128, 16, 8
    g = torch.Generator(device=dev)
    g.manual_seed(1007)
    rows = []
    for n in counts:
        nb = -(-n // bs) + 1
        kc = torch.zeros((nb, H, D // x, bs, x), dtype=torch.float16, device=dev)
        vc = torch.zeros((nb, H, D, bs), dtype=torch.float16, device=dev)
        k = torch.rand((n, H, D), generator=g, device=dev).to(torch.float16)
        v = torch.rand((n, H, D), generator=g, device=dev).to(torch.float16)
        slots = torch.arange(n, dtype=torch.int32, device=dev)

        def call(i):
            kernels.reshape_and_cache(k, v, kc, vc, slots)

        dev_ms = graph_launch_ms(call, 100)
        for _ in range(20):
            call(0)
        torch.cuda.synchronize()
        lat = []
        for _ in range(100):
            t0 = time.perf_counter()
            call(0)
            torch.cuda.synchronize()
            lat.append(time.perf_counter() - t0)
        lat.sort()
        written = n * H * D * 2 * 2
        nbytes = 2 * written + n * 4
        kcc, vcc = kc.cpu().zero_(), vc.cpu().zero_()
        kk, vv, ss = k.cpu(), v.cpu(), slots.cpu()
        t = cb.time_calls(lambda: cb.scatter_append_paged5d(kk, vv, kcc, vcc, ss), budget_s=cpu_budget_s)
        same = bool(torch.equal(kcc, kc.cpu()) and torch.equal(vcc, vc.cpu()))
        rows.append(dict(tokens=n, bytes_per_launch=nbytes, us=round(dev_ms * 1e3, 3),
                         gbs=round(nbytes / (dev_ms * 1e-3) / 1e9, 1),
                         frac=round(nbytes / (dev_ms * 1e-3) / 1e9 / PEAK_GBS, 4),
                         write_gbs=round(written / (dev_ms * 1e-3) / 1e9, 1),
                         call_latency_us=round(lat[len(lat) // 2] * 1e6, 1),
                         cpu_baseline=dict(us=round(t["median_s"] * 1e6, 2),
                                           gbs=round(nbytes / t["median_s"] / 1e9, 2), cores=t["threads"],
                                           kind="port", iters=t["iters"]),
                         cpu_equal=same))
    return dict(workload="reference append benchmark: fp16, 8 kv heads, D128, bs16, slots 0..N-1, "
                         "N in {1, 8, 16, 64, 128, 256, 512, 1024}", rows=rows,
                method="device: HIP graph of 100 launches (median of 5 replays); call_latency: call + "
                       "synchronise, median of 100; CPU: torch scatter into the paged 5-D caches, median over "
                       "a 0.5 s sample")


def bench_cpu(res, budget_s):
    """CPU baseline leg: the oracle package's torch-CPU gather + SDPA, same
    inputs (layer 0), full batch.  The reported value follows
    tests/bench_paged_vs_gather.py:84-103 of the reference: each step relays
    the paged 5-D caches out as token-major copies, then gathers and runs
    SDPA per sequence.  token_major_pool times the same decode from pools
    already token-major (MHATokenPool's layout, memory_pool.py:102-108),
    built outside the timed region."""
    from oracle import cpu_baseline as cb

    inp = res["inp"]
    kc, vc = inp["pools"][0]
    bs = inp["bs"]
    k5, v5 = kc.cpu(), vc.cpu()
    q, bt, ctx = inp["q"].cpu(), inp["bt"].cpu(), inp["ctx"].cpu()
    t = cb.time_decode(q, k5, v5, bt, ctx, bs, res["scale"], budget_s=budget_s, fn=cb.gather_sdpa_decode_paged5d)
    cpu_out = cb.gather_sdpa_decode_paged5d(q, k5, v5, bt, ctx, bs, res["scale"])
    k_pool, v_pool = cb.paged5d_to_token_major(k5, v5)
    tm = cb.time_decode(q, k_pool, v_pool, bt, ctx, bs, res["scale"], budget_s=budget_s / 2)
    diff = (cpu_out.float() - res["out0"].float().cpu()).abs().max().item()
    gbs = res["nbytes"] / t["median_s"] / 1e9
    return dict(value=round(gbs, 2), unit="GB/s", cores=t["threads"], kind="port",
                sample=(f"full batch (64 seqs, one layer): relayout of the paged 5-D caches to token-major, "
                        f"then gather+SDPA per sequence, torch-CPU bf16, median of {t['iters']} iterations"),
                us_per_step=round(t["median_s"] * 1e6, 1), cpu=t["cpu"],
                label="CPU restatement of the reference's gather+SDPA path (MLX CPU backend unavailable offline)",
                token_major_pool=dict(us_per_step=round(tm["median_s"] * 1e6, 1),
                                      gbs=round(res["nbytes"] / tm["median_s"] / 1e9, 2), iters=tm["iters"]),
                max_abs_diff_vs_gpu=round(diff, 5))


def only_leg(args, dev, kernels):
    """One leg alone, for rocprofv3 counter runs."""
    if args.only == "decode":
        res = bench_decode(args, dev, kernels)
        print(json.dumps(dict(leg="decode", kernel=DECODE_KERNEL, bytes_per_launch=res["nbytes"],
                              mean_launch_us=round(res["mean_ms"] * 1e3, 2), launches=args.steps + args.warmup)))
    elif args.only == "append":
        out = bench_append(dev, kernels)
        print(json.dumps(dict(leg="append", **out)))
    elif args.only == "splitk":
        print(json.dumps(dict(leg="splitk", **bench_splitk(dev, kernels))))
    elif args.only == "radix":
        print(json.dumps(dict(leg="radix", **bench_radix(dev, kernels))))
    elif args.only == "radix_fp8":
        print(json.dumps(dict(leg="radix_fp8", **bench_radix(dev, kernels, fp8=True))))
    elif args.only == "rows":
        print(json.dumps(dict(leg="rows", **bench_rows(dev, kernels))))
    elif args.only == "fp8":
        print(json.dumps(dict(leg="fp8", **bench_fp8(dev, kernels))))
    elif args.only == "sweep":
        print(json.dumps(dict(leg="sweep", **bench_batch_sweep(dev, kernels))))
    elif args.only == "ref_decode":
        print(json.dumps(dict(leg="ref_decode", **bench_ref_decode(dev, kernels))))
    elif args.only == "ref_append":
        print(json.dumps(dict(leg="ref_append", **bench_ref_append(dev, kernels))))
    else:
        n = 1 << 30
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps(dict(leg="copy", bytes_read_per_launch=n, bytes_written_per_launch=n,
                              launches=args.steps)))


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} (WORLD_SIZE={world}) is not supported; "
              "the paged-KV path is benchmarked on a single MI355X", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    if args.lib:
        from sglang_mlx_amd import _lib
        _lib.LIB_PATH = os.path.abspath(args.lib)
    from sglang_mlx_amd import kernels

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.only:
        only_leg(args, dev, kernels)
        return
    res = bench_decode(args, dev, kernels)
    inp = res["inp"]
    B = inp["B"]
    # The counter summary's traffic holds for the build it was measured on:
    # it is marked stale when this run's mean launch time differs from the
    # kernel average recorded with it by more than 5%.
    traffic, traffic_avg_us = read_traffic("paged_decode_llama3_8b_traffic.txt")
    mean_us = res["mean_ms"] * 1e3
    if traffic is None:
        traffic_note = "no counter summary"
    elif traffic_avg_us is None or abs(mean_us - traffic_avg_us) > 0.05 * traffic_avg_us:
        traffic_note = (f"STALE: profiles/paged_decode_llama3_8b_traffic.txt was measured at a kernel average of "
                        f"{traffic_avg_us} us, this run's mean launch is {mean_us:.2f} us")
    else:
        traffic_note = (f"profiles/paged_decode_llama3_8b_traffic.txt (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated; "
                        f"kernel average there {traffic_avg_us} us, here {mean_us:.2f} us)")
    us = res["ms_step"] * 1e3
    value = res["nbytes"] / (res["ms_step"] * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "llama3-8b paged decode layer: B64, 32 q / 8 kv heads, D128, bs16, ctx U[512,4096], bf16",
            "batch": B, "num_heads": inp["Hq"], "num_kv_heads": inp["Hkv"], "head_size": inp["D"],
            "block_size": inp["bs"], "ctx_range": [512, 4096], "mean_ctx": float(inp["ctx_np"].mean()),
            "num_blocks": inp["nb"], "kv_pools_rotated": len(inp["pools"]), "parallelism": "none (1 GPU)",
        },
        "us_per_step": round(us, 2),
        "tokens_per_s": round(B / (res["ms_step"] * 1e-3), 1),
        "hbm_frac": round(value / PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm",
            "achieved": round(res["achieved"], 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(res["achieved"] / PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_note,
            "kernel": DECODE_KERNEL,
            "bytes_per_launch": res["nbytes"],
            "mean_launch_us": round(res["mean_ms"] * 1e3, 2),
            "timing": "HIP events around the timed region's back-to-back launches, divided by the steps",
            "median_single_launch_us": round(res["median_single_ms"] * 1e3, 2),
        },
    }
    if not args.no_append:
        line["append"] = bench_append(dev, kernels)
    if not args.no_splitk:
        line["split_k"] = bench_splitk(dev, kernels)
    if not args.no_radix:
        line["radix_shared"] = bench_radix(dev, kernels)
        if not args.no_fp8:
            line["radix_shared_fp8"] = bench_radix(dev, kernels, fp8=True)
    if not args.no_rows:
        line["token_rows"] = bench_rows(dev, kernels)
    if not args.no_fp8:
        line["fp8_kv"] = bench_fp8(dev, kernels)
    if not args.no_sweep:
        line["batch_sweep"] = bench_batch_sweep(dev, kernels)
    if not args.no_ref:
        line["ref_decode_b1"] = bench_ref_decode(dev, kernels)
        line["ref_append"] = bench_ref_append(dev, kernels)
    if not args.no_cpu:
        line["cpu_baseline"] = bench_cpu(res, args.cpu_budget)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    # Leave nothing queued or cached on the device when the interpreter
    # tears down (graphs and pools of every leg are released here).
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
