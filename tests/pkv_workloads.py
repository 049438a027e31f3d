"""The radix-shared decode workload, shared by bench.py and the GPU tests.

256 sequences with Llama-3-8B heads (32 query / 8 KV, head size 128, block
size 16) whose block tables all start with the same 128 blocks (a 2048-token
shared prefix), each followed by U[64, 512] private tokens in blocks spread
over a pool of 1.2x the blocks needed.  Tables are built with the product's
BlockAllocator / BlockTable (block 0 is never handed out).

Between decode steps, ``churn()`` evicts 10% of the private blocks and
re-allocates them: the victims go back to the free stack in a seeded random
order, and the same number of blocks is allocated for the victims' positions.
The allocator is a LIFO stack, so the blocks that come back are the evicted
ones, but in the shuffled order: blocks move between sequences and positions
(freeing and re-allocating in one order would give every position its own
block back).  Each re-allocated block's tokens are rewritten through
reshape_and_cache into every layer pool, and the int32 tables and context
lengths are rebuilt, and so is the shared-prefix plan of paged_attention_cascade.
"""

from __future__ import annotations

import math

import numpy as np
import torch

B, HQ, HKV, D, BS = 256, 32, 8, 128, 16
SHARED_BLOCKS = 128
PRIV_LO, PRIV_HI = 64, 512
K_SCALE, V_SCALE = 0.05, 0.02


class RadixSharedWorkload:
    def __init__(self, dev, kernels, layers: int = 4, fp8: bool = False, seed: int = 1005):
        from sglang_mlx_amd.srt.mem_cache import BlockAllocator, BlockTable

        self.dev, self.kernels, self.fp8 = dev, kernels, fp8
        self.rng = np.random.default_rng(seed)
        self.priv_tokens = self.rng.integers(PRIV_LO, PRIV_HI + 1, size=B)
        self.nb = int((SHARED_BLOCKS + (-(-self.priv_tokens // BS)).sum()) * 1.2) + 1
        self.alloc = BlockAllocator(self.nb)
        self.shared = self.alloc.alloc(SHARED_BLOCKS)
        self.tables = []
        for i in range(B):
            t = BlockTable.from_prefix(self.alloc, BS, self.shared)
            t.append_slots(int(self.priv_tokens[i]), self.alloc)
            self.tables.append(t)
        self.alloc.free(self.shared)  # the tables hold the prefix from here on
        self.max_blocks = max(len(t.blocks) for t in self.tables) + 1
        self.max_seq_len = self.max_blocks * BS
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.pools = []
        for _ in range(layers):
            if fp8:
                kc = torch.empty((self.nb, HKV, D // 16, BS, 16), dtype=torch.uint8, device=dev)
                vc = torch.empty((self.nb, HKV, D, BS), dtype=torch.uint8, device=dev)
                kernels.convert_fp8(kc, torch.randn(kc.shape, generator=g, device=dev), K_SCALE)
                kernels.convert_fp8(vc, torch.randn(vc.shape, generator=g, device=dev), V_SCALE)
            else:
                kc = torch.randn((self.nb, HKV, D // 8, BS, 8), generator=g, device=dev).to(torch.bfloat16)
                vc = torch.randn((self.nb, HKV, D, BS), generator=g, device=dev).to(torch.bfloat16)
            self.pools.append((kc, vc))
        self.scales = dict(k_scale=K_SCALE, v_scale=V_SCALE) if fp8 else {}
        self.q = torch.randn((B, HQ, D), generator=g, device=dev).to(torch.bfloat16)
        # Enough source rows for the largest possible churn (10% of the most
        # private blocks the contexts allow, whole blocks).
        rows = (B * -(-PRIV_HI // BS) // 10 + 1) * BS
        self.src_k = torch.randn((rows, HKV, D), generator=g, device=dev).to(torch.bfloat16)
        self.src_v = torch.randn((rows, HKV, D), generator=g, device=dev).to(torch.bfloat16)
        self.scale = 1.0 / math.sqrt(D)

    def block_tables(self):
        from sglang_mlx_amd.srt.mem_cache import build_block_tables

        return build_block_tables(self.tables, self.max_blocks)

    def churn(self) -> dict:
        """One evict/re-allocate step (see the module docstring).  Returns the
        victims (sequence, block index), the blocks in the order they were
        freed, the blocks allocated, the slots rewritten (int32, in source-row
        order), and the device block tables and context lengths."""
        private = [(i, j) for i, t in enumerate(self.tables) for j in range(SHARED_BLOCKS, len(t.blocks))]
        pick = self.rng.choice(len(private), size=len(private) // 10, replace=False)
        victims = [private[k] for k in pick]
        order = self.rng.permutation(len(victims))
        freed = [self.tables[victims[k][0]].blocks[victims[k][1]] for k in order]
        self.alloc.free(freed)
        fresh = self.alloc.alloc(len(victims))
        slots = []
        for (i, j), blk in zip(victims, fresh):
            self.tables[i].blocks[j] = blk
            ntok = min(BS, self.tables[i].num_tokens - j * BS)
            slots.extend(blk * BS + o for o in range(ntok))
        slots = np.asarray(slots, dtype=np.int32)
        sd = torch.from_numpy(slots).to(self.dev, non_blocking=True)
        n = slots.shape[0]
        for kc, vc in self.pools:
            self.kernels.reshape_and_cache(self.src_k[:n], self.src_v[:n], kc, vc, sd, **self.scales)
        bt, ctx = self.block_tables()
        return dict(victims=victims, freed=freed, fresh=fresh, slots=slots, bt=bt, ctx=ctx,
                    bt_dev=torch.from_numpy(bt).to(self.dev, non_blocking=True),
                    ctx_dev=torch.from_numpy(ctx).to(self.dev, non_blocking=True),
                    plan=self.plan(bt, ctx))

    def plan(self, bt, ctx):
        """The shared-prefix plan of the current tables (host work, like the
        tables themselves)."""
        from sglang_mlx_amd.srt.mem_cache import build_cascade_plan

        return build_cascade_plan(bt, ctx, BS, HQ, HKV, device=self.dev)

    def decode(self, layer: int, bt_dev, ctx_dev):
        kc, vc = self.pools[layer]
        return self.kernels.paged_attention_v1(self.q, kc, vc, bt_dev, ctx_dev, HKV, self.scale, BS,
                                               self.max_seq_len, **self.scales)

    def decode_cascade(self, layer: int, bt_dev, ctx_dev, plan):
        kc, vc = self.pools[layer]
        return self.kernels.paged_attention_cascade(self.q, kc, vc, bt_dev, ctx_dev, HKV, self.scale, BS,
                                                    self.max_seq_len, plan, **self.scales)
