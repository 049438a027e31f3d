"""Block-granular bookkeeping driving the HIP kernels end to end: a prompt's
whole blocks are shared through BlockRadixCache, a forked request takes a
copy-on-write copy of the shared partial block (copy_blocks), new tokens are
appended into the paged 5-D caches (reshape_and_cache) at the slots the
block tables hand out, and paged_attention_v1 decodes every request from the
built tables.  The expected outputs come from each request's own dense K/V
sequence kept on the host (float64 softmax attention, the oracle's
restatement of paged_attention_kernels.metal:37-168), so a wrong slot, a
missed copy or a shared block written through would all show.  Tolerance:
bf16, 1e-2 abs / 2e-2 rel."""

import math

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from pkv_cases import normal
from pkv_torch import to_f64, to_index, to_torch
from sglang_mlx_amd import kernels
from sglang_mlx_amd.srt.mem_cache import BlockAllocator, BlockRadixCache, BlockTable, build_block_tables

pytestmark = pytest.mark.gpu

Hq, Hkv, D, BS, NB = 8, 2, 64, 16, 64
X = 8  # 16-byte K chunks of bf16


class Request:
    def __init__(self, table):
        self.table = table
        self.k = np.zeros((0, Hkv, D), dtype=np.uint16)   # dense bf16 bits, context order
        self.v = np.zeros((0, Hkv, D), dtype=np.uint16)


def write(req, alloc, kc, vc, k_new, v_new):
    """Append tokens: copy-on-write first, then the append kernel."""
    slots, copies = req.table.append_slots(k_new.shape[0], alloc)
    if copies:
        kernels.copy_blocks([kc], [vc], torch.tensor(copies, dtype=torch.int64))
    kernels.reshape_and_cache(to_torch(k_new, "bfloat16"), to_torch(v_new, "bfloat16"), kc, vc,
                              to_index(slots))
    req.k = np.concatenate([req.k, k_new])
    req.v = np.concatenate([req.v, v_new])


def fork(req, alloc):
    child = Request(req.table.fork(alloc))
    child.k, child.v = req.k.copy(), req.v.copy()
    return child


def test_radix_sharing_copy_on_write_append_and_decode():
    rng = np.random.default_rng(11)
    alloc = BlockAllocator(NB)
    radix = BlockRadixCache(BS, alloc, clock=iter(range(10 ** 6)).__next__)
    kc = to_torch(orc.to_storage(rng.standard_normal((NB, Hkv, D // X, BS, X), dtype=np.float32), "bfloat16"),
                  "bfloat16")
    vc = to_torch(orc.to_storage(rng.standard_normal((NB, Hkv, D, BS), dtype=np.float32), "bfloat16"), "bfloat16")
    tok = lambda n: normal(rng, (n, Hkv, D), "bfloat16")

    # A: a 40-token prompt (blocks full, full, 8/16); its whole blocks go into the tree.
    prompt = list(rng.integers(0, 1000, size=40))
    a = Request(BlockTable(BS))
    write(a, alloc, kc, vc, tok(40), tok(40))
    assert radix.insert(prompt, a.table.blocks) == 0
    # B: the same first 32 tokens from the tree, then 12 of its own.
    blocks, _ = radix.match_prefix(prompt[:32] + [5, 6, 7])
    assert blocks == a.table.blocks[:2]
    b = Request(BlockTable.from_prefix(alloc, BS, blocks))
    b.k, b.v = a.k[:32].copy(), a.v[:32].copy()
    write(b, alloc, kc, vc, tok(12), tok(12))
    # C: a fork of A (parallel sampling); its first append copies A's partial block.
    c = fork(a, alloc)
    shared_tail = a.table.blocks[2]
    write(c, alloc, kc, vc, tok(3), tok(3))
    assert c.table.blocks[2] != shared_tail and c.table.blocks[:2] == a.table.blocks[:2]
    # A keeps writing into its own (now unshared) partial block.
    write(a, alloc, kc, vc, tok(2), tok(2))
    assert a.table.blocks[2] == shared_tail
    # D: a long request crossing several blocks.
    d = Request(BlockTable(BS))
    write(d, alloc, kc, vc, tok(70), tok(70))

    reqs = [a, b, c, d]
    bt, ctx = build_block_tables([r.table for r in reqs])
    assert ctx.tolist() == [42, 44, 43, 70]
    q = normal(rng, (len(reqs), Hq, D), "bfloat16")
    scale = 1.0 / math.sqrt(D)
    out = kernels.paged_attention_v1(to_torch(q, "bfloat16"), kc, vc, to_index(bt), to_index(ctx), Hkv, scale, BS,
                                     int(bt.shape[1] * BS))
    torch.cuda.synchronize()
    q64 = orc.decode(q, "bfloat16")
    for i, r in enumerate(reqs):
        exp = orc._softmax_attend(q64[i], orc.decode(r.k, "bfloat16"), orc.decode(r.v, "bfloat16"), scale, None)
        np.testing.assert_allclose(to_f64(out)[i], exp, atol=1e-2, rtol=2e-2)

    # Evicting the tree drops only its references; releasing every table
    # returns every block.
    assert radix.evict(100) == 2
    for r in reqs:
        r.table.release(alloc)
    assert alloc.available_size == NB - 1
