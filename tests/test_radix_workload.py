"""The radix-shared decode workload at full size (256 sequences, 128 shared
blocks = 2048 tokens, U[64, 512] private tokens, block size 16, 10%
evict/re-allocate churn per step), exactly as bench.py runs it
(tests/pkv_workloads.py).

CPU: the allocator and block-table state after setup and after each churn
step equals a brute-force restatement of the LIFO free stack
(memory_pool.py:27-68 applied to block ids), bit for bit, and the paged
kernels' invariants hold (identical shared prefix in every row, no private
block in two rows or in the prefix, one slot per logical token).

GPU: the same steps on real caches (bf16 and FP8 E4M3).  After each step the
whole layer pool equals the oracle's append applied to a host copy, bit for
bit, and the decode of all 256 sequences x 32 heads matches the oracle on
the current tables (bf16 query: 1e-2 abs / 2e-2 rel), through
paged_attention_v1 and through paged_attention_cascade with the plan rebuilt
from the churned tables."""

import numpy as np
import pytest
import torch

from pkv_workloads import BS, RadixSharedWorkload, SHARED_BLOCKS, B


class LifoModel:
    """Reference-counted LIFO stack of block ids, block 0 never handed out."""

    def __init__(self, nb):
        self.stack = list(range(nb - 1, 0, -1))
        self.ref = [0] * nb

    def alloc(self, n):
        assert 0 < n <= len(self.stack)
        out = self.stack[len(self.stack) - n:]
        del self.stack[len(self.stack) - n:]
        for b in out:
            self.ref[b] = 1
        return out

    def share(self, blocks):
        for b in blocks:
            self.ref[b] += 1

    def free(self, blocks):
        for b in blocks:
            self.ref[b] -= 1
            if self.ref[b] == 0:
                self.stack.append(b)


def model_setup(w):
    m = LifoModel(w.nb)
    shared = m.alloc(SHARED_BLOCKS)
    tables = []
    for n in w.priv_tokens:
        m.share(shared)
        tables.append(list(shared) + m.alloc(int(-(-int(n) // BS))))
    m.free(shared)
    return m, shared, tables


def expected_tables(tables, ctx_of, width):
    bt = np.full((len(tables), width), -1, dtype=np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    return bt, np.asarray(ctx_of, dtype=np.int32)


def check_state(w, m, shared, tables, bt, ctx):
    exp_bt, exp_ctx = expected_tables(tables, [SHARED_BLOCKS * BS + int(n) for n in w.priv_tokens], w.max_blocks)
    assert np.array_equal(bt, exp_bt) and np.array_equal(ctx, exp_ctx)
    assert w.alloc.available_size == len(m.stack)
    assert [w.alloc.refcount(b) for b in range(w.nb)] == m.ref
    assert (bt[:, :SHARED_BLOCKS] == np.asarray(shared)).all()
    priv = [b for t in tables for b in t[SHARED_BLOCKS:]]
    assert len(priv) == len(set(priv)) and not set(priv) & set(shared) and 0 not in priv
    for b in shared:
        assert m.ref[b] == B
    for i in range(0, B, 17):
        slots = {int(bt[i, p // BS]) * BS + p % BS for p in range(int(ctx[i]))}
        assert len(slots) == ctx[i]


def replay_churn(m, tables, info):
    victims = info["victims"]
    # The freed blocks are exactly the victims' blocks, in some order.
    assert sorted(info["freed"]) == sorted(tables[i][j] for i, j in victims)
    before = [tables[i][j] for i, j in victims]
    m.free(info["freed"])
    fresh = m.alloc(len(victims))
    assert info["fresh"] == fresh
    for (i, j), b in zip(victims, fresh):
        tables[i][j] = b
    return before, fresh


def test_churn_state_matches_brute_force_lifo():
    w = RadixSharedWorkload("cpu", kernels=None, layers=0)
    m, shared, tables = model_setup(w)
    bt, ctx = w.block_tables()
    check_state(w, m, shared, tables, bt, ctx)
    moved = 0
    for _ in range(5):
        info = w.churn()
        before, fresh = replay_churn(m, tables, info)
        check_state(w, m, shared, tables, info["bt"], info["ctx"])
        moved += sum(b != f for b, f in zip(before, fresh))
        # Slots rewritten: every token of every re-allocated block, in order.
        exp = [b * BS + o for (i, j), b in zip(info["victims"], fresh)
               for o in range(min(BS, int(info["ctx"][i]) - j * BS))]
        assert info["slots"].tolist() == exp
    assert moved > 0   # blocks really change hands


@pytest.mark.gpu
@pytest.mark.parametrize("cache", ["bfloat16", "fp8_e4m3"])
def test_full_shape_with_churn_on_gpu(cache):
    from oracle import pagedkv_oracle as orc
    from pkv_torch import to_f64, to_numpy
    from sglang_mlx_amd import kernels

    fp8 = cache == "fp8_e4m3"
    w = RadixSharedWorkload(torch.device("cuda"), kernels, layers=1, fp8=fp8)
    m, shared, tables = model_setup(w)
    kc, vc = w.pools[0]
    torch.cuda.synchronize()
    kc_np, vc_np = to_numpy(kc), to_numpy(vc)
    q_np = to_numpy(w.q)
    ks, vs = (w.scales["k_scale"], w.scales["v_scale"]) if fp8 else (1.0, 1.0)
    for step in range(3):
        info = w.churn()
        replay_churn(m, tables, info)
        check_state(w, m, shared, tables, info["bt"], info["ctx"])
        n = info["slots"].shape[0]
        kc_np, vc_np = orc.reshape_and_cache_paged5d(to_numpy(w.src_k[:n]), to_numpy(w.src_v[:n]), kc_np, vc_np,
                                                     info["slots"], "bfloat16", cache, ks, vs)
        out = w.decode(0, info["bt_dev"], info["ctx_dev"])
        torch.cuda.synchronize()
        assert np.array_equal(to_numpy(kc), kc_np), f"K pool differs after churn step {step}"
        assert np.array_equal(to_numpy(vc), vc_np), f"V pool differs after churn step {step}"
        ref = orc.paged_attention(q_np, kc_np, vc_np, info["bt"], info["ctx"], 8, w.scale, BS, w.max_seq_len,
                                  None, "bfloat16", cache, ks, vs)
        np.testing.assert_allclose(to_f64(out), ref, atol=1e-2, rtol=2e-2, err_msg=f"churn step {step}")
        # The shared-prefix (cascade) decode of the same step, with the plan
        # rebuilt from the churned tables.
        assert info["plan"].groups[0][1] == SHARED_BLOCKS * BS
        outc = w.decode_cascade(0, info["bt_dev"], info["ctx_dev"], info["plan"])
        torch.cuda.synchronize()
        np.testing.assert_allclose(to_f64(outc), ref, atol=1e-2, rtol=2e-2, err_msg=f"cascade, churn step {step}")
