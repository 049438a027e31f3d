"""Long-context split-K decode at every Qwen2-7B configuration of the
benchmark: 28 query / 4 KV heads (GQA 7), head size 128, block size 16,
bf16, batch 1 and 4, contexts of 32K, 64K and 128K tokens, through
paged_attention_v1 (the library's own partitioning) and paged_attention_v2
with 512- and 4096-token partitions.  Inputs are generated on the device
from a seeded generator (up to 1.07 GB of KV).

Three checks per configuration:
  * one whole sequence, all 28 heads, against the float64 oracle (its
    blocks gathered into a compact cache so that host memory stays bounded):
    bf16 tolerance 1e-2 abs / 2e-2 rel;
  * every row: v1, v2(512) and v2(4096) agree within the same tolerance
    (the merge is an identity; only float32 summation order and the 16-bit
    rounding of the softmax weights differ);
  * closed form: the first query head of every KV group has q = 0, so all
    its weights are exp(0) = 1 and the output is sum(V) / (ctx + 1e-6), the
    mean of V over the context.  The float64 mean is computed on the device;
    the bound is bf16 output rounding (2^-8 relative) plus 1e-6.  Dropping
    one 512-token partition moves that mean by about 6% at 128K, so a lost,
    doubled or misweighted partition fails here even where the first two
    checks' tolerance is wide compared to outputs of size 1/sqrt(ctx).
"""

import math

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from pkv_torch import to_f64, to_numpy
from sglang_mlx_amd import _ext

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS = 28, 4, 128, 16
GROUP = HQ // HKV
CONFIGS = [(1, 32768), (1, 65536), (1, 131072), (4, 32768), (4, 65536), (4, 131072)]


def make_inputs(B, ctx, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    nblk = ctx // BS
    nb = int(B * nblk * 1.1) + 1
    q = torch.randn((B, HQ, D), generator=g, device="cuda").to(torch.bfloat16)
    q[:, ::GROUP] = 0
    kc = torch.randn((nb, HKV, D // 8, BS, 8), generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn((nb, HKV, D, BS), generator=g, device="cuda").to(torch.bfloat16)
    perm = torch.randperm(nb - 1, generator=torch.Generator().manual_seed(seed)) + 1
    bt = perm[:B * nblk].reshape(B, nblk).to(torch.int32).cuda()
    lens = torch.full((B,), ctx, dtype=torch.int32, device="cuda")
    return q, kc, vc, bt, lens


@pytest.mark.parametrize("B,ctx", CONFIGS)
def test_qwen2_long_context(B, ctx):
    print(f"\nqwen2 split-K B={B} ctx={ctx}", flush=True)
    q, kc, vc, bt, lens = make_inputs(B, ctx, seed=9000 + B * 1000 + ctx // 1024)
    scale = 1.0 / math.sqrt(D)
    args = (q, kc, vc, bt, lens, HKV, scale, BS, ctx)
    v1 = _ext.paged_attention_v1(*args)
    v2 = _ext.paged_attention_v2(*args, partition_size=512)
    v4 = _ext.paged_attention_v2(*args, partition_size=4096)
    torch.cuda.synchronize()
    outs = {"v1": to_f64(v1), "v2_512": to_f64(v2), "v2_4096": to_f64(v4)}
    for name, o in outs.items():
        assert np.isfinite(o).all(), name

    # Oracle on the last sequence, all heads.
    s = B - 1
    idx = bt[s].long()
    kcs = to_numpy(kc.index_select(0, idx))
    vcs = to_numpy(vc.index_select(0, idx))
    compact = np.arange(ctx // BS, dtype=np.int32)[None, :]
    ref = orc.paged_attention(to_numpy(q[s:s + 1]), kcs, vcs, compact, np.array([ctx], dtype=np.int32), HKV, scale,
                              BS, ctx, None, "bfloat16", "bfloat16")[0]
    del kcs, vcs
    for name, o in outs.items():
        np.testing.assert_allclose(o[s], ref, atol=1e-2, rtol=2e-2, err_msg=name)

    # v1 == v2(512) == v2(4096), every row.
    np.testing.assert_allclose(outs["v2_512"], outs["v1"], atol=1e-2, rtol=2e-2)
    np.testing.assert_allclose(outs["v2_4096"], outs["v1"], atol=1e-2, rtol=2e-2)

    # Uniform-weight heads: exact mean of V over the context.
    for seq in range(B):
        v = vc.index_select(0, bt[seq].long())                  # [nblk, Hkv, D, BS]
        mean = (v.double().sum(dim=(0, 3)) / (ctx + 1e-6)).cpu().numpy()   # [Hkv, D]
        for name, o in outs.items():
            got = o[seq, ::GROUP]                                # [Hkv, D]
            np.testing.assert_allclose(got, mean, atol=1e-6, rtol=2 ** -8, err_msg=f"{name} seq {seq}")
