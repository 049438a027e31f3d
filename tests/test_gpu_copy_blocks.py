"""GPU parity of copy_blocks / swap_blocks against the oracle, bit-exact over
whole caches: the reference's known-answer tests
(tests/test_paged_attention_kernel.py:400-438), paged caches of every cache
dtype over several layers, out-of-range pairs (skipped), a 2000-pair copy of
32 KiB blocks, and swaps between GPU buffers and between host and GPU."""

import numpy as np
import pytest
import torch

from oracle import pagedkv_oracle as orc
from sglang_mlx_amd import kernels

pytestmark = pytest.mark.gpu


def test_reference_kat_copy_blocks_multiple_layers():
    keys = [np.arange(24, dtype=np.float32).reshape(4, 2, 3) + layer * 100 for layer in range(2)]
    vals = [k + 1000 for k in keys]
    kc = [torch.from_numpy(k).cuda() for k in keys]
    vc = [torch.from_numpy(v).cuda() for v in vals]
    mapping = torch.tensor([[0, 2], [1, 3]], dtype=torch.int32)
    nk, nv = kernels.copy_blocks(kc, vc, mapping)
    torch.cuda.synchronize()
    ek, ev = orc.copy_blocks(keys, vals, mapping.numpy())
    for layer in range(2):
        assert nk[layer] is kc[layer] and nv[layer] is vc[layer]
        np.testing.assert_array_equal(nk[layer].cpu().numpy(), ek[layer])
        np.testing.assert_array_equal(nv[layer].cpu().numpy(), ev[layer])


def test_reference_kat_swap_blocks_noncontiguous_mapping():
    src = np.arange(24, dtype=np.float32).reshape(4, 2, 3)
    dst = np.full((4, 2, 3), -1, dtype=np.float32)
    d = torch.from_numpy(dst).cuda()
    out = kernels.swap_blocks(torch.from_numpy(src).cuda(), d, torch.tensor([[0, 2], [3, 1]], dtype=torch.int32))
    torch.cuda.synchronize()
    assert out is d
    np.testing.assert_array_equal(out.cpu().numpy(), orc.swap_blocks(src, dst, np.array([[0, 2], [3, 1]])))


def random_mapping(rng, nb, n):
    perm = rng.permutation(nb)
    return np.stack([perm[:n], perm[n:2 * n]], axis=1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.uint8])
def test_paged_caches_every_dtype(dtype):
    rng = np.random.default_rng(1)
    nb, H, D, bs = 48, 4, 64, 16
    x = 16 // torch.empty((), dtype=dtype).element_size()
    layers = 3
    kc = [torch.randint(0, 255, (nb, H, D // x, bs, x), dtype=torch.uint8).to(dtype).cuda() for _ in range(layers)]
    vc = [torch.randint(0, 255, (nb, H, D, bs), dtype=torch.uint8).to(dtype).cuda() for _ in range(layers)]
    k0 = [t.cpu().numpy() if dtype != torch.bfloat16 else t.view(torch.int16).cpu().numpy() for t in kc]
    v0 = [t.cpu().numpy() if dtype != torch.bfloat16 else t.view(torch.int16).cpu().numpy() for t in vc]
    m = random_mapping(rng, nb, 15)
    m = np.concatenate([m, [[nb, 0], [0, nb + 3], [-1, 2]]])  # out of range: skipped
    kernels.copy_blocks(kc, vc, torch.from_numpy(m))
    torch.cuda.synchronize()
    ek, ev = orc.copy_blocks(k0, v0, m)
    for layer in range(layers):
        got_k = kc[layer] if dtype != torch.bfloat16 else kc[layer].view(torch.int16)
        got_v = vc[layer] if dtype != torch.bfloat16 else vc[layer].view(torch.int16)
        np.testing.assert_array_equal(got_k.cpu().numpy(), ek[layer])
        np.testing.assert_array_equal(got_v.cpu().numpy(), ev[layer])


def test_many_pairs_of_32kib_blocks():
    # Llama-3-8B blocks (8 KV heads x D128 x 16 tokens, bf16 = 32 KiB), 2000 pairs, 2 layers.
    rng = np.random.default_rng(2)
    nb = 4100
    g = torch.Generator(device="cuda")
    g.manual_seed(2)
    kc = [torch.randint(-30000, 30000, (nb, 8, 16, 16, 8), generator=g, device="cuda", dtype=torch.int16)
          for _ in range(2)]
    vc = [torch.randint(-30000, 30000, (nb, 8, 128, 16), generator=g, device="cuda", dtype=torch.int16)
          for _ in range(2)]
    k0 = [t.cpu().numpy() for t in kc]
    v0 = [t.cpu().numpy() for t in vc]
    m = random_mapping(rng, nb, 2000)
    kernels.copy_blocks([t.view(torch.bfloat16) for t in kc], [t.view(torch.bfloat16) for t in vc],
                        torch.from_numpy(m).cuda())
    torch.cuda.synchronize()
    ek, ev = orc.copy_blocks(k0, v0, m)
    for layer in range(2):
        np.testing.assert_array_equal(kc[layer].cpu().numpy(), ek[layer])
        np.testing.assert_array_equal(vc[layer].cpu().numpy(), ev[layer])


@pytest.mark.parametrize("direction", ["gpu_to_gpu", "host_to_gpu", "gpu_to_host"])
def test_swap_blocks(direction):
    rng = np.random.default_rng(3)
    src_np = rng.integers(0, 2 ** 15, size=(40, 2, 64, 16), dtype=np.int16)
    dst_np = rng.integers(0, 2 ** 15, size=(30, 2, 64, 16), dtype=np.int16)
    m = np.stack([rng.permutation(40)[:12], rng.permutation(30)[:12]], axis=1)
    m = np.concatenate([m, [[40, 0], [0, 30]]])  # out of range: skipped
    src = torch.from_numpy(src_np)
    dst = torch.from_numpy(dst_np.copy())
    if direction in ("gpu_to_gpu", "gpu_to_host"):
        src = src.cuda()
    if direction in ("gpu_to_gpu", "host_to_gpu"):
        dst = dst.cuda()
    else:
        dst = dst.pin_memory()
    out = kernels.swap_blocks(src, dst, torch.from_numpy(m))
    torch.cuda.synchronize()
    assert out is dst
    np.testing.assert_array_equal(out.cpu().numpy(), orc.swap_blocks(src_np, dst_np, m))
