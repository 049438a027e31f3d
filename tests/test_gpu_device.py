"""Device-attribute entry points (mlx_device.cpp:12-20, bindings.cpp:125-133):
get_max_shared_memory_per_block_device_attribute and get_device_attribute,
through the C-ABI, against torch's own view of the device and against the
LDS the decode kernels allocate."""

import pytest
import torch

from sglang_mlx_amd import _ext

pytestmark = pytest.mark.gpu

# hipDeviceAttribute_t values of ROCm 7.2 (hip/hip_runtime_api.h).
HIP_ATTR_MULTIPROCESSOR_COUNT = 63
HIP_ATTR_MAX_SHARED_MEMORY_PER_BLOCK = 74
HIP_ATTR_WARP_SIZE = 87

# LDS of the persistent decode kernel at head size 128 with 8 wavefronts:
# double-buffered float4 merge tiles [2][8][8][64], (max, sum) [2][2][8][16]
# floats, and the longest-first order (1024 context lengths + 1024 ranks).
PERSIST_LDS_BYTES = 2 * 8 * 8 * 64 * 16 + 2 * 2 * 8 * 16 * 4 + 1024 * 4 + 1024 * 4


def test_max_shared_memory_per_block():
    lds = _ext.get_max_shared_memory_per_block_device_attribute()
    assert lds == _ext.get_device_attribute(HIP_ATTR_MAX_SHARED_MEMORY_PER_BLOCK)
    assert lds == _ext.get_max_shared_memory_per_block_device_attribute(0)
    assert PERSIST_LDS_BYTES == 141_312
    assert lds >= PERSIST_LDS_BYTES       # MI355X: 160 KiB per workgroup


def test_device_attribute_matches_torch():
    props = torch.cuda.get_device_properties(0)
    assert _ext.get_device_attribute(HIP_ATTR_MULTIPROCESSOR_COUNT) == props.multi_processor_count
    assert _ext.get_device_attribute(HIP_ATTR_WARP_SIZE, 0) == 64


def test_bad_device_raises_runtime_error():
    with pytest.raises(RuntimeError, match="hipDeviceGetAttribute"):
        _ext.get_device_attribute(HIP_ATTR_MULTIPROCESSOR_COUNT, torch.cuda.device_count() + 3)
    with pytest.raises(RuntimeError, match="hipDeviceGetAttribute"):
        _ext.get_max_shared_memory_per_block_device_attribute(torch.cuda.device_count() + 3)
    # The failed query leaves no pending HIP error behind: the library's
    # next launch and torch's next kernel both succeed.
    src = torch.arange(64, dtype=torch.float32, device="cuda")
    dst = torch.empty(64, dtype=torch.uint8, device="cuda")
    _ext.convert_fp8(dst, src, 1.0)
    y = src * 2
    torch.cuda.synchronize()
    assert y[5].item() == 10.0 and dst[1].item() == 0x38   # 1.0 in E4M3


def test_launch_status_ignores_an_earlier_pending_error():
    # A HIP call outside the library fails and leaves its error pending; the
    # library's next launch reports its own success and leaves nothing
    # pending for torch.  (HIP is opened by its soname, so this is the
    # runtime torch already loaded, not a second copy.)
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so.7")
    src = torch.ones(64, dtype=torch.float32, device="cuda")
    dst = torch.empty(64, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    n = ctypes.c_int(0)
    assert hip.hipDeviceGetAttribute(ctypes.byref(n), HIP_ATTR_MULTIPROCESSOR_COUNT,
                                     torch.cuda.device_count() + 3) != 0
    _ext.convert_fp8(dst, src, 1.0)
    y = src + 1
    torch.cuda.synchronize()
    assert (dst == 0x38).all() and (y == 2).all()
