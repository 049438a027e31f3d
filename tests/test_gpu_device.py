"""Device-attribute entry points (mlx_device.cpp:12-20, bindings.cpp:125-133):
get_max_shared_memory_per_block_device_attribute and get_device_attribute,
through the C-ABI, against torch's own view of the device and against the
LDS the decode kernels allocate."""

import ctypes
import re
import subprocess

import pytest
import torch

from sglang_mlx_amd import _ext, _lib

pytestmark = pytest.mark.gpu

# hipDeviceAttribute_t values of ROCm 7.2 (hip/hip_runtime_api.h).
HIP_ATTR_MULTIPROCESSOR_COUNT = 63
HIP_ATTR_MAX_SHARED_MEMORY_PER_BLOCK = 74
HIP_ATTR_WARP_SIZE = 87


class FuncAttributes(ctypes.Structure):
    """hipFuncAttributes (hip/hip_runtime_api.h of ROCm 7.2)."""
    _fields_ = [("binaryVersion", ctypes.c_int), ("cacheModeCA", ctypes.c_int),
                ("constSizeBytes", ctypes.c_size_t), ("localSizeBytes", ctypes.c_size_t),
                ("maxDynamicSharedSizeBytes", ctypes.c_int), ("maxThreadsPerBlock", ctypes.c_int),
                ("numRegs", ctypes.c_int), ("preferredShmemCarveout", ctypes.c_int), ("ptxVersion", ctypes.c_int),
                ("sharedSizeBytes", ctypes.c_size_t)]


def kernel_attributes():
    """{kernel symbol: hipFuncAttributes} for every kernel of the library, read
    from the HIP runtime with the kernel handles the library exports."""
    names = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                           check=True).stdout
    kernels = sorted({m.group(1) for m in re.finditer(r" V (_ZN3pkv\w*kernel\w*)", names)})
    lib = _lib.lib()
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipFuncGetAttributes.restype = ctypes.c_int
    hip.hipFuncGetAttributes.argtypes = [ctypes.POINTER(FuncAttributes), ctypes.c_void_p]
    out = {}
    for k in kernels:
        attr = FuncAttributes()
        handle = ctypes.cast(getattr(lib, k), ctypes.c_void_p).value
        assert hip.hipFuncGetAttributes(ctypes.byref(attr), handle) == 0, k
        out[k] = attr
    return out


def test_max_shared_memory_per_block():
    lds = _ext.get_max_shared_memory_per_block_device_attribute()
    assert lds == _ext.get_device_attribute(HIP_ATTR_MAX_SHARED_MEMORY_PER_BLOCK)
    assert lds == _ext.get_max_shared_memory_per_block_device_attribute(0)
    assert lds == 160 * 1024              # MI355X: 160 KiB per workgroup


def test_kernels_fit_lds_and_do_not_spill():
    # Every kernel's static LDS, as the runtime reports it, fits a workgroup;
    # the decode kernels of the hot path (16-bit queries at head sizes up to
    # 128: the persistent kernel in both its layouts, the grouped kernel,
    # the cascade and the partition kernel) keep their registers out of
    # scratch.  (Float32 queries and head sizes 192/256 do spill: 48-68
    # bytes in the grouped kernel, up to 284 in the float32 D256 kernels.)
    lds = _ext.get_max_shared_memory_per_block_device_attribute()
    attrs = kernel_attributes()
    assert len(attrs) > 100
    for k, a in attrs.items():
        assert a.sharedSizeBytes <= lds, (k, a.sharedSizeBytes)
    hot = [k for k in attrs if re.search(r"(persist|group|cascade|part)_kernelINS_(4BF16|3F16)E", k)
           and not re.search(r"Li(192|256)E", k)]
    assert any("persist" in k and "Li128ELi0E" in k for k in hot)  # the token-row variant is covered
    assert any("group_kernel" in k for k in hot) and any("cascade_kernel" in k for k in hot)
    for k in hot:
        # The grouped kernel over 16-bit caches at head sizes 120/128 keeps
        # two values of its item prologue in 12 bytes of scratch (stored and
        # reloaded once per item, outside the tile loop).  FP8 kernels call
        # the out-of-line fix-up of exponent-15 codes, and a call may reserve
        # a small frame that no instruction of theirs touches.
        limit = 16 if "group_kernel" in k else 0
        if "ENS_3FP8E" in k:
            limit = max(limit, 64)
        assert attrs[k].localSizeBytes <= limit, (k, attrs[k].localSizeBytes)


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
