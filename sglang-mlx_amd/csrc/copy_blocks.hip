// Whole-block copies between paged caches for gfx950.
//
// Semantics follow the reference kernels copy_blocks and swap_blocks
// (paged_attention/metal/cache/copy_blocks.metal:9-39, :55-70; host side
// paged_attention/mlx_cache.cpp:302-370): for every (src, dst) pair of the
// block mapping, block dst of the destination plane receives block src of the
// source plane; a block is block_bytes contiguous bytes, so every cache layout
// and dtype is the same byte copy.  copy_blocks passes each layer's K and V as
// planes that are their own source; swap_blocks passes one (src, dst) pair.
//
// One launch covers up to kMaxCopyPlanes planes.  The grid is flat: workgroup
// x handles one 16 KiB chunk (256 lanes x 4 vectors of 16 bytes) of one pair,
// z is the plane.  Each lane issues its four loads before its four stores.
// Pairs whose block ids fall outside the planes are skipped (the reference
// does not check them).
#include "pkv_device.h"
#include "pkv_launch.h"

namespace pkv {

namespace {
constexpr int kCopyThreads = 256;
constexpr int kCopyVecs = 4;  // 16-byte vectors per lane per chunk
constexpr int64_t kChunkBytes = (int64_t)kCopyThreads * kCopyVecs * 16;
}  // namespace

template <bool VEC>
__global__ __launch_bounds__(kCopyThreads) void copy_blocks_kernel(BlockCopyParams p) {
  const int64_t chunks = VEC ? (p.block_bytes + kChunkBytes - 1) / kChunkBytes
                             : (p.block_bytes + kCopyThreads - 1) / kCopyThreads;
  const int64_t pair = (int64_t)blockIdx.x / chunks;
  const int64_t chunk = (int64_t)blockIdx.x - pair * chunks;
  const int plane = blockIdx.z;
  const int64_t s = p.mapping[2 * pair];
  const int64_t d = p.mapping[2 * pair + 1];
  if (s < 0 || s >= p.src_blocks || d < 0 || d >= p.dst_blocks) return;
  const char* src = p.src[plane] + s * p.block_bytes;
  char* dst = p.dst[plane] + d * p.block_bytes;
  if constexpr (VEC) {
    const int64_t nvec = p.block_bytes / 16;
    const int64_t v0 = chunk * (kCopyThreads * kCopyVecs) + threadIdx.x;
    uint4 x[kCopyVecs];
#pragma unroll
    for (int u = 0; u < kCopyVecs; ++u) {
      const int64_t v = v0 + (int64_t)u * kCopyThreads;
      x[u] = v < nvec ? reinterpret_cast<const uint4*>(src)[v] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kCopyVecs; ++u) {
      const int64_t v = v0 + (int64_t)u * kCopyThreads;
      if (v < nvec) reinterpret_cast<uint4*>(dst)[v] = x[u];
    }
  } else {
    const int64_t i = chunk * kCopyThreads + threadIdx.x;
    if (i < p.block_bytes) dst[i] = src[i];
  }
}

hipError_t launch_copy_blocks(const BlockCopyParams& p, bool aligned, hipStream_t stream) {
  if (p.num_pairs == 0 || p.num_planes == 0 || p.block_bytes == 0) return hipSuccess;
  const bool vec = aligned && p.block_bytes % 16 == 0;
  const int64_t chunks = vec ? (p.block_bytes + kChunkBytes - 1) / kChunkBytes
                             : (p.block_bytes + kCopyThreads - 1) / kCopyThreads;
  const dim3 grid((unsigned)(p.num_pairs * chunks), 1, (unsigned)p.num_planes);
  if (vec)
    hipLaunchKernelGGL(copy_blocks_kernel<true>, grid, dim3(kCopyThreads), 0, stream, p);
  else
    hipLaunchKernelGGL(copy_blocks_kernel<false>, grid, dim3(kCopyThreads), 0, stream, p);
  return hipGetLastError();
}

int64_t copy_blocks_max_grid_pairs(int64_t block_bytes, bool aligned) {
  const bool vec = aligned && block_bytes % 16 == 0;
  const int64_t chunks = vec ? (block_bytes + kChunkBytes - 1) / kChunkBytes
                             : (block_bytes + kCopyThreads - 1) / kCopyThreads;
  // HIP bounds a launch to 2^32 work-items.
  return (((int64_t)1 << 32) / kCopyThreads - 1) / (chunks > 0 ? chunks : 1);
}

}  // namespace pkv
