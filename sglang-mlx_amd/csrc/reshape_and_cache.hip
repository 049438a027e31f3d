// Slot-mapped KV append for gfx950.
//
// Semantics follow the reference kernels reshape_and_cache
// (paged_attention/metal/cache/reshape_and_cache.metal:35-69) and
// reshape_and_cache_flash (:115-136): token i is written to slot
// slot_mapping[i] (block = slot / block_size, offset = slot % block_size);
// negative slots are skipped.  Element conversion is static_cast semantics
// (:9-12): identical types copy bits, float -> f16/bf16 rounds to nearest even.
//
// Two layouts:
//  * paged 5-D: K [nb, H, D/x, bs, x], V [nb, H, D, bs].  One wavefront per
//    (token, head): K leaves as D/x 16-byte chunks at a stride of bs*16 bytes,
//    V as D single elements at a stride of bs elements (the layout makes V
//    token-minor, so its stores cannot be wider than one element).
//  * token-major (MHATokenPool / flash): K and V [num_slots, H, D].  A token's
//    K row and V row are each one contiguous H*D run in both source and
//    destination, so every lane moves 16-byte vectors and every wavefront
//    covers 1 KiB of one row.  Rows of at least 64 vectors go one token per
//    wavefront with nontemporal stores; shorter rows one token per
//    workgroup.
#include "pkv_device.h"
#include "pkv_launch.h"

namespace pkv {

// ---- vector helpers ----------------------------------------------------------
// Load VE elements of type S starting at src (aligned when ALIGNED) and
// convert them to VE elements of type D written to dst.
template <class S, class D, int VE, bool ALIGNED>
__device__ __forceinline__ void convert_run(const typename Elem<S>::storage* __restrict__ src,
                                            typename Elem<D>::storage* __restrict__ dst) {
  if constexpr (ALIGNED && Elem<S>::kBytes == Elem<D>::kBytes && Elem<S>::kBytes * VE == 16 &&
                std::is_same<S, D>::value) {
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
  } else if constexpr (ALIGNED && Elem<D>::kBytes == 2 && Elem<S>::kBytes == 4 && VE == 8) {
    const float4 a = reinterpret_cast<const float4*>(src)[0];
    const float4 b = reinterpret_cast<const float4*>(src)[1];
    uint4 o;
    o.x = pack2(from_f32<D>(a.x), from_f32<D>(a.y));
    o.y = pack2(from_f32<D>(a.z), from_f32<D>(a.w));
    o.z = pack2(from_f32<D>(b.x), from_f32<D>(b.y));
    o.w = pack2(from_f32<D>(b.z), from_f32<D>(b.w));
    *reinterpret_cast<uint4*>(dst) = o;
  } else {
#pragma unroll
    for (int i = 0; i < VE; ++i) dst[i] = convert_elem<S, D>(src[i]);
  }
}

// One 16-byte cache vector (16 / sizeof(CT) elements) read from an aligned
// source run and converted.
template <class S, class D>
__device__ __forceinline__ uint4 load_vec16(const typename Elem<S>::storage* __restrict__ src) {
  constexpr int VE = 16 / Elem<D>::kBytes;
  if constexpr (std::is_same<S, D>::value) {
    return *reinterpret_cast<const uint4*>(src);
  } else {
    typename Elem<D>::storage t[VE];
    convert_run<S, D, VE, true>(src, t);
    return *reinterpret_cast<const uint4*>(t);
  }
}

// ---- paged 5-D layout: one wavefront per (token, head) ------------------------
template <class KT, class CT, bool ALIGNED>
__global__ __launch_bounds__(256) void rac_paged5d_kernel(RacParams p) {
  using KS = typename Elem<KT>::storage;
  using CS = typename Elem<CT>::storage;
  constexpr int X = 16 / Elem<CT>::kBytes;  // elements per 16-byte K chunk
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= p.num_tokens * p.num_heads) return;
  const int64_t tok = wid / p.num_heads;
  const int head = (int)(wid - tok * p.num_heads);
  const int32_t slot = p.slot_mapping[tok];
  if (slot < 0 || (int64_t)slot >= p.num_slots) return;
  const int64_t blk = slot / p.block_size;
  const int off = slot - (int)blk * p.block_size;
  const int D = p.head_size;
  const KS* ksrc = static_cast<const KS*>(p.key) + tok * p.key_stride + (int64_t)head * D;
  const KS* vsrc = static_cast<const KS*>(p.value) + tok * p.value_stride + (int64_t)head * D;
  const int64_t region = ((int64_t)blk * p.num_heads + head) * (int64_t)D * p.block_size;
  CS* kdst = static_cast<CS*>(p.key_cache) + region;    // [D/X][bs][X]
  CS* vdst = static_cast<CS*>(p.value_cache) + region;  // [D][bs]
  const int nchunk = D / X;
  for (int c = lane; c < nchunk; c += 64)
    convert_run<KT, CT, X, ALIGNED>(ksrc + c * X, kdst + ((int64_t)c * p.block_size + off) * X);
  for (int d = lane; d < D; d += 64)
    vdst[(int64_t)d * p.block_size + off] = convert_elem<KT, CT>(vsrc[d]);
}

// ---- token-major layout: one workgroup per token, 16-byte vectors ----------------
template <class KT, class CT, int VE, bool ALIGNED>
__global__ __launch_bounds__(256) void rac_token_major_kernel(RacParams p) {
  using KS = typename Elem<KT>::storage;
  using CS = typename Elem<CT>::storage;
  const int64_t tok = blockIdx.x;
  const int32_t slot = p.slot_mapping[tok];
  if (slot < 0 || (int64_t)slot >= p.num_slots) return;
  const int row = p.num_heads * p.head_size;
  const int nvec = row / VE;  // vectors per K (or V) row
  const KS* ksrc = static_cast<const KS*>(p.key) + tok * p.key_stride;
  const KS* vsrc = static_cast<const KS*>(p.value) + tok * p.value_stride;
  CS* kdst = static_cast<CS*>(p.key_cache) + (int64_t)slot * row;
  CS* vdst = static_cast<CS*>(p.value_cache) + (int64_t)slot * row;
  for (int v = threadIdx.x; v < 2 * nvec; v += blockDim.x) {
    const bool is_v = v >= nvec;
    const int e = (is_v ? v - nvec : v) * VE;
    convert_run<KT, CT, VE, ALIGNED>((is_v ? vsrc : ksrc) + e, (is_v ? vdst : kdst) + e);
  }
}

// ---- token-major layout, wide rows: one wavefront per token -----------------------
// Each lane moves 16-byte cache vectors lane, lane+64, ... of the token's K
// row and V row (NV of each, 64 * NV / 2 < vectors per row <= 64 * NV).  All
// loads are issued, the workgroup's wavefronts meet at a barrier, then all
// store: keeping a CU's reads and writes in separate phases (rather than each
// wavefront storing the moment its loads land) measured ~10% faster on
// MI355X.  The row loads do not wait for the slot id: a padding token's row
// is read and dropped.  The stores are nontemporal: each cache line is
// written once and nothing in this launch reads it back.  (Inactive lanes
// take zeros through a conditional expression; guarding the loads with an
// if-statement instead measured ~15% slower at the same instruction count.)
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

template <class KT, class CT, int NV>
__global__ __launch_bounds__(256) void rac_token_major_wave_kernel(RacParams p) {
  using KS = typename Elem<KT>::storage;
  using CS = typename Elem<CT>::storage;
  constexpr int VE = 16 / Elem<CT>::kBytes;  // elements per 16-byte cache vector
  const int lane = threadIdx.x & 63;
  const int tok = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  // Wavefronts past the last token stay for the barrier and move nothing.
  const bool live = tok < p.num_tokens;
  const int row = p.num_heads * p.head_size;
  const int nvec = row / VE;  // 64 * (NV/2) < nvec <= 64 * NV
  const int32_t slot = live ? p.slot_mapping[tok] : -1;
  const KS* ksrc = static_cast<const KS*>(p.key) + (int64_t)tok * p.key_stride;
  const KS* vsrc = static_cast<const KS*>(p.value) + (int64_t)tok * p.value_stride;
  uint4 kx[NV], vx[NV];
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int i = 64 * c + lane;
    const bool ok = live && i < nvec;
    kx[c] = ok ? load_vec16<KT, CT>(ksrc + i * VE) : make_uint4(0, 0, 0, 0);
    vx[c] = ok ? load_vec16<KT, CT>(vsrc + i * VE) : make_uint4(0, 0, 0, 0);
  }
  __syncthreads();
  if (slot >= 0 && (int64_t)slot < p.num_slots) {
    CS* kdst = static_cast<CS*>(p.key_cache) + (int64_t)slot * row;
    CS* vdst = static_cast<CS*>(p.value_cache) + (int64_t)slot * row;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      const int i = 64 * c + lane;
      if (i < nvec) {
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, kx[c]), reinterpret_cast<u32x4_t*>(kdst + i * VE));
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, vx[c]), reinterpret_cast<u32x4_t*>(vdst + i * VE));
      }
    }
  }
}

// ---- host launchers -----------------------------------------------------------------
template <class KT, class CT>
static hipError_t launch_rac_typed(const RacParams& p, bool aligned, hipStream_t stream) {
  if (p.layout == 0) {
    const int64_t waves = p.num_tokens * p.num_heads;
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (aligned)
      hipLaunchKernelGGL((rac_paged5d_kernel<KT, CT, true>), grid, dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((rac_paged5d_kernel<KT, CT, false>), grid, dim3(256), 0, stream, p);
  } else {
    constexpr int VE = 16 / Elem<CT>::kBytes;
    const int row = p.num_heads * p.head_size;
    const bool vec = aligned && (row % VE == 0);
    int threads = vec ? 2 * (row / VE) : 2 * row;
    threads = threads >= 256 ? 256 : ((threads + 63) / 64) * 64;
    const dim3 grid((unsigned)p.num_tokens);
    // The one-wavefront-per-token kernels index tokens with 32-bit ints.
    const int nvec = (vec && p.num_tokens <= INT32_MAX - 3) ? row / VE : 0;
    const dim3 wgrid((unsigned)((p.num_tokens + 3) / 4));
    if (vec && nvec > 64 && nvec <= 128)
      hipLaunchKernelGGL((rac_token_major_wave_kernel<KT, CT, 2>), wgrid, dim3(256), 0, stream, p);
    else if (vec && nvec > 128 && nvec <= 256)
      hipLaunchKernelGGL((rac_token_major_wave_kernel<KT, CT, 4>), wgrid, dim3(256), 0, stream, p);
    else if (vec && nvec > 256 && nvec <= 512)
      hipLaunchKernelGGL((rac_token_major_wave_kernel<KT, CT, 8>), wgrid, dim3(256), 0, stream, p);
    else if (vec && nvec > 512 && nvec <= 1024)
      hipLaunchKernelGGL((rac_token_major_wave_kernel<KT, CT, 16>), wgrid, dim3(256), 0, stream, p);
    else if (vec)
      hipLaunchKernelGGL((rac_token_major_kernel<KT, CT, VE, true>), grid, dim3(threads), 0, stream, p);
    else
      hipLaunchKernelGGL((rac_token_major_kernel<KT, CT, 1, false>), grid, dim3(threads), 0, stream, p);
  }
  return hipGetLastError();
}

hipError_t launch_reshape_and_cache(const RacParams& p, bool aligned, hipStream_t stream) {
  if (p.num_tokens == 0) return hipSuccess;
  const int kt = p.kv_dtype, ct = p.cache_dtype;
  if (kt == kF32 && ct == kF32) return launch_rac_typed<F32, F32>(p, aligned, stream);
  if (kt == kF16 && ct == kF16) return launch_rac_typed<F16, F16>(p, aligned, stream);
  if (kt == kBF16 && ct == kBF16) return launch_rac_typed<BF16, BF16>(p, aligned, stream);
  if (kt == kF32 && ct == kF16) return launch_rac_typed<F32, F16>(p, aligned, stream);
  if (kt == kF32 && ct == kBF16) return launch_rac_typed<F32, BF16>(p, aligned, stream);
  return hipErrorInvalidValue;
}

}  // namespace pkv
