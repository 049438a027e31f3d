// Element-wise precision conversion with a scale for gfx950: the reference's
// convert_fp8_kernel<SRC_T, DST_T> (paged_attention/metal/convert_fp8.metal:
// 13-47, instantiated for all 16 pairs of float, half, bfloat16 and E4M3
// codes at :58-80), which the reference compiles but never binds.
//
//   E4M3 -> T     : decode(code) * scale, rounded to T
//   T -> E4M3     : encode(float(x) / scale)
//   E4M3 -> E4M3  : encode(decode(code) * scale)
//   T -> U        : float(x) * scale, rounded to U
//
// float -> half rounds to nearest even; float -> bfloat16 rounds to nearest
// even with every NaN becoming 0x7FC0 (the reference's software bfloat); the
// E4M3 codec is pkv_fp8.h.  HBM-bound: each thread converts eight elements per
// step with one vector load and one vector store; the last n % 8 elements (and
// unaligned buffers) take a scalar loop.
#include "pkv_fp8.h"
#include "pkv_launch.h"

namespace pkv {

namespace {
constexpr int kConvThreads = 256;

template <class T> __device__ __forceinline__ float load1(const void* p, int64_t i) {
  return to_f32<T>(static_cast<const typename Elem<T>::storage*>(p)[i]);
}
template <> __device__ __forceinline__ float load1<FP8>(const void* p, int64_t i) {
  const uint32_t c = static_cast<const uint8_t*>(p)[i];
  return f16_bits_to_f32(fp8x4_exact<F16>(c).x & 0xffffu);
}
template <class T> __device__ __forceinline__ void store1(void* p, int64_t i, float v) {
  static_cast<typename Elem<T>::storage*>(p)[i] = from_f32<T>(v);
}
template <> __device__ __forceinline__ void store1<FP8>(void* p, int64_t i, float v) {
  static_cast<uint8_t*>(p)[i] = (uint8_t)fp8_e4m3_encode(v);
}

// Eight consecutive elements starting at element 8*j.
template <class T> struct Vec8;
template <> struct Vec8<F32> {
  static __device__ __forceinline__ void load(const void* p, int64_t j, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[2 * j], b = reinterpret_cast<const float4*>(p)[2 * j + 1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  }
  static __device__ __forceinline__ void store(void* p, int64_t j, const float (&v)[8]) {
    reinterpret_cast<float4*>(p)[2 * j] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[2 * j + 1] = make_float4(v[4], v[5], v[6], v[7]);
  }
};
template <class T> struct Vec8Half {
  static __device__ __forceinline__ void load(const void* p, int64_t j, float (&v)[8]) {
    const uint4 w = reinterpret_cast<const uint4*>(p)[j];
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = to_f32<T>((uint16_t)(u[i] & 0xffffu));
      v[2 * i + 1] = to_f32<T>((uint16_t)(u[i] >> 16));
    }
  }
  static __device__ __forceinline__ void store(void* p, int64_t j, const float (&v)[8]) {
    uint32_t u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = pack2(from_f32<T>(v[2 * i]), from_f32<T>(v[2 * i + 1]));
    reinterpret_cast<uint4*>(p)[j] = make_uint4(u[0], u[1], u[2], u[3]);
  }
};
template <> struct Vec8<F16> : Vec8Half<F16> {};
template <> struct Vec8<BF16> : Vec8Half<BF16> {};
template <> struct Vec8<FP8> {
  static __device__ __forceinline__ void load(const void* p, int64_t j, float (&v)[8]) {
    const uint2 w = reinterpret_cast<const uint2*>(p)[j];
    const uint2 a = fp8x4_exact<F16>(w.x), b = fp8x4_exact<F16>(w.y);
    const uint32_t u[4] = {a.x, a.y, b.x, b.y};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = f16_bits_to_f32(u[i] & 0xffffu);
      v[2 * i + 1] = f16_bits_to_f32(u[i] >> 16);
    }
  }
  static __device__ __forceinline__ void store(void* p, int64_t j, const float (&v)[8]) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo |= fp8_e4m3_encode(v[i]) << (8 * i);
      hi |= fp8_e4m3_encode(v[4 + i]) << (8 * i);
    }
    reinterpret_cast<uint2*>(p)[j] = make_uint2(lo, hi);
  }
};

template <class S, class D> __device__ __forceinline__ float apply_scale(float x, float scale) {
  if constexpr (!std::is_same<S, FP8>::value && std::is_same<D, FP8>::value)
    return __fdiv_rn(x, scale);  // quantisation divides (convert_fp8.metal:33-35)
  else
    return x * scale;
}

template <class S, class D>
__global__ __launch_bounds__(kConvThreads) void convert_kernel(void* dst, const void* src, int64_t n, float scale,
                                                               int vec) {
  const int64_t stride = (int64_t)gridDim.x * kConvThreads;
  const int64_t tid = (int64_t)blockIdx.x * kConvThreads + threadIdx.x;
  int64_t done = 0;
  if (vec) {
    const int64_t n8 = n / 8;
    for (int64_t j = tid; j < n8; j += stride) {
      float v[8];
      Vec8<S>::load(src, j, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = apply_scale<S, D>(v[i], scale);
      Vec8<D>::store(dst, j, v);
    }
    done = n8 * 8;
  }
  for (int64_t i = done + tid; i < n; i += stride) store1<D>(dst, i, apply_scale<S, D>(load1<S>(src, i), scale));
}

template <class S, class D>
hipError_t launch_pair(void* dst, const void* src, int64_t n, float scale, hipStream_t stream) {
  const bool vec = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15u) == 0;
  const int64_t work = vec ? n / 8 + n % 8 : n;
  int64_t blocks = (work + kConvThreads - 1) / kConvThreads;
  if (blocks > 16384) blocks = 16384;  // grid-stride beyond 4M threads
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL((convert_kernel<S, D>), dim3((unsigned)blocks), dim3(kConvThreads), 0, stream, dst, src, n, scale,
                     vec ? 1 : 0);
  return hipGetLastError();
}

template <class S>
hipError_t launch_from(void* dst, const void* src, int64_t n, float scale, int dst_dtype, hipStream_t stream) {
  switch (dst_dtype) {
    case kF32: return launch_pair<S, F32>(dst, src, n, scale, stream);
    case kF16: return launch_pair<S, F16>(dst, src, n, scale, stream);
    case kBF16: return launch_pair<S, BF16>(dst, src, n, scale, stream);
    default: return launch_pair<S, FP8>(dst, src, n, scale, stream);
  }
}
}  // namespace

hipError_t launch_convert_fp8(void* dst, const void* src, int64_t n, float scale, int src_dtype, int dst_dtype,
                              hipStream_t stream) {
  if (n == 0) return hipSuccess;
  switch (src_dtype) {
    case kF32: return launch_from<F32>(dst, src, n, scale, dst_dtype, stream);
    case kF16: return launch_from<F16>(dst, src, n, scale, dst_dtype, stream);
    case kBF16: return launch_from<BF16>(dst, src, n, scale, dst_dtype, stream);
    default: return launch_from<FP8>(dst, src, n, scale, dst_dtype, stream);
  }
}

}  // namespace pkv
