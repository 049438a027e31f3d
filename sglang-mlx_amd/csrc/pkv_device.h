// Device helpers shared by the gfx950 paged-KV kernels: element-type traits,
// bit-exact conversions, wave64 cross-row reductions and MFMA wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pkv {

// ---------------------------------------------------------------------------
// Element types.  Caches are stored as raw 16/32-bit words; the tag types
// select conversions and MFMA flavours at compile time.
// ---------------------------------------------------------------------------
struct F32 {};
struct F16 {};
struct BF16 {};
struct FP8 {};  // E4M3 codes in the reference's format (float8.metal:13-38)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <class T> struct Elem;
template <> struct Elem<F32> {
  using storage = float;
  static constexpr int kBytes = 4;
};
template <> struct Elem<F16> {
  using storage = uint16_t;
  static constexpr int kBytes = 2;
};
template <> struct Elem<BF16> {
  using storage = uint16_t;
  static constexpr int kBytes = 2;
};
template <> struct Elem<FP8> {
  using storage = uint8_t;
  static constexpr int kBytes = 1;
};

// ---- scalar conversions ---------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}
// float -> bf16, round to nearest even; every NaN becomes 0x7FC0.
// (The rule of the reference's software bfloat, utils.metal:21-35.)
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
// float -> fp16 with the hardware conversion (round to nearest even).
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
// float -> fp16 of a value computed in float, rounded twice as written: the
// empty asm keeps the compiler from fusing the producing multiply and this
// conversion into v_fma_mixlo_f16 (a * b + 0), which rounds once and turns
// -0 products into +0.
__device__ __forceinline__ uint32_t f32_to_f16_bits_unfused(float f) {
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <class T> __device__ __forceinline__ float to_f32(typename Elem<T>::storage v);
template <> __device__ __forceinline__ float to_f32<F32>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<F16>(uint16_t v) { return f16_bits_to_f32(v); }
template <> __device__ __forceinline__ float to_f32<BF16>(uint16_t v) { return bf16_bits_to_f32(v); }

template <class T> __device__ __forceinline__ typename Elem<T>::storage from_f32(float v);
template <> __device__ __forceinline__ float from_f32<F32>(float v) { return v; }
template <> __device__ __forceinline__ uint16_t from_f32<F16>(float v) {
  return (uint16_t)f32_to_f16_bits_unfused(v);
}
template <> __device__ __forceinline__ uint16_t from_f32<BF16>(float v) { return (uint16_t)f32_to_bf16_bits(v); }

// Element conversion used by the append: identical types copy bits, other
// pairs go through float (static_cast semantics, reshape_and_cache.metal:9-12).
template <class S, class D>
__device__ __forceinline__ typename Elem<D>::storage convert_elem(typename Elem<S>::storage v) {
  return from_f32<D>(to_f32<S>(v));
}
template <> __device__ __forceinline__ uint16_t convert_elem<F16, F16>(uint16_t v) { return v; }
template <> __device__ __forceinline__ uint16_t convert_elem<BF16, BF16>(uint16_t v) { return v; }
template <> __device__ __forceinline__ float convert_elem<F32, F32>(float v) { return v; }

// Pack two 16-bit words.
__device__ __forceinline__ uint32_t pack2(uint32_t lo, uint32_t hi) { return (lo & 0xffffu) | (hi << 16); }

// ---------------------------------------------------------------------------
// Wave64 reductions across the four 16-lane rows that share a column
// (lanes l, l^16, l^32, l^48).  gfx950's v_permlane16_swap / v_permlane32_swap
// exchange whole rows between two VGPRs on the VALU; called with the same
// value in both operands, the two results hold {x_l, x_partner} in either
// order, so a commutative op over them is the xor-16 / xor-32 all-reduce.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float xchg16_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xchg32_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xchg16_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xchg32_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float column_max(float x) { return xchg32_max(xchg16_max(x)); }
__device__ __forceinline__ float column_sum(float x) { return xchg32_sum(xchg16_sum(x)); }

// ---------------------------------------------------------------------------
// MFMA wrappers for 16-bit cache types.
//   mma_k32: D[16x16] += A[16x32] * B[32x16]; lane l supplies A[l%16][k-group
//            l/16] and B[k-group l/16][l%16] as 8 elements (16 bytes).
//   mma_k16: D[16x16] += A[16x16] * B[16x16]; 4 elements (8 bytes) per lane.
//   Output: lane l, register r holds D[4*(l/16) + r][l%16].
// Operands travel as raw bit vectors (uint4 / uint2).
// ---------------------------------------------------------------------------
template <class T> struct Mma;
template <> struct Mma<BF16> {
  static __device__ __forceinline__ f32x4 k32(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 k16(uint2 a, uint2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4, a),
                                                     __builtin_bit_cast(bf16x4, b), c, 0, 0, 0);
  }
};
template <> struct Mma<F16> {
  static __device__ __forceinline__ f32x4 k32(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 k16(uint2 a, uint2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
};

}  // namespace pkv
