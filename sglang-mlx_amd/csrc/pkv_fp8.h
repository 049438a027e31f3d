// FP8 E4M3 codec of the reference (paged_attention/metal/float8.metal) for
// gfx950.
//
// Format: sign, 4 exponent bits (bias 7), 3 mantissa bits; exponent 0 is
// zero / subnormal (m/8 * 2^-6), exponent 15 is +-inf (m = 0) or NaN -- an
// IEEE-style format, not OCP E4M3FN.  The two agree on every code whose
// exponent is below 15, which is what gfx950's conversion instructions
// decode; the 14 codes with exponent 15 and a nonzero mantissa below 7 (and
// the two infinities) are fixed up in software where they occur.
//
// The encoder restates detail::fp32_to_fp8<4, 3, 7> (float8.metal:72-120)
// step by step, including its behaviour away from the normal range: values
// with 256 <= |x| < 2^14 take its subnormal branch and keep three low bits
// of a shifted significand (256 encodes as +0), subnormals round half up,
// and a value that rounds up to 2^-6 wraps to +-0.  For |x| >= 2^14 the
// reference's shift counts are out of range (undefined); this encoder
// returns +-inf there, the value of the reference's overflow branch.
#pragma once

#include "pkv_device.h"

namespace pkv {

// float -> E4M3 code (low 8 bits).
__device__ __forceinline__ uint32_t fp8_e4m3_encode(float f) {
  const uint32_t bits = __float_as_uint(f);
  const uint32_t s = (bits >> 31) << 7;
  const uint32_t a = bits & 0x7fffffffu;
  if (a >= 0x7f800000u) return s | 0x78u | (a != 0x7f800000u ? 1u : 0u);  // inf, NaN (:80-83)
  const int e8 = (int)(a >> 23) - 120;  // biased fp8 exponent: (e - 127) + 7
  const uint32_t m = a & 0x7fffffu;
  if (e8 >= 21) return s | 0x78u;  // reference undefined here (see above)
  if (e8 >= 1 && e8 <= 14) {       // normal: round to nearest even (:91-104)
    uint32_t mant = m >> 20;
    const uint32_t rnd = (m >> 19) & 1u;
    const uint32_t sticky = (m & 0x7ffffu) != 0u ? 1u : 0u;
    mant += rnd & (sticky | (mant & 1u));
    int e = e8;
    if (mant >> 3) {
      mant = 0;
      if (++e > 14) return s | 0x78u;
    }
    return s | ((uint32_t)e << 3) | (mant & 7u);
  }
  if (e8 < -2) return s;                  // (:108-109)
  const int rshift = (1 - e8) + 20;       // 1 .. 23 for e8 in [-2, 20]
  const uint32_t full = 0x800000u | m;    // (:111-118)
  const uint32_t rounded = (full + (1u << (rshift - 1))) >> rshift;
  return rounded == 0u ? s : (s | (rounded & 7u));
}

// Nonzero iff one of the four codes in w has exponent 15: masking leaves at
// most 0x78 per byte and adding 8 carries into bit 7 exactly for 0x78.
__device__ __forceinline__ uint32_t fp8x4_special(uint32_t w) {
  return ((w & 0x78787878u) + 0x08080808u) & 0x80808080u;
}

// Four codes (byte i = element i) -> four 16-bit values of MT (BF16 or F16),
// as (elements 0,1 | elements 2,3).  Exact for every code: E4M3 values are
// representable in both types.  The fast form is the hardware conversion,
// right for all codes with exponent below 15; fp8x4_fix corrects the others.
template <class MT> __device__ __forceinline__ uint2 fp8x4_cvt(uint32_t w);
template <> __device__ __forceinline__ uint2 fp8x4_cvt<BF16>(uint32_t w) {
  return make_uint2(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)));
}
template <> __device__ __forceinline__ uint2 fp8x4_cvt<F16>(uint32_t w) {
  return make_uint2(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true)));
}

template <class MT> struct Special16;
template <> struct Special16<BF16> {
  static constexpr uint32_t kInf = 0x7f80u, kNaN = 0x7fc0u;
};
template <> struct Special16<F16> {
  static constexpr uint32_t kInf = 0x7c00u, kNaN = 0x7e00u;
};

// Exponent-15 codes -> +-inf (mantissa 0) or the unsigned NaN the
// reference's decoder returns (float8.metal:27-31).
template <class MT> __device__ __noinline__ uint2 fp8x4_fix(uint32_t w, uint2 r) {
  uint32_t h[4] = {r.x & 0xffffu, r.x >> 16, r.y & 0xffffu, r.y >> 16};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t c = (w >> (8 * i)) & 0xffu;
    if (((c >> 3) & 15u) == 15u)
      h[i] = (c & 7u) ? Special16<MT>::kNaN : (Special16<MT>::kInf | ((c & 0x80u) << 8));
  }
  return make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
}

template <class MT> __device__ __forceinline__ uint2 fp8x4_exact(uint32_t w) {
  uint2 r = fp8x4_cvt<MT>(w);
  if (fp8x4_special(w)) r = fp8x4_fix<MT>(w, r);
  return r;
}

// fp8x4_exact without the out-of-line fix-up (selects instead of a call),
// for code that holds many values live where the call would make the
// compiler save them to scratch.
template <class MT> __device__ __forceinline__ uint2 fp8x4_exact_inline(uint32_t w) {
  const uint2 r = fp8x4_cvt<MT>(w);
  uint32_t h[4] = {r.x & 0xffffu, r.x >> 16, r.y & 0xffffu, r.y >> 16};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t c = (w >> (8 * i)) & 0xffu;
    const uint32_t fix = (c & 7u) ? Special16<MT>::kNaN : (Special16<MT>::kInf | ((c & 0x80u) << 8));
    h[i] = ((c >> 3) & 15u) == 15u ? fix : h[i];
  }
  return make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
}

}  // namespace pkv
