// Block-table decode attention for gfx950 (paged 5-D KV layout).
//
// Semantics: paged_attention_kernels.metal:37-168 of the reference --
// per (sequence s, query head h), softmax over the first ctx tokens of
// scale * q.k (+ alibi[h] * (t - ctx + 1)), weighted sum of V, denominator
// (sum + 1e-6), fp32 accumulation, zero output when ctx == 0 or
// ctx > max_seq_len.  GQA: kv_head = h / (Hq / Hkv).
//
// Two kernels, no communication between workgroups inside a launch:
//
// paged_decode_part_kernel -- one workgroup (4 wavefronts) per
//   (partition, sequence, unit), unit = (KV head, slice of at most 16 query
//   heads of its GQA group).  The unit index varies fastest, so with 8 KV
//   heads consecutive workgroups -- which the dispatcher spreads over the 8
//   XCDs -- put each KV head on one XCD and its L2.  Wavefront w handles
//   16-token tiles w, w+4, ... of the partition.  Per tile it computes
//   S^T[16 tok x 16 heads] with v_mfma_f32_16x16x32_{bf16,f16}: the A operand
//   is the K tile straight from HBM -- in the paged 5-D layout, lane l reading
//   the 16 bytes at (64*j + l) * 16 of a (block, head) region is exactly row
//   l%16, k-group l/16 of k-step j, so each k-step is one contiguous 1 KiB
//   load -- and the B operand is the query group, held in registers for the
//   whole partition.  The output layout of that MFMA (lane l, register r =
//   token 4*(l/16)+r, head l%16) is the B-operand layout of
//   v_mfma_f32_16x16x16, so the softmax probabilities feed P*V without
//   leaving registers; V^T tiles are 8-byte loads of 4 consecutive tokens of
//   one dimension (contiguous in the V layout).  The next tile's K and V are
//   loaded before the current tile is consumed (two register sets), so every
//   wavefront keeps 8 KiB of loads in flight while it computes.  Softmax runs
//   online in the log2 domain.  A sequence that fits in one partition gets
//   its output row directly; otherwise the partition's (max, sum) and
//   normalised output go to the fp32 workspace.
//
// paged_decode_reduce_kernel -- one wavefront per (sequence, query head) of a
//   sequence with more than one partition: log-sum-exp merge of the
//   partitions, M = max m_p, w_p = l_p * 2^(m_p - M),
//   out = sum_p w_p o_p / (sum_p w_p + 1e-6).
//
// The split is invisible in the result: sum_p w_p equals the single-pass
// softmax denominator, so the merge is an algebraic identity with the
// reference's single softmax.
#pragma once

#include <algorithm>

#include "pkv_fp8.h"
#include "pkv_launch.h"

namespace pkv {

// Wavefronts per workgroup of the partition kernel (8 measured slower at the
// long-context configurations: fewer resident workgroups per CU).
constexpr int kPartWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Two probabilities -> packed 16-bit MFMA operand word (hardware
// round-to-nearest-even conversions; probabilities are never NaN).
template <class CT> __device__ __forceinline__ uint32_t pack_p(float a, float b);
template <> __device__ __forceinline__ uint32_t pack_p<BF16>(float a, float b) {
  // One v_cvt_pk_bf16_f32 (round to nearest even, as the scalar conversion).
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
template <> __device__ __forceinline__ uint32_t pack_p<F16>(float a, float b) {
  return pack2(__builtin_bit_cast(uint16_t, (_Float16)a), __builtin_bit_cast(uint16_t, (_Float16)b));
}

// 2^x with the hardware v_exp_f32 (results below 2^-126 flush to zero, which
// no softmax weight here can notice: the largest weight of a row is >= 1).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The running maximum of a softmax row is only raised when a new score
// exceeds it by more than this (log2 units): weights 2^(s - m) then stay
// below 2^8, and the rescale of the accumulators is skipped for almost every
// tile.  Any reference maximum gives the same normalised result.
constexpr float kRescaleSlack = 8.f;

// Tile buffers per wavefront where the register budget allows four (see
// Prefetch), and of the partition kernel (two: fewer registers, more
// resident workgroups per CU, measured 1-4% faster than three or four at
// 32K-128K contexts).
constexpr int kMaxBuffers = 4;
constexpr int kPartBuffers = 2;
// The one-sequence persistent kernel is used from one (sequence, unit) item
// per resident workgroup, where the longest-first order gives the longest
// items a workgroup of their own.  (From two, the Llama-3-8B layer at 48 and
// 63 sequences fell to the partition kernel: 97.3 and 109.2 us against 76.6
// and 95.9 us persistent.)
constexpr int kPersistMinItemsPerWorkgroup = 1;

// Query element pair -> (hi, lo) words of the cache type; q = hi + lo to
// within 2^-16 relative, so a float32 query keeps its precision through the
// 16-bit MFMA (two MFMAs per k-step).
template <class CT> __device__ __forceinline__ void split_q(float x, uint32_t& hi, uint32_t& lo);
template <> __device__ __forceinline__ void split_q<BF16>(float x, uint32_t& hi, uint32_t& lo) {
  hi = f32_to_bf16_bits(x);
  lo = f32_to_bf16_bits(x - bf16_bits_to_f32(hi));
}
template <> __device__ __forceinline__ void split_q<F16>(float x, uint32_t& hi, uint32_t& lo) {
  hi = f32_to_f16_bits(x);
  lo = f32_to_f16_bits(x - f16_bits_to_f32(hi));
}

// MFMA operand type of a (query, cache) type pair: the cache type, or for
// FP8 caches the query's 16-bit type (E4M3 values are exact in both) and
// float16 for a float32 query (more mantissa for its hi/lo split).
template <class QT, class CT> struct MmaOf { using type = CT; };
template <class QT> struct MmaOf<QT, FP8> {
  using type = std::conditional_t<std::is_same<QT, BF16>::value, BF16, F16>;
};

// One wavefront's 16-token tile in registers, as MFMA operands.
template <int D, bool F8 = false> struct Tile {
  static constexpr int KSTEPS = (D + 31) / 32;  // 16x16x32 k-steps over the head dimension
  static constexpr int DT = (D + 15) / 16;      // 16-wide dimension tiles of the output
  uint4 k[KSTEPS];
  uint2 v[DT];
  int kpb;  // block of this lane's K row (token tt0 + col), -1 if masked out
  int vpb;  // block of this lane's 4 V tokens, -1 if masked out
};
// FP8 caches: the tile arrives as raw codes (8 K codes per k-step, 4 V codes
// per dimension tile: half the bytes of a 16-bit tile, the same number of
// loads) and is dequantised into k / v when consumed.
template <int D> struct Tile<D, true> : Tile<D, false> {
  uint2 k8[Tile<D, false>::KSTEPS];
  uint32_t v8[Tile<D, false>::DT];
};

// FP8 tiles at head sizes that are multiples of 64 are loaded wide: 16 K
// codes and 8 V codes per lane and load, half the load instructions of the
// 8- and 4-byte form (which measured 77 us at the Llama-3-8B layer against
// 66 us wide, loads alone).  Lane g then holds K chunks g, g+4, ... (16
// dims each) of its token, so k-step j's eight dims of lane g are
// 64(j/2) + 16g + 8(j%2) .. +7 instead of 32j + 8g; the query operand takes
// the same dims (the dot product is a sum over d, so any order of d that K
// and Q share gives the same scores).
template <class CT, int D> struct WideFp8 {
  static constexpr bool value = std::is_same<CT, FP8>::value && D % 64 == 0;
};
// First of the eight head dims lane g holds in k-step j.
template <bool WIDE> __device__ __forceinline__ constexpr int kstep_dim0(int j, int g) {
  return WIDE ? 64 * (j >> 1) + 16 * g + 8 * (j & 1) : 32 * j + 8 * g;
}

// Register sets per wavefront (tiles in flight + 1), as many as leave room
// for occupancy 2: four for a 16-bit query, head size 128 or below 120 and
// blocks of 16 or 32 tokens (each CU then keeps 8 wavefronts x 24 KiB of
// loads in flight); three where a float32 query (hi/lo split), per-lane
// block ids (8-token blocks) or D = 120 need the registers; two above 128
// and for a float32 query with 8-token blocks at D >= 120.
template <class QT, int D, int BS> struct Prefetch {
  static constexpr bool kF32 = std::is_same<QT, F32>::value;
  static constexpr bool kTight = kF32 || BS < kTile || D == 120;
  static constexpr int kBuffers = (D > 128 || (kF32 && BS < kTile && D >= 120)) ? 2 : kTight ? 3 : kMaxBuffers;
};

// Word 3 of a raw (stride 0) buffer resource on gfx9-family GPUs.
constexpr int kBufferRsrcWord3 = 0x00020000;

// Issues the loads of the tile of tokens tt0 .. tt0+15; b0 is the block of
// tokens tt0 .. tt0+7 and b1 the block of tokens tt0+8 .. tt0+15 (-1 =
// masked out; equal when block_size >= 16).  Both are wave-uniform.
//
// With block_size >= 16 the tile lies in one block: the (block, head)
// regions of K and V become buffer resources in SGPRs, sized to the region
// (D * block_size elements), and every lane loads at a fixed offset into
// them.  No per-tile vector address arithmetic remains, the hardware range
// check returns zero for anything outside the region, and a masked-out block
// gets a zero-sized resource, so its loads return zero without touching
// memory.
//
// With 8-token blocks each half of the tile has its own block; lanes then
// address memory directly, and masked-out blocks read block 0 instead (in
// bounds) and are discarded by the caller.  In both cases the number of
// loads per tile is fixed, so the next tiles' loads stay in flight while the
// current one is consumed.
template <int D, int BS, int CPOL = 0>
__device__ __forceinline__ void load_tile(Tile<D>& t, const uint16_t* kbase, const uint16_t* vbase,
                                          int64_t k_block_stride, int64_t v_block_stride, int b0, int b1, int tt0,
                                          int g, int col) {
  if constexpr (BS >= kTile) {
    const int b = b0;
    t.kpb = t.vpb = b;
    const int off = tt0 % BS;
    const int64_t bb = b < 0 ? 0 : b;
    const int bytes = b < 0 ? 0 : D * BS * 2;
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(kbase + bb * k_block_stride), (short)0, bytes, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(vbase + bb * v_block_stride), (short)0, bytes, kBufferRsrcWord3);
    // K region [D/8][BS][8]: lane (g, col), k-step j reads chunk 4j+g of
    // token off+col.  V region [D][BS]: lane (g, col), dimension tile dt
    // reads tokens off+4g .. +3 of dimension 16*dt + col.  The lane part of
    // each offset is loop-invariant; the token offset within the block is
    // wave-uniform and goes into the scalar offset.
    const int ko = (col * 8 + g * (BS * 8)) * 2;
    const int vo = (4 * g + col * BS) * 2;
#pragma unroll
    for (int j = 0; j < Tile<D>::KSTEPS; ++j)
      t.k[j] = __builtin_bit_cast(uint4,
                                  __builtin_amdgcn_raw_buffer_load_b128(kr, ko + j * (4 * BS * 16), off * 16, CPOL));
#pragma unroll
    for (int dt = 0; dt < Tile<D>::DT; ++dt)
      t.v[dt] = __builtin_bit_cast(uint2,
                                   __builtin_amdgcn_raw_buffer_load_b64(vr, vo + dt * (16 * BS * 2), off * 2, CPOL));
  } else {
    constexpr int NCHUNK = D / 8;  // 16-byte K chunks per token
    const int kpb = col < 8 ? b0 : b1;  // K row = token tt0 + col
    t.kpb = kpb;
    const uint16_t* kp = kbase + (int64_t)(kpb < 0 ? 0 : kpb) * k_block_stride + (col % BS) * 8;
    const int vpb = g < 2 ? b0 : b1;     // V tokens tt0 + 4g .. +3
    t.vpb = vpb;
    const uint16_t* vp = vbase + (int64_t)(vpb < 0 ? 0 : vpb) * v_block_stride + ((4 * g) % BS);
#pragma unroll
    for (int j = 0; j < Tile<D>::KSTEPS; ++j) {
      const int c = 4 * j + g;
      if (NCHUNK % 4 == 0 || c < NCHUNK)
        t.k[j] = *reinterpret_cast<const uint4*>(kp + c * (BS * 8));
      else
        t.k[j] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int dt = 0; dt < Tile<D>::DT; ++dt) {
      const int d = 16 * dt + col;
      if (D % 16 == 0 || d < D)
        t.v[dt] = *reinterpret_cast<const uint2*>(vp + d * BS);
      else
        t.v[dt] = make_uint2(0, 0);
    }
  }
}

// load_tile for FP8 caches in the paged 5-D layout with x = 16: K [D/16][bs][16]
// bytes, V [D][bs] bytes per (block, head).  Lane (g, col) takes the 8 codes
// of k-step j that the 16-bit path gives it (dimensions 8(4j + g) .. +7, the
// half g & 1 of 16-byte chunk 2j + g/2 of token col), and the 4 V codes of
// tokens 4g .. 4g+3 of dimension 16dt + col.  Same addressing schemes as
// load_tile: buffer resources with a wave-uniform token offset for blocks of
// 16 and more, per-lane addresses (masked blocks read block 0) for 8.
//
// Head sizes that are multiples of 64 (WideFp8): lane (g, col) takes K chunks
// g + 4m (16 codes, one 16-byte load each) of token col into k8[2m], k8[2m+1],
// and 8 V codes per 8-byte load: dimension 32i + 16(g & 1) + col, tokens
// 8(g >> 1) .. +7, into v8[2i] (tokens +0..3) and v8[2i+1] (+4..7).  Each V
// load instruction covers 32 whole dimension rows.  dequant_tile then swaps
// rows between the two words (v_permlane16_swap) so that v8[2i] and
// v8[2i+1] become the operands of dimension tiles 2i and 2i+1.
template <int D, int BS, int CPOL = 0>
__device__ __forceinline__ void load_tile_fp8(Tile<D, true>& t, const uint8_t* kbase, const uint8_t* vbase,
                                              int64_t k_block_stride, int64_t v_block_stride, int b0, int b1, int tt0,
                                              int g, int col) {
  constexpr int NCHUNK = D / 8;  // 8-code K groups per token
  if constexpr (D % 64 == 0) {
    constexpr int KM = D / 64;  // 16-byte K loads per lane
    constexpr int VI = D / 32;  // 8-byte V loads per lane
    const int vrow = 16 * (g & 1) + col;
    if constexpr (BS >= kTile) {
      const int b = b0;
      t.kpb = t.vpb = b;
      const int off = tt0 % BS;
      const int64_t bb = b < 0 ? 0 : b;
      const int bytes = b < 0 ? 0 : D * BS;
      const __amdgpu_buffer_rsrc_t kr =
          __builtin_amdgcn_make_buffer_rsrc((void*)(kbase + bb * k_block_stride), (short)0, bytes, kBufferRsrcWord3);
      const __amdgpu_buffer_rsrc_t vr =
          __builtin_amdgcn_make_buffer_rsrc((void*)(vbase + bb * v_block_stride), (short)0, bytes, kBufferRsrcWord3);
      const int ko = g * (BS * 16) + col * 16;
      const int vo = vrow * BS + 8 * (g >> 1);
#pragma unroll
      for (int m = 0; m < KM; ++m) {
        const uint4 w =
            __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, ko + m * (4 * BS * 16), off * 16, CPOL));
        t.k8[2 * m] = make_uint2(w.x, w.y);
        t.k8[2 * m + 1] = make_uint2(w.z, w.w);
      }
#pragma unroll
      for (int i = 0; i < VI; ++i) {
        const uint2 w = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(vr, vo + i * (32 * BS), off, CPOL));
        t.v8[2 * i] = w.x;
        t.v8[2 * i + 1] = w.y;
      }
    } else {
      const int kpb = col < 8 ? b0 : b1;  // K row = token tt0 + col
      t.kpb = kpb;
      const uint8_t* kp = kbase + (int64_t)(kpb < 0 ? 0 : kpb) * k_block_stride + (col % BS) * 16 + g * (BS * 16);
      const int vpb = g < 2 ? b0 : b1;  // V tokens tt0 + 8(g >> 1) .. +7 (and, after the swap, tt0 + 4g .. +3)
      t.vpb = vpb;
      const uint8_t* vp = vbase + (int64_t)(vpb < 0 ? 0 : vpb) * v_block_stride + vrow * BS + (8 * (g >> 1)) % BS;
#pragma unroll
      for (int m = 0; m < KM; ++m) {
        const uint4 w = *reinterpret_cast<const uint4*>(kp + m * (4 * BS * 16));
        t.k8[2 * m] = make_uint2(w.x, w.y);
        t.k8[2 * m + 1] = make_uint2(w.z, w.w);
      }
#pragma unroll
      for (int i = 0; i < VI; ++i) {
        const uint2 w = *reinterpret_cast<const uint2*>(vp + i * (32 * BS));
        t.v8[2 * i] = w.x;
        t.v8[2 * i + 1] = w.y;
      }
    }
  } else if constexpr (BS >= kTile) {
    const int b = b0;
    t.kpb = t.vpb = b;
    const int off = tt0 % BS;
    const int64_t bb = b < 0 ? 0 : b;
    const int bytes = b < 0 ? 0 : D * BS;
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(kbase + bb * k_block_stride), (short)0, bytes, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(vbase + bb * v_block_stride), (short)0, bytes, kBufferRsrcWord3);
    const int ko = (g >> 1) * (BS * 16) + col * 16 + (g & 1) * 8;
    const int vo = col * BS + 4 * g;
#pragma unroll
    for (int j = 0; j < Tile<D>::KSTEPS; ++j) {
      const int c = 4 * j + g;
      t.k8[j] = (NCHUNK % 4 == 0 || c < NCHUNK)
                    ? __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(kr, ko + j * (2 * BS * 16),
                                                                                      off * 16, CPOL))
                    : make_uint2(0, 0);
    }
#pragma unroll
    for (int dt = 0; dt < Tile<D>::DT; ++dt)
      t.v8[dt] = __builtin_amdgcn_raw_buffer_load_b32(vr, vo + dt * (16 * BS), off, CPOL);
  } else {
    const int kpb = col < 8 ? b0 : b1;  // K row = token tt0 + col
    t.kpb = kpb;
    const uint8_t* kp = kbase + (int64_t)(kpb < 0 ? 0 : kpb) * k_block_stride + (col % BS) * 16 + (g & 1) * 8 +
                        (g >> 1) * (BS * 16);
    const int vpb = g < 2 ? b0 : b1;  // V tokens tt0 + 4g .. +3
    t.vpb = vpb;
    const uint8_t* vp = vbase + (int64_t)(vpb < 0 ? 0 : vpb) * v_block_stride + ((4 * g) % BS) + col * BS;
#pragma unroll
    for (int j = 0; j < Tile<D>::KSTEPS; ++j) {
      const int c = 4 * j + g;
      t.k8[j] = (NCHUNK % 4 == 0 || c < NCHUNK) ? *reinterpret_cast<const uint2*>(kp + j * (2 * BS * 16))
                                                : make_uint2(0, 0);
    }
#pragma unroll
    for (int dt = 0; dt < Tile<D>::DT; ++dt) t.v8[dt] = *reinterpret_cast<const uint32_t*>(vp + dt * (16 * BS));
  }
}

// ---------------------------------------------------------------------------
// Float32 caches (the reference's (float, float) instantiation,
// paged_attention_inst.metal:69): K [D/4][bs][4] and V [D][bs] floats per
// (block, head).  Scores and PV run on v_mfma_f32_16x16x4_f32 over the
// values as stored, so K, V, the query and the softmax weights are never
// rounded to 16 bits.
//   K: lane (g, col) loads 16-byte chunk 4m + g of token col (dims 16m + 4g
//      .. +3) into k[m]; score MFMA (m, s) takes component s, so its k-index
//      g stands for dim 16m + 4g + s, and the query operand carries the same
//      dim (load_query).
//   V: lane (g, col) loads tokens 4g .. 4g+3 of dim 16dt + col (16
//      contiguous bytes of [D][bs]) into v[dt]; PV MFMA r takes component r,
//      whose k-index g stands for token 4g + r -- the token whose weight for
//      head col is register r of the score MFMA's output in that lane.
// ---------------------------------------------------------------------------
template <int D> struct TileF32 {
  static constexpr int KM = (D + 15) / 16;  // 16-byte K loads per lane
  static constexpr int DT = (D + 15) / 16;  // 16-dim tiles of the output (and V loads)
  float4 k[KM];
  float4 v[DT];
  int kpb, vpb;  // as Tile
};

// The register tile of a cache type, and its load instructions per lane.
template <class CT, int D> struct TileSel {
  using type = Tile<D, std::is_same<CT, FP8>::value>;
  static constexpr int kLoads = Tile<D>::KSTEPS + Tile<D>::DT;
};
template <int D> struct TileSel<F32, D> {
  using type = TileF32<D>;
  static constexpr int kLoads = TileF32<D>::KM + TileF32<D>::DT;
};
template <class CT, int D> using TileOf = typename TileSel<CT, D>::type;

// load_tile for float32 caches; same addressing schemes (buffer resources
// and a wave-uniform token offset for blocks of 16 and more; per-lane
// addresses, masked blocks reading block 0, for 8).  Chunks and dims past
// the head size (D = 120) read as zero.
template <int D, int BS, int CPOL = 0>
__device__ __forceinline__ void load_tile_f32(TileF32<D>& t, const float* kbase, const float* vbase,
                                              int64_t k_block_stride, int64_t v_block_stride, int b0, int b1, int tt0,
                                              int g, int col) {
  constexpr int KM = TileF32<D>::KM;
  constexpr int DT = TileF32<D>::DT;
  constexpr int NCHUNK = D / 4;  // 16-byte K chunks per token
  if constexpr (BS >= kTile) {
    const int b = b0;
    t.kpb = t.vpb = b;
    const int off = tt0 % BS;
    const int64_t bb = b < 0 ? 0 : b;
    const int bytes = b < 0 ? 0 : D * BS * 4;
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(kbase + bb * k_block_stride), (short)0, bytes, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(vbase + bb * v_block_stride), (short)0, bytes, kBufferRsrcWord3);
    // K chunk c of token u at (c * BS + u) * 16 bytes; V dim d, token u at
    // (d * BS + u) * 4 bytes.
    const int ko = (g * BS + col) * 16;
    const int vo = (col * BS + 4 * g) * 4;
#pragma unroll
    for (int m = 0; m < KM; ++m) {
      const int c = 4 * m + g;
      t.k[m] = (D % 16 == 0 || c < NCHUNK)
                   ? __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(kr, ko + m * (4 * BS * 16),
                                                                                      off * 16, CPOL))
                   : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d = 16 * dt + col;
      t.v[dt] = (D % 16 == 0 || d < D)
                    ? __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(vr, vo + dt * (16 * BS * 4),
                                                                                       off * 4, CPOL))
                    : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  } else {
    const int kpb = col < 8 ? b0 : b1;  // K row = token tt0 + col
    t.kpb = kpb;
    const float* kp = kbase + (int64_t)(kpb < 0 ? 0 : kpb) * k_block_stride + (col % BS) * 4;
    const int vpb = g < 2 ? b0 : b1;  // V tokens tt0 + 4g .. +3
    t.vpb = vpb;
    const float* vp = vbase + (int64_t)(vpb < 0 ? 0 : vpb) * v_block_stride + ((4 * g) % BS);
#pragma unroll
    for (int m = 0; m < KM; ++m) {
      const int c = 4 * m + g;
      t.k[m] = (D % 16 == 0 || c < NCHUNK) ? *reinterpret_cast<const float4*>(kp + c * (BS * 4))
                                           : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d = 16 * dt + col;
      t.v[dt] = (D % 16 == 0 || d < D) ? *reinterpret_cast<const float4*>(vp + d * BS)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
}

// Raw FP8 codes -> MFMA operands (MT = BF16 or F16), exactly: the hardware
// conversion, and for the rare tile holding a code with exponent 15 (which
// the hardware reads as an E4M3FN number) the reference's inf / NaN.
// Returns whether the tile holds exponent-15 codes (+-inf or NaN), K or V.
template <class MT, int D> __device__ __forceinline__ bool dequant_tile(Tile<D, true>& t) {
  constexpr int KSTEPS = Tile<D>::KSTEPS;
  constexpr int DT = Tile<D>::DT;
  if constexpr (D % 64 == 0) {
    // Wide V words: row r of the wavefront (lanes 16r .. 16r+15) holds, for
    // its column, tokens 8(r >> 1) .. +7 of dimension tile 2i + (r & 1) in
    // (v8[2i], v8[2i+1]).  Swapping the odd rows of v8[2i] with the even
    // rows of v8[2i+1] leaves tokens 4r .. 4r+3 of tile 2i in v8[2i] and of
    // tile 2i+1 in v8[2i+1], the PV operand layout.
#pragma unroll
    for (int i = 0; i < DT / 2; ++i) {
      const auto r = __builtin_amdgcn_permlane16_swap(t.v8[2 * i], t.v8[2 * i + 1], false, false);
      t.v8[2 * i] = r[0];
      t.v8[2 * i + 1] = r[1];
    }
  }
  uint32_t probe = 0;
#pragma unroll
  for (int j = 0; j < KSTEPS; ++j) {
    probe |= (t.k8[j].x & 0x78787878u) + 0x08080808u;
    probe |= (t.k8[j].y & 0x78787878u) + 0x08080808u;
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) probe |= (t.v8[dt] & 0x78787878u) + 0x08080808u;
#pragma unroll
  for (int j = 0; j < KSTEPS; ++j) {
    const uint2 lo = fp8x4_cvt<MT>(t.k8[j].x), hi = fp8x4_cvt<MT>(t.k8[j].y);
    t.k[j] = make_uint4(lo.x, lo.y, hi.x, hi.y);
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) t.v[dt] = fp8x4_cvt<MT>(t.v8[dt]);
  const bool special = __any((probe & 0x80808080u) != 0u);
  if (special) {
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) {
      const uint2 lo = fp8x4_exact<MT>(t.k8[j].x), hi = fp8x4_exact<MT>(t.k8[j].y);
      t.k[j] = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) t.v[dt] = fp8x4_exact<MT>(t.v8[dt]);
  }
  return special;
}

// Whether any V element of a 16-bit tile is +-inf or NaN (wave-wide): the
// exponent fields' running maximum per 16-bit half (v_pk_max_u16) reaches
// all ones exactly when some element's exponent is all ones.
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
template <class MT, int D> __device__ __forceinline__ bool v_nonfinite(const Tile<D, false>& t) {
  constexpr unsigned short kExp16 = std::is_same<MT, BF16>::value ? 0x7F80 : 0x7C00;
  constexpr uint32_t kExp = (uint32_t)kExp16 * 0x00010001u;
  u16x2_t m = {0, 0};
#pragma unroll
  for (int dt = 0; dt < Tile<D>::DT; ++dt) {
    m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2_t, t.v[dt].x & kExp));
    m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2_t, t.v[dt].y & kExp));
  }
  return __any(m.x == kExp16 || m.y == kExp16);
}

// ---------------------------------------------------------------------------
// Token-row layout (MHATokenPool [rows, Hkv, D] and the flash layout
// [blocks, block_size, Hkv, D]): a token's K and V rows of one head are D
// contiguous elements at its row, row_stride elements apart from the next
// row.  rows[i] is the row of tile token i (-1: masked out).
//
// K needs no reshaping: lane (g, col) reads dimensions 32j + 8g .. +8 of
// token col, exactly the chunks the paged layout gives it.  The PV operand
// wants tokens 4g .. 4g+3 of one dimension in each lane, i.e. four rows per
// lane: lanes instead load 8 consecutive dimensions of one token (lane
// (g, 4a + i): token 4g + i, 16 bytes) and 4x4 transposes inside each quad
// of lanes (DPP moves, no LDS) turn each half into an operand tile; which
// dimension each operand row then stands for is tile_dim's business.  Each
// load instruction reads 64 contiguous bytes of each of 16 rows (8-byte loads
// read 32), which halves the V requests per tile.
// ---------------------------------------------------------------------------

// Quad transpose of 16-bit elements: lane i of a quad holds row i of a 4x4
// matrix as (x: elements 0, 1; y: elements 2, 3); on return lane j holds
// column j in the same form.  `sel` is quad_transpose_sel(i).
//
// Step 1 trades halves with lane i^2: lanes 0, 1 keep x and take the partner's
// x, lanes 2, 3 take the partner's y and keep y, so that lane i holds
// (P, Q) = rows (i&1, (i&1)+2) of columns 0,1 (lanes 0, 1) or 2,3 (lanes
// 2, 3).  Step 2 interleaves 16-bit halves with lane i^1 through v_perm.
// Every DPP move reads a register as loaded or as produced by the previous
// step's selects, never a select of its own step's inputs: the form
// select -> DPP -> select over the same values was miscompiled (a select's
// input overwritten before its last use) by the ROCm 7.2 compiler.
__device__ __forceinline__ uint32_t quad_transpose_sel(int i) {
  // v_perm byte selectors over {S0 = partner, S1 = own}: bytes 0-3 are own,
  // 4-7 the partner's.  Even lanes: (own.lo, partner.lo); odd lanes:
  // (partner.hi, own.hi).
  return (i & 1) ? 0x03020706u : 0x05040100u;
}

__device__ __forceinline__ uint2 quad_transpose16(uint2 r, int i, uint32_t sel) {
  // quad_perm selectors: [2,3,0,1] reads lane i^2, [1,0,3,2] lane i^1.
  // Every lane's source lies in its quad, so the moves need no old value
  // (mov_dpp; update_dpp with old = 0 cost a v_mov per move).
  constexpr int kSwap2 = 2 | (3 << 2) | (0 << 4) | (1 << 6);
  constexpr int kSwap1 = 1 | (0 << 2) | (3 << 4) | (2 << 6);
  const uint32_t ax = (uint32_t)__builtin_amdgcn_mov_dpp((int)r.x, kSwap2, 0xf, 0xf, false);
  const uint32_t ay = (uint32_t)__builtin_amdgcn_mov_dpp((int)r.y, kSwap2, 0xf, 0xf, false);
  const bool low = i < 2;
  const uint32_t P = low ? r.x : ay;
  const uint32_t Q = low ? ax : r.y;
  const uint32_t Pp = (uint32_t)__builtin_amdgcn_mov_dpp((int)P, kSwap1, 0xf, 0xf, false);
  const uint32_t Qp = (uint32_t)__builtin_amdgcn_mov_dpp((int)Q, kSwap1, 0xf, 0xf, false);
  return make_uint2(__builtin_amdgcn_perm(Pp, P, sel), __builtin_amdgcn_perm(Qp, Q, sel));
}

// First of the four consecutive head dimensions that rows 4g .. 4g+3 of PV
// dimension tile dt (and so acc.o[dt] of row group g) stand for.  Paged
// layout: tile dt is dimensions 16dt .. 16dt+15 in order.  Token rows load 8
// dimensions of one token per lane, so tiles pair up: tiles 2e and 2e+1 hold
// 32e + 8q + {0..3} and 32e + 8q + {4..7} in row group q; an odd last tile
// (head sizes 80, 112) is loaded and ordered as in the paged layout.
template <int D, bool ROWS> __device__ __forceinline__ constexpr int tile_dim(int dt, int g) {
  if constexpr (ROWS) {
    if (dt < Tile<D>::DT / 2 * 2) return 32 * (dt >> 1) + 8 * g + 4 * (dt & 1);
  }
  return 16 * dt + 4 * g;
}

// Token rows at head sizes that are multiples of 32 load V whole-row
// (load_tile_rows_whole): lane (g, n) takes dimensions n*NDL .. n*NDL+NDL-1
// (NDL = D / 16) of tokens 4g .. 4g+3, so a quarter-wavefront reads one
// token's row in one piece, and v_perm alone regroups the four tokens into
// operand tiles: tile dt, row n stands for dimension n*NDL + dt.  Output
// row 4g + r of tile dt is then dimension (4g + r)*NDL + dt, no longer four
// consecutive dimensions, so the writers store element by element.
template <int D, bool ROWS> struct RowsWhole {
  static constexpr bool value = ROWS && D % 32 == 0;
};
template <int D, bool ROWS> __device__ __forceinline__ constexpr int out_dim(int dt, int g, int r) {
  if constexpr (RowsWhole<D, ROWS>::value) return (4 * g + r) * (D / 16) + dt;
  return tile_dim<D, ROWS>(dt, g) + r;
}

// rk: row of token col (the lane's K token); rv: row of token 4g + (col & 3)
// (the lane's V token).  V: lane (g, 4a + i) loads dimensions 32e + 8a .. +7
// of token 4g + i into tiles 2e (first four) and 2e + 1 (last four), see
// tile_dim; an odd last tile takes dimensions 16dt + 4a .. +3.  V = false:
// K only (whole-row V comes from load_v_whole).
template <int D, bool V = true>
__device__ __forceinline__ void load_tile_rows(Tile<D>& t, const uint16_t* kbase, const uint16_t* vbase,
                                               int64_t k_row_stride, int64_t v_row_stride, int rk, int rv,
                                               int g, int col) {
  constexpr int NCHUNK = D / 8;  // 16-byte K chunks per token
  t.kpb = rk;
  t.vpb = 0;  // V validity follows the K rows (same token rows)
  const uint16_t* kp = kbase + (int64_t)(rk < 0 ? 0 : rk) * k_row_stride;
  const uint16_t* vp = vbase + (int64_t)(rv < 0 ? 0 : rv) * v_row_stride;
#pragma unroll
  for (int j = 0; j < Tile<D>::KSTEPS; ++j) {
    const int c = 4 * j + g;
    t.k[j] = (NCHUNK % 4 == 0 || c < NCHUNK) ? *reinterpret_cast<const uint4*>(kp + c * 8) : make_uint4(0, 0, 0, 0);
  }
  if constexpr (!V) return;
  constexpr int PAIRS = Tile<D>::DT / 2;
#pragma unroll
  for (int e = 0; e < PAIRS; ++e) {
    const int d = 32 * e + 8 * (col >> 2);
    const uint4 x = (D % 32 == 0 || d < D) ? *reinterpret_cast<const uint4*>(vp + d) : make_uint4(0, 0, 0, 0);
    t.v[2 * e] = make_uint2(x.x, x.y);
    t.v[2 * e + 1] = make_uint2(x.z, x.w);
  }
  if constexpr (Tile<D>::DT % 2 == 1) {
    constexpr int dt = Tile<D>::DT - 1;
    const int d = 16 * dt + 4 * (col >> 2);
    t.v[dt] = d < D ? *reinterpret_cast<const uint2*>(vp + d) : make_uint2(0, 0);
  }
}

// load_tile_rows through buffer resources with 32-bit byte offsets (the
// persistent kernel's form; k_bytes/v_bytes bound the reachable range):
// one VGPR per address and no 64-bit arithmetic per tile.  V = false: K only.
template <int D, int CPOL = 0, bool V = true>
__device__ __forceinline__ void load_tile_rows_buf(Tile<D>& t, __amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr,
                                                   uint32_t k_row_bytes, uint32_t v_row_bytes, int rk, int rv, int g,
                                                   int col) {
  constexpr int NCHUNK = D / 8;
  t.kpb = rk;
  t.vpb = 0;
  // The products stay 32-bit (v_mul_lo_u32): folded with the add below the
  // compiler would use v_mad_u64_u32, whose 64-bit result pair is one more
  // live register pair per tile.
  uint32_t ko = (uint32_t)(rk < 0 ? 0 : rk) * k_row_bytes;
  uint32_t vo = (uint32_t)(rv < 0 ? 0 : rv) * v_row_bytes;
  asm volatile("" : "+v"(ko), "+v"(vo));
  ko += (uint32_t)g * 16u;
  vo += (uint32_t)(col >> 2) * 16u;
#pragma unroll
  for (int j = 0; j < Tile<D>::KSTEPS; ++j) {
    const int c = 4 * j + g;
    t.k[j] = (NCHUNK % 4 == 0 || c < NCHUNK)
                 ? __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, ko + j * 64, 0, CPOL))
                 : make_uint4(0, 0, 0, 0);
  }
  if constexpr (!V) return;
  constexpr int PAIRS = Tile<D>::DT / 2;
#pragma unroll
  for (int e = 0; e < PAIRS; ++e) {
    const int d = 32 * e + 8 * (col >> 2);
    const uint4 x = (D % 32 == 0 || d < D)
                        ? __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, vo + e * 64, 0, CPOL))
                        : make_uint4(0, 0, 0, 0);
    t.v[2 * e] = make_uint2(x.x, x.y);
    t.v[2 * e + 1] = make_uint2(x.z, x.w);
  }
  if constexpr (Tile<D>::DT % 2 == 1) {
    // Dimensions 16dt + 4a .. +3: byte offset 32dt + 8a from the row.
    constexpr int dt = Tile<D>::DT - 1;
    const int d = 16 * dt + 4 * (col >> 2);
    t.v[dt] = d < D ? __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                    vr, vo - (uint32_t)(col >> 2) * 8u + dt * 32, 0, CPOL))
                    : make_uint2(0, 0);
  }
}

// Whole-row V (RowsWhole, head sizes that are multiples of 32): lane (g, n)
// loads dimensions n*NDL .. n*NDL + NDL - 1 (NDL = D / 16) of tokens 4g ..
// 4g+3, so one load instruction of a quarter-wave covers a token's whole
// row.  Word m of token 4g + e (dimensions n*NDL + 2m, +1) goes to word
// e*W + m of t.v (W = NDL / 2 words per token; set_raw / raw_at address
// t.v as 32-bit words), and transpose_tile_rows regroups the words into the
// PV operand tiles 2m and 2m + 1.
template <int D> __device__ __forceinline__ void set_raw(Tile<D>& t, int i, uint32_t w) {
  if (i & 1)
    t.v[i >> 1].y = w;
  else
    t.v[i >> 1].x = w;
}
template <int D> __device__ __forceinline__ uint32_t raw_at(const Tile<D>& t, int i) {
  return (i & 1) ? t.v[i >> 1].y : t.v[i >> 1].x;
}
// Through a buffer resource with 32-bit offsets (rv: rows of tokens 4g ..
// 4g+3, -1 masked; masked rows read row 0, which the K-row masks discard).
template <int D, int CPOL = 0>
__device__ __forceinline__ void load_v_whole_buf(Tile<D>& t, __amdgpu_buffer_rsrc_t vr, uint32_t v_row_bytes, int4 rv,
                                                 int col) {
  constexpr int NDL = D / 16, W = NDL / 2;
  const int rows[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t vo = (uint32_t)(rows[e] < 0 ? 0 : rows[e]) * v_row_bytes + (uint32_t)col * (NDL * 2);
    uint32_t w[W];
    if constexpr (W == 1) {
      w[0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(vr, vo, 0, CPOL);
    } else if constexpr (W == 2) {
      const uint2 x = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(vr, vo, 0, CPOL));
      w[0] = x.x, w[1] = x.y;
    } else if constexpr (W == 3) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b96(vr, vo, 0, CPOL);
      w[0] = x[0], w[1] = x[1], w[2] = x[2];
    } else {
      static_assert(W % 2 == 0, "W = 4, 6 or 8 words per token");
#pragma unroll
      for (int h = 0; h < W / 4; ++h) {
        const uint4 x = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, vo + h * 16, 0, CPOL));
        w[4 * h] = x.x, w[4 * h + 1] = x.y, w[4 * h + 2] = x.z, w[4 * h + 3] = x.w;
      }
      if constexpr (W % 4 == 2) {
        const uint2 x =
            __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(vr, vo + (W / 4) * 16, 0, CPOL));
        w[W - 2] = x.x, w[W - 1] = x.y;
      }
    }
#pragma unroll
    for (int m = 0; m < W; ++m) set_raw<D>(t, e * W + m, w[m]);
  }
}
// Through 64-bit addresses (vbase: the head's base; v_row_stride in
// elements, a multiple of 8).
template <int D>
__device__ __forceinline__ void load_v_whole(Tile<D>& t, const uint16_t* vbase, int64_t v_row_stride, int4 rv,
                                             int col) {
  constexpr int NDL = D / 16, W = NDL / 2;
  const int rows[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t* vp =
        reinterpret_cast<const uint32_t*>(vbase + (int64_t)(rows[e] < 0 ? 0 : rows[e]) * v_row_stride + col * NDL);
#pragma unroll
    for (int m = 0; m < W; ++m) set_raw<D>(t, e * W + m, vp[m]);
  }
}

template <int D> __device__ __forceinline__ void transpose_tile_rows(Tile<D>& t, int col) {
  if constexpr (D % 32 == 0) {
    // Whole-row V: word m of the four tokens holds dimensions (2m, 2m+1);
    // tile 2m takes their low halves (tokens 4g, 4g+1 | 4g+2, 4g+3), tile
    // 2m + 1 the high ones.
    constexpr int W = D / 32;
    uint32_t r[4][W];
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int m = 0; m < W; ++m) r[e][m] = raw_at<D>(t, e * W + m);
#pragma unroll
    for (int m = 0; m < W; ++m) {
      t.v[2 * m] = make_uint2(__builtin_amdgcn_perm(r[1][m], r[0][m], 0x05040100u),
                              __builtin_amdgcn_perm(r[3][m], r[2][m], 0x05040100u));
      t.v[2 * m + 1] = make_uint2(__builtin_amdgcn_perm(r[1][m], r[0][m], 0x07060302u),
                                  __builtin_amdgcn_perm(r[3][m], r[2][m], 0x07060302u));
    }
  } else {
    const uint32_t sel = quad_transpose_sel(col & 3);
#pragma unroll
    for (int dt = 0; dt < Tile<D>::DT; ++dt) t.v[dt] = quad_transpose16(t.v[dt], col & 3, sel);
  }
}

// Row ids of a tile's tokens for the token-row layout, staged in LDS by the
// workgroup (rows[i]: token i of the range, -1 masked).  at() returns the
// lane's (K row, V row) for tile `tile`.
struct LdsRows {
  const int32_t* rows;
  template <int D, int CPOL = 0>
  __device__ __forceinline__ void load_tile(Tile<D>& t, const DecodeParams& p, const uint16_t* kbase,
                                            const uint16_t* vbase, int tile, int /*k*/, int g, int col) const {
    const int32_t* r = rows + tile * kTile;
    if constexpr (D % 32 == 0) {
      load_tile_rows<D, false>(t, kbase, vbase, p.k_block_stride, p.v_block_stride, r[col], 0, g, col);
      load_v_whole<D>(t, vbase, p.v_block_stride, *reinterpret_cast<const int4*>(r + 4 * g), col);
    } else {
      load_tile_rows<D>(t, kbase, vbase, p.k_block_stride, p.v_block_stride, r[col], r[4 * g + (col & 3)], g, col);
    }
  }
};

// Row ids of the tiles one wavefront streams, in the wavefront's own LDS
// region (`ids`, N * 64 entries, 16-byte aligned): entry e is token e % 16 of
// the wavefront's tile number e / 16 (0-based in the order the wavefront
// takes them), so a tile's ids are 16 consecutive entries, and each lane
// reads its K row (one entry) and its four V rows (one 16-byte read)
// directly.  Ids outside the cache (block ids outside [0, num_blocks)) are
// -1.  (Held in registers instead, a tile's ids took a select over the
// registers and five lane permutes: ~40 more instructions per tile.)
template <int MAXT> struct WaveRows {
  static constexpr int N = (MAXT * kTile + 63) / 64;
  int32_t* ids;
  // 32-bit buffer views of the item's K and V head (set with the item).
  __amdgpu_buffer_rsrc_t kr, vr;

  // Tiles first, first + nw, ... of tokens [0, bound) of the block-table
  // row `row` (block size 1 << shift): token t lives in row
  // bt[t >> shift] << shift | t & (block size - 1).  The loads are
  // unconditional (tokens past the bound read its last entry) so that they
  // issue back to back.  Only this wavefront reads the entries it writes,
  // so no barrier is needed.
  __device__ __forceinline__ void load(const int32_t* row, int shift, int64_t num_blocks, int bound, int first,
                                       int nw, int lane) {
    int b[N];
#pragma unroll
    for (int c = 0; c < N; ++c) {
      const int e = 64 * c + lane;
      const int t = (first + (e >> 4) * nw) * kTile + (e & 15);
      b[c] = row[min(t, bound - 1) >> shift];
    }
#pragma unroll
    for (int c = 0; c < N; ++c) {
      const int e = 64 * c + lane;
      const int t = (first + (e >> 4) * nw) * kTile + (e & 15);
      const bool ok = t < bound && (int64_t)(uint32_t)b[c] < num_blocks;
      ids[e] = ok ? (b[c] << shift) + (t & ((1 << shift) - 1)) : -1;
    }
  }
  template <int D, int CPOL = 0>
  __device__ __forceinline__ void load_tile(Tile<D>& t, const DecodeParams& p, const uint16_t* /*kbase*/,
                                            const uint16_t* /*vbase*/, int /*tile*/, int k, int g, int col) const {
    const int32_t* r = ids + k * kTile;
    if constexpr (D % 32 == 0) {
      const int4 rv = *reinterpret_cast<const int4*>(r + 4 * g);
      load_tile_rows_buf<D, CPOL, false>(t, kr, vr, (uint32_t)p.k_block_stride * 2u, 0u, r[col], 0, g, col);
      load_v_whole_buf<D, CPOL>(t, vr, (uint32_t)p.v_block_stride * 2u, rv, col);
    } else {
      load_tile_rows_buf<D, CPOL>(t, kr, vr, (uint32_t)p.k_block_stride * 2u, (uint32_t)p.v_block_stride * 2u, r[col],
                                  r[4 * g + (col & 3)], g, col);
    }
  }
};

// Block ids of the tiles one wavefront streams, held lane-indexed in a few
// VGPRs so that each tile's ids reach SGPRs with a v_readlane: entry e =
// 64 * c + lane of array c is block half e % PER_TILE of the wavefront's
// tile number e / PER_TILE (0-based in the order the wavefront takes them).
// MAXT bounds the tiles per wavefront.
template <int BS, int MAXT> struct WaveBlocks {
  static constexpr int PER_TILE = BS >= kTile ? 1 : 2;
  static constexpr int N = (MAXT * PER_TILE + 63) / 64;
  int v[N];

  // Tiles first, first + nw, ... of tokens [t0, t1) of the block-table row
  // `row`, whose blocks lb0 .. lb0+nlb-1 cover the range.  Ids outside
  // [0, num_blocks) become -1.
  __device__ __forceinline__ void load(const int32_t* row, int64_t num_blocks, int nlb, int lb0, int t0, int first,
                                       int nw, int lane) {
#pragma unroll
    for (int c = 0; c < N; ++c) {
      const int e = 64 * c + lane;
      const int tile = first + (e / PER_TILE) * nw;
      const int lb = (t0 + tile * kTile + (e % PER_TILE) * 8) / BS - lb0;
      int b = -1;
      if (lb < nlb) {
        b = row[lb0 + lb];
        b = (int64_t)(uint32_t)b < num_blocks ? b : -1;
      }
      v[c] = b;
    }
  }
  // Block of entry e, for a different e in each lane (entries past the
  // array read entry e % 64 of the first register; the caller ignores them).
  // Entry e sits in register e / 64 of lane e % 64: every register is read
  // from that lane and the reader keeps the one its own e names (selecting
  // the register before the exchange would apply the reader's choice to the
  // source lane's registers).
  __device__ __forceinline__ int fetch(int e) const {
    const int c = e >> 6, l = e & 63;
    int x = __shfl(v[0], l);
#pragma unroll
    for (int i = 1; i < N; ++i) {
      const int y = __shfl(v[i], l);
      if (c == i) x = y;
    }
    return x;
  }
  // Block of entry e (wave-uniform e).
  __device__ __forceinline__ int get(int e) const {
    const int c = e >> 6, l = e & 63;
    int r = __builtin_amdgcn_readlane(v[0], l);
#pragma unroll
    for (int i = 1; i < N; ++i)
      if (c == i) r = __builtin_amdgcn_readlane(v[i], l);
    return r;
  }
};

// ---------------------------------------------------------------------------
// Shared pieces of the two decode kernels.
// ---------------------------------------------------------------------------

// One wavefront's softmax state: unnormalised output (MFMA accumulator
// layout: lane l, register r of tile dt = head l%16, dim 16*dt + 4*(l/16) + r),
// the reference maximum the weights are taken against, the weight sum of
// this lane's 4 tokens per tile, and the true running maximum.  While tiles
// stream, m_max is the lane's own running maximum (over the scores it
// holds); reduce_max() turns it into the column's, once, before it is read.
// Keeping the cross-lane step out of the tile loop leaves it off every
// tile's path from the scores to the weights: a tile needs the column
// maximum only when some lane's scores pass the rescale slack.
template <int D> struct WaveAcc {
  f32x4 o[Tile<D>::DT];
  float m_run, l_run, m_max;
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int dt = 0; dt < Tile<D>::DT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run = -INFINITY;
    l_run = 0.f;
    m_max = -INFINITY;
  }
  __device__ __forceinline__ void reduce_max() { m_max = column_max(m_max); }
};

// Query rows h0 .. h0+nh-1 of sequence seq -> B-operand registers (head =
// col, dims kstep_dim0(j, g) .. +8); a float32 query is split into hi + lo
// words.
// Float32 caches: the float32 query as loaded, dims 16m + 4g .. +3 (the
// lane's K chunk of TileF32) in word m of (qa, qb): m < KSTEPS in qa, the
// rest in qb (2 * KSTEPS >= KM for every head size).
template <int D>
__device__ __forceinline__ float4 query_f32(const uint4 (&qa)[Tile<D>::KSTEPS], const uint4 (&qb)[Tile<D>::KSTEPS],
                                            int m) {
  return __builtin_bit_cast(float4, m < Tile<D>::KSTEPS ? qa[m] : qb[m - Tile<D>::KSTEPS]);
}
template <int D>
__device__ __forceinline__ void load_query_f32(const float* qrow, bool active, int g, uint4 (&qa)[Tile<D>::KSTEPS],
                                               uint4 (&qb)[Tile<D>::KSTEPS]) {
  constexpr int KS = Tile<D>::KSTEPS;
  static_assert(2 * KS >= TileF32<D>::KM, "the float32 query must fit the operand words");
#pragma unroll
  for (int m = 0; m < 2 * KS; ++m) {
    const int d0 = 16 * m + 4 * g;
    const uint4 w = (active && m < TileF32<D>::KM && d0 < D) ? *reinterpret_cast<const uint4*>(qrow + d0)
                                                            : make_uint4(0, 0, 0, 0);
    if (m < KS)
      qa[m] = w;
    else
      qb[m - KS] = w;
  }
}

template <class QT, class CT, int D, bool WIDE = false>
__device__ __forceinline__ void load_query(const DecodeParams& p, int seq, int h0, int nh, int g, int col,
                                           uint4 (&qa)[Tile<D>::KSTEPS],
                                           uint4 (&qb)[std::is_same<QT, F32>::value ? Tile<D>::KSTEPS : 1]) {
  using QS = typename Elem<QT>::storage;
  constexpr bool SPLIT_Q = std::is_same<QT, F32>::value;
  const QS* qrow = static_cast<const QS*>(p.q) + (int64_t)seq * p.q_stride + (int64_t)(h0 + col) * D;
  if constexpr (std::is_same<CT, F32>::value) {
    static_assert(SPLIT_Q, "float32 caches take a float32 query");
    load_query_f32<D>(qrow, col < nh, g, qa, qb);
  } else {
#pragma unroll
    for (int j = 0; j < Tile<D>::KSTEPS; ++j) {
      const int d0 = kstep_dim0<WIDE>(j, g);
      uint4 a = make_uint4(0, 0, 0, 0), b = make_uint4(0, 0, 0, 0);
      if (col < nh && d0 < D) {
        if constexpr (SPLIT_Q) {
          const float4 x0 = *reinterpret_cast<const float4*>(qrow + d0);
          const float4 x1 = *reinterpret_cast<const float4*>(qrow + d0 + 4);
          uint32_t h[8], l[8];
          split_q<CT>(x0.x, h[0], l[0]);
          split_q<CT>(x0.y, h[1], l[1]);
          split_q<CT>(x0.z, h[2], l[2]);
          split_q<CT>(x0.w, h[3], l[3]);
          split_q<CT>(x1.x, h[4], l[4]);
          split_q<CT>(x1.y, h[5], l[5]);
          split_q<CT>(x1.z, h[6], l[6]);
          split_q<CT>(x1.w, h[7], l[7]);
          a = make_uint4(pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7]));
          b = make_uint4(pack2(l[0], l[1]), pack2(l[2], l[3]), pack2(l[4], l[5]), pack2(l[6], l[7]));
        } else {
          a = *reinterpret_cast<const uint4*>(qrow + d0);
        }
      }
      qa[j] = a;
      if constexpr (SPLIT_Q) qb[j] = b;
    }
  }
}

// Consumes one loaded tile of tokens tt0 .. tt0+15 into acc.  TAIL: the tile
// crosses t1, so tokens at or past t1 are masked.  Tokens of masked-out
// blocks contribute nothing either.  Masked tokens get score -inf and V zero
// (a slot may hold anything, including NaN); with block_size >= 16 a masked
// block's loads already returned zero, so only its scores need masking.
// ctx is the context length of the lane's column (its ALiBi origin).
// COLMASK: columns with col_on false take no part in this tile (their
// scores are -inf), for tiles that serve only some of the columns; check_v
// says whether any column the caller will write may be off, in which case a
// tile with a non-finite V element keeps the off columns' accumulators out
// of the PV product (0 * inf would be NaN).
//
// The online-softmax step shared by every cache type: scores sacc (lane
// (g, col), register r = token vtok + r, head col) -> weights pr against the
// running reference maximum, updating acc's maxima, sum and (on a raised
// reference) its accumulators.  kpb / vpb / zero_v: the tile's masking state
// as consume_tile describes it.  KU: every K row of the tile lies in block
// vpb (paged tiles of blocks of 16 and more), so vpb alone says whether the
// rows are live and no lane needs another's kpb.
template <int D, int BS, bool TAIL, bool COLMASK, bool KU = false>
__device__ __forceinline__ void softmax_tile(const DecodeParams& p, f32x4 sacc, int vtok, int t1, uint32_t ctx,
                                             int g, float slope, int kpb, int vpb, bool zero_v, bool col_on,
                                             WaveAcc<D>& acc, float (&pr)[4]) {
  constexpr int DT = Tile<D>::DT;
  float sc[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) sc[r] = sacc[r] * p.scale_log2;
  if (p.alibi != nullptr) {
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] += slope * (float)(vtok + r - (int)ctx + 1);
  }
  if constexpr (COLMASK) {
    if (!col_on) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = -INFINITY;
    }
  }
  if (TAIL || zero_v) {
    // Lane (g, col) holds scores of tokens vtok..vtok+3 for head col; the K
    // row of token tt0 + i was loaded by lane col = i.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool krow_ok = KU || __shfl(kpb, 4 * g + r, 16) >= 0;
      sc[r] = (vtok + r < t1 && vpb >= 0 && krow_ok) ? sc[r] : -INFINITY;
    }
  } else if constexpr (BS >= kTile) {
    if (vpb < 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = -INFINITY;
    }
  }
  // The lane's maximum decides whether any column passes the slack (m_run
  // is the same in a column's four lanes); only then is the column's taken.
  const float ml = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
  acc.m_max = fmaxf(acc.m_max, ml);
  if (__any(ml > acc.m_run + kRescaleSlack)) {
    const float m_new = fmaxf(acc.m_run, column_max(ml));
    const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(acc.m_run - m_new);
    acc.l_run *= alpha;
    // In place (each register multiplied where it lives): as a plain
    // product the compiler copied all DT x 4 accumulators on the path that
    // skips the rescale, every tile.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) asm("v_mul_f32 %0, %0, %1" : "+v"(acc.o[dt][r]) : "v"(alpha));
    acc.m_run = m_new;
  }
  const float m_use = acc.m_run == -INFINITY ? 0.f : acc.m_run;
#pragma unroll
  for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(sc[r] - m_use);
  acc.l_run += (pr[0] + pr[1]) + (pr[2] + pr[3]);
}

template <class QT, class CT, int D, int BS, bool ROWS, bool TAIL, bool COLMASK = false>
__device__ __forceinline__ void consume_tile_h(const DecodeParams& p, Tile<D, std::is_same<CT, FP8>::value>& t,
                                               int tt0, int t1, uint32_t ctx, int g, int col,
                                               const uint4 (&qa)[Tile<D>::KSTEPS],
                                               const uint4 (&qb)[std::is_same<QT, F32>::value ? Tile<D>::KSTEPS : 1],
                                               float slope, WaveAcc<D>& acc, bool col_on = true,
                                               bool check_v = true) {
  constexpr int KSTEPS = Tile<D>::KSTEPS;
  constexpr int DT = Tile<D>::DT;
  constexpr bool SPLIT_Q = std::is_same<QT, F32>::value;
  constexpr bool F8 = std::is_same<CT, FP8>::value;
  using MT = typename MmaOf<QT, CT>::type;
  const int vtok = tt0 + 4 * g;
  // COLMASK: inactive columns have p = 0, and 0 * inf = NaN; a tile with a
  // non-finite V element keeps their accumulators out of the PV product.
  bool v_special = false;
  if constexpr (F8) {
    const bool sp = dequant_tile<MT, D>(t);
    if constexpr (COLMASK) v_special = sp;
  }
  if constexpr (ROWS) transpose_tile_rows<D>(t, col);
  bool zero_v = false;
  if constexpr (TAIL) {
    zero_v = true;
  } else if constexpr (ROWS || BS < kTile) {
    zero_v = !__all(t.vpb >= 0 && t.kpb >= 0);
  }
  if (zero_v) {
    uint32_t m01, m23;
    if constexpr (ROWS) {
      // Token rows: V tokens 4g .. 4g+3 are valid where their (shared) K
      // row is, which lane 4g + r of this row group holds.
      const bool v0 = vtok + 0 < t1 && __shfl(t.kpb, 4 * g + 0, 16) >= 0;
      const bool v1 = vtok + 1 < t1 && __shfl(t.kpb, 4 * g + 1, 16) >= 0;
      const bool v2 = vtok + 2 < t1 && __shfl(t.kpb, 4 * g + 2, 16) >= 0;
      const bool v3 = vtok + 3 < t1 && __shfl(t.kpb, 4 * g + 3, 16) >= 0;
      m01 = (v0 ? 0x0000ffffu : 0u) | (v1 ? 0xffff0000u : 0u);
      m23 = (v2 ? 0x0000ffffu : 0u) | (v3 ? 0xffff0000u : 0u);
    } else {
      const uint32_t ok = t.vpb >= 0 ? 0xffffffffu : 0u;
      m01 = ok & ((vtok + 0 < t1 ? 0x0000ffffu : 0u) | (vtok + 1 < t1 ? 0xffff0000u : 0u));
      m23 = ok & ((vtok + 2 < t1 ? 0x0000ffffu : 0u) | (vtok + 3 < t1 ? 0xffff0000u : 0u));
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      t.v[dt].x &= m01;
      t.v[dt].y &= m23;
    }
  }
  // ---- S^T = K * Q^T ----
  f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < KSTEPS; ++j) {
    sacc = Mma<MT>::k32(t.k[j], qa[j], sacc);
    if constexpr (SPLIT_Q) sacc = Mma<MT>::k32(t.k[j], qb[j], sacc);
  }
  // ---- online softmax (log2 domain) ----
  float pr[4];
  softmax_tile<D, BS, TAIL, COLMASK, !ROWS && BS >= kTile>(p, sacc, vtok, t1, ctx, g, slope, t.kpb, t.vpb, zero_v,
                                                          col_on, acc, pr);
  // ---- O^T += V^T * P^T ----
  const uint2 pp = make_uint2(pack_p<MT>(pr[0], pr[1]), pack_p<MT>(pr[2], pr[3]));
  if constexpr (COLMASK) {
    if constexpr (!F8) v_special = check_v && v_nonfinite<MT, D>(t);
    if (v_special && check_v) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const f32x4 r = Mma<MT>::k16(t.v[dt], pp, acc.o[dt]);
        acc.o[dt] = col_on ? r : acc.o[dt];
      }
      return;
    }
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc.o[dt] = Mma<MT>::k16(t.v[dt], pp, acc.o[dt]);
}

// consume_tile for float32 caches (TileF32; paged layout, no column masks):
// the same masking and softmax, with the scores and PV on
// v_mfma_f32_16x16x4_f32.  Each product chain is split over four
// accumulators so that consecutive MFMAs do not wait on each other.
template <int D, int BS, bool TAIL>
__device__ __forceinline__ void consume_tile_f32(const DecodeParams& p, TileF32<D>& t, int tt0, int t1, uint32_t ctx,
                                                 int g, const uint4 (&qa)[Tile<D>::KSTEPS],
                                                 const uint4 (&qb)[Tile<D>::KSTEPS], float slope, WaveAcc<D>& acc) {
  constexpr int KM = TileF32<D>::KM;
  constexpr int DT = TileF32<D>::DT;
  const int vtok = tt0 + 4 * g;
  bool zero_v = false;
  if constexpr (TAIL) {
    zero_v = true;
  } else if constexpr (BS < kTile) {
    zero_v = !__all(t.vpb >= 0 && t.kpb >= 0);
  }
  if (zero_v) {
    // Masked tokens' V may hold anything (NaN included): zero it, since
    // their weights are 0.
    const bool ok = t.vpb >= 0;
    const bool u0 = ok && vtok + 0 < t1, u1 = ok && vtok + 1 < t1;
    const bool u2 = ok && vtok + 2 < t1, u3 = ok && vtok + 3 < t1;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      t.v[dt].x = u0 ? t.v[dt].x : 0.f;
      t.v[dt].y = u1 ? t.v[dt].y : 0.f;
      t.v[dt].z = u2 ? t.v[dt].z : 0.f;
      t.v[dt].w = u3 ? t.v[dt].w : 0.f;
    }
  }
  // ---- S^T = K * Q^T ----
  f32x4 s4[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s4[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < KM; ++m) {
    const float4 q = query_f32<D>(qa, qb, m);
    s4[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(t.k[m].x, q.x, s4[0], 0, 0, 0);
    s4[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(t.k[m].y, q.y, s4[1], 0, 0, 0);
    s4[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(t.k[m].z, q.z, s4[2], 0, 0, 0);
    s4[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(t.k[m].w, q.w, s4[3], 0, 0, 0);
  }
  const f32x4 sacc = (s4[0] + s4[1]) + (s4[2] + s4[3]);
  float pr[4];
  softmax_tile<D, BS, TAIL, false, BS >= kTile>(p, sacc, vtok, t1, ctx, g, slope, t.kpb, t.vpb, zero_v, true, acc, pr);
  // ---- O^T += V^T * P^T: MFMA r takes tokens 4g + r ----
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    f32x4 o = acc.o[dt];
    o = __builtin_amdgcn_mfma_f32_16x16x4f32(t.v[dt].x, pr[0], o, 0, 0, 0);
    o = __builtin_amdgcn_mfma_f32_16x16x4f32(t.v[dt].y, pr[1], o, 0, 0, 0);
    o = __builtin_amdgcn_mfma_f32_16x16x4f32(t.v[dt].z, pr[2], o, 0, 0, 0);
    o = __builtin_amdgcn_mfma_f32_16x16x4f32(t.v[dt].w, pr[3], o, 0, 0, 0);
    acc.o[dt] = o;
  }
}

// Consumes one loaded tile (consume_tile_h for 16-bit and FP8 caches,
// consume_tile_f32 for float32 caches).
template <class QT, class CT, int D, int BS, bool ROWS, bool TAIL, bool COLMASK = false>
__device__ __forceinline__ void consume_tile(const DecodeParams& p, TileOf<CT, D>& t, int tt0, int t1, uint32_t ctx,
                                             int g, int col, const uint4 (&qa)[Tile<D>::KSTEPS],
                                             const uint4 (&qb)[std::is_same<QT, F32>::value ? Tile<D>::KSTEPS : 1],
                                             float slope, WaveAcc<D>& acc, bool col_on = true,
                                             bool check_v = true) {
  if constexpr (std::is_same<CT, F32>::value) {
    static_assert(!ROWS && !COLMASK, "float32 caches are read in the paged layout by the one-sequence kernels");
    consume_tile_f32<D, BS, TAIL>(p, t, tt0, t1, ctx, g, qa, qb, slope, acc);
  } else {
    consume_tile_h<QT, CT, D, BS, ROWS, TAIL, COLMASK>(p, t, tt0, t1, ctx, g, col, qa, qb, slope, acc, col_on,
                                                       check_v);
  }
}

// load_query with the lane's own sequence and query head (columns of one
// MFMA serving several sequences); inactive lanes get zeros.
template <class QT, class CT, int D, bool WIDE = false>
__device__ __forceinline__ void load_query_lane(const DecodeParams& p, int seq, int head, bool active, int g,
                                                uint4 (&qa)[Tile<D>::KSTEPS],
                                                uint4 (&qb)[std::is_same<QT, F32>::value ? Tile<D>::KSTEPS : 1]) {
  using QS = typename Elem<QT>::storage;
  constexpr bool SPLIT_Q = std::is_same<QT, F32>::value;
  const QS* qrow = static_cast<const QS*>(p.q) + (int64_t)(active ? seq : 0) * p.q_stride +
                   (int64_t)(active ? head : 0) * D;
#pragma unroll
  for (int j = 0; j < Tile<D>::KSTEPS; ++j) {
    const int d0 = kstep_dim0<WIDE>(j, g);
    uint4 a = make_uint4(0, 0, 0, 0), b = make_uint4(0, 0, 0, 0);
    if (active && d0 < D) {
      if constexpr (SPLIT_Q) {
        const float4 x0 = *reinterpret_cast<const float4*>(qrow + d0);
        const float4 x1 = *reinterpret_cast<const float4*>(qrow + d0 + 4);
        const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        uint32_t h[8], l[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) split_q<CT>(x[e], h[e], l[e]);
        a = make_uint4(pack2(h[0], h[1]), pack2(h[2], h[3]), pack2(h[4], h[5]), pack2(h[6], h[7]));
        b = make_uint4(pack2(l[0], l[1]), pack2(l[2], l[3]), pack2(l[4], l[5]), pack2(l[6], l[7]));
      } else {
        a = *reinterpret_cast<const uint4*>(qrow + d0);
      }
    }
    qa[j] = a;
    if constexpr (SPLIT_Q) qb[j] = b;
  }
}

// Streams the 16-token tiles first, first+NW, ... of tokens [t0, t1) of one
// (sequence, KV head) through the online softmax into acc.  blk holds the
// wavefront's block ids (WaveBlocks::load with the same first, NW, t0);
// first must be wave-uniform.  Tiles that lie entirely inside the range go
// through a prefetching loop; the one tile that crosses t1 (if any) is
// consumed last, with masking, by the wavefront it belongs to.  MAXBUF caps
// the tiles a wavefront keeps in flight (the default policy's depth suits
// few workgroups per CU; with a full CU of eight streaming wavefronts, two
// tiles each keep the memory system just as busy).
// Cache policy of stream_tiles' paged-layout tile loads: nt (non-temporal),
// as each K/V tile is read once per launch there.  Same-process medians:
// Llama-3-8B layer 106.7 -> 96.8 us, its FP8 form 60.2 -> 54.1 us.  Token
// rows keep the default policy (nt: 121.2 -> 148.0 us, as a 256-byte row is
// read by several instructions and nt drops its lines in between).  The
// grouped kernel chooses per job: nt for a private tile (read once), the
// default policy for a shared-prefix tile, which the other items of its KV
// head then read from L2.
constexpr int kStreamCpol = 2;

template <class QT, class CT, int D, int BS, int NW, int MAXT, int MAXBUF = 4, bool ROWS = false,
          class Blocks = WaveBlocks<BS, MAXT>>
__device__ __forceinline__ void stream_tiles(const DecodeParams& p, const typename Elem<CT>::storage* kbase,
                                             const typename Elem<CT>::storage* vbase,
                                             const Blocks& blk, int t0, int t1, uint32_t ctx,
                                             int first, int g, int col, const uint4 (&qa)[Tile<D>::KSTEPS],
                                             const uint4 (&qb)[std::is_same<QT, F32>::value ? Tile<D>::KSTEPS : 1],
                                             float slope, WaveAcc<D>& acc) {
  [[maybe_unused]] constexpr int KSTEPS = Tile<D>::KSTEPS;
  [[maybe_unused]] constexpr int DT = Tile<D>::DT;
  constexpr int PT = WaveBlocks<BS, MAXT>::PER_TILE;
  constexpr bool F8 = std::is_same<CT, FP8>::value;
  constexpr bool F32C = std::is_same<CT, F32>::value;
  using TileT = TileOf<CT, D>;
  const int ntiles = (t1 - t0 + kTile - 1) / kTile;
  const int nfull = (t1 - t0) / kTile;  // tiles entirely inside [t0, t1)
  if (first >= ntiles) return;

  // Loads per tile, and the wait that leaves only the newer tiles' loads in
  // flight.  Waiting for the current tile's loads explicitly (instead of
  // letting each use wait) also tells the compiler that every older load has
  // landed, so reusing registers across the loop back-edge costs no drain.
  constexpr int NBUF = Prefetch<QT, D, BS>::kBuffers < MAXBUF ? Prefetch<QT, D, BS>::kBuffers : MAXBUF;
  static_assert(NBUF >= 2, "the prefetch loop needs at least two tile buffers");
  constexpr int LOADS = TileSel<CT, D>::kLoads;
  constexpr int AHEAD = (NBUF - 1) * LOADS;
  static_assert(AHEAD < 64, "vmcnt counts at most 63 outstanding loads");
  // s_waitcnt immediate (gfx9 encoding): vmcnt in bits 3:0 and 15:14,
  // expcnt 6:4 and lgkmcnt 11:8 left at their maxima (no wait).
  constexpr int kWaitAhead = (AHEAD & 15) | ((AHEAD >> 4) << 14) | (7 << 4) | (15 << 8);

  auto consume = [&](auto tail_tag, TileT& t, int tt0) {
    consume_tile<QT, CT, D, BS, ROWS, decltype(tail_tag)::value>(p, t, tt0, t1, ctx, g, col, qa, qb, slope, acc);
  };
  using Full = std::integral_constant<bool, false>;
  using Tail = std::integral_constant<bool, true>;
  // pad: a load past the wavefront's last full tile, issued only to keep
  // the loads per iteration fixed.  With blocks of 16 and more it gets the
  // zero-sized buffer resource of a masked block, so it counts towards the
  // wait like any other load but reads nothing.
  auto load = [&](TileT& t, int tile, bool pad) {
    if constexpr (ROWS) {
      blk.template load_tile<D>(t, p, kbase, vbase, tile, (tile - first) / NW, g, col);
    } else {
      const int k = (tile - first) / NW;
      int b0 = blk.get(k * PT);
      int b1 = PT == 2 ? blk.get(k * PT + 1) : b0;
      if constexpr (BS >= kTile) {
        if (pad) b0 = b1 = -1;
      }
      if constexpr (F8)
        load_tile_fp8<D, BS, kStreamCpol>(t, kbase, vbase, p.k_block_stride, p.v_block_stride, b0, b1, t0 + tile * kTile, g,
                             col);
      else if constexpr (F32C)
        load_tile_f32<D, BS, kStreamCpol>(t, kbase, vbase, p.k_block_stride, p.v_block_stride, b0, b1, t0 + tile * kTile,
                                          g, col);
      else
        load_tile<D, BS, kStreamCpol>(t, kbase, vbase, p.k_block_stride, p.v_block_stride, b0, b1, t0 + tile * kTile, g, col);
    }
  };

  // Full tiles: NBUF register sets, the loads of the wavefront's tile
  // i + NW*(NBUF-1) issued before tile i is consumed, so each wavefront keeps
  // NBUF - 1 tiles in flight.  Past its last full tile a wavefront still
  // issues a tile's loads per iteration so that every iteration waits for
  // the same count: zero-sized ones with blocks of 16 and more (see load),
  // otherwise re-reads of its last tile (in bounds).  (Driving the loop by the tile index rather than a 0-based
  // per-wavefront counter keeps the compiler's register allocation of the
  // rotating tile sets tight.)
  if (first < nfull) {
    const int last = first + ((nfull - 1 - first) / NW) * NW;
    TileT t[NBUF];
#pragma unroll
    for (int b = 0; b < NBUF - 1; ++b) load(t[b], min(first + b * NW, last), first + b * NW > last);
    int tile = first;
    while (true) {
#pragma unroll
      for (int b = 0; b < NBUF; ++b) {
        // Raised wave priority while the next tile's loads issue, so a
        // wavefront with loads to send wins instruction arbitration over
        // siblings busy with MFMA work: 106.2 against 106.6 us at the
        // Llama-3-8B layer, same process (the FP8 layer is unchanged).
        __builtin_amdgcn_s_setprio(1);
        load(t[(b + NBUF - 1) % NBUF], min(tile + (NBUF - 1) * NW, last), tile + (NBUF - 1) * NW > last);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_s_waitcnt(kWaitAhead);
        consume(Full{}, t[b], t0 + tile * kTile);
        tile += NW;
        if (tile >= nfull) {
          // Token rows leave the loop directly: through the loop's own exit
          // test the compiler kept a path from here back to the loop head,
          // along which this tile's loads were still in flight, and so
          // waited for all loads at the head of every other tile (the
          // prefetch lost for half the tiles: 125 -> 118 us at the
          // Llama-3-8B layer on MHATokenPool rows).  The paged layout
          // keeps the plain exit (0.3 us faster there).
          if constexpr (ROWS) goto full_done;
          break;
        }
      }
      if (tile >= nfull) break;
    }
  full_done:;
  }
  // The tile that crosses t1, if this wavefront owns it.
  if (nfull < ntiles && nfull >= first && (nfull - first) % NW == 0) {
    TileT tt;
    load(tt, nfull, false);
    consume(Tail{}, tt, t0 + nfull * kTile);
  }
}

// Merges the NW wavefronts' states of one workgroup.  Every wavefront first
// moves its accumulators onto its true maximum, so that the final
// denominator is sum(exp(s - max)) + 1e-6 exactly as the reference's.  On
// return wavefront 0 holds the merged output in acc.o, the maximum in M and
// the weight sum in L (per column); other wavefronts' results are
// undefined.  Contains one workgroup barrier.
template <int D, int NW>
__device__ __forceinline__ void merge_waves(WaveAcc<D>& acc, float (*s_red)[Tile<D>::DT * 4][64],
                                            float (*s_m)[16], float (*s_l)[16], int wave, int lane, int g, int col,
                                            float& M, float& L) {
  constexpr int DT = Tile<D>::DT;
  acc.reduce_max();
  if (acc.m_max != -INFINITY && acc.m_max != acc.m_run) {
    const float f = exp2f(acc.m_run - acc.m_max);
    acc.l_run *= f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc.o[dt] *= f;
    acc.m_run = acc.m_max;
  }
  const float l_col = column_sum(acc.l_run);
  if (wave > 0) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) s_red[wave - 1][dt * 4 + r][lane] = acc.o[dt][r];
  }
  if (g == 0) {
    s_m[wave][col] = acc.m_run;
    s_l[wave][col] = l_col;
  }
  __syncthreads();
  if (wave != 0) return;
  M = acc.m_run;
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, s_m[w][col]);
  const float mu = M == -INFINITY ? 0.f : M;
  const float a0 = exp2f(acc.m_run - mu);
  L = l_col * a0;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc.o[dt] *= a0;
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    const float aw = exp2f(s_m[w][col] - mu);
    L += s_l[w][col] * aw;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc.o[dt][r] += aw * s_red[w - 1][dt * 4 + r][lane];
  }
}

// Writes out[row] = o / (L + 1e-6) from wavefront 0's merged state.
template <class QT, int D, bool ROWS = false>
__device__ __forceinline__ void write_output(const DecodeParams& p, int64_t hrow, const WaveAcc<D>& acc, float L,
                                             int g) {
  using QS = typename Elem<QT>::storage;
  const float inv = p.v_scale / (L + 1e-6f);
  QS* out = static_cast<QS*>(p.out) + hrow * D;
#pragma unroll
  for (int dt = 0; dt < Tile<D>::DT; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = out_dim<D, ROWS>(dt, g, r);
      if (D % 16 == 0 || d < D) out[d] = from_f32<QT>(acc.o[dt][r] * inv);
    }
}

// Four consecutive output elements (16-byte aligned for float32, 8-byte
// aligned for the half types).
template <class QT>
__device__ __forceinline__ void store4(typename Elem<QT>::storage* dst, float a, float b, float c, float d) {
  if constexpr (std::is_same<QT, F32>::value) {
    *reinterpret_cast<float4*>(dst) = make_float4(a, b, c, d);
  } else {
    const uint32_t lo = (uint32_t)from_f32<QT>(a) | ((uint32_t)from_f32<QT>(b) << 16);
    const uint32_t hi = (uint32_t)from_f32<QT>(c) | ((uint32_t)from_f32<QT>(d) << 16);
    *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
  }
}

// Merge of the NW wavefronts' states that leaves every wavefront with an
// equal share of the output: each wavefront moves its state onto its true
// maximum and stores it in LDS; after one barrier, wavefront w combines
// dimension tiles w, w+NW, ... of every head row and writes them.  (With one
// wavefront doing all of the merge, the others would queue the next item's
// loads ahead of its output stores and it would start that item late.)
// The weights and sums follow the same order as merge_waves, so the result
// is the reference's sum(exp(s - max) v) / (sum(exp(s - max)) + 1e-6).
// hrow: the output row of the lane's column; active: whether the column
// has one.
template <class QT, int D, int NW, bool ROWS = false>
__device__ __forceinline__ void merge_store_waves(const DecodeParams& p, WaveAcc<D>& acc,
                                                  float4 (*s_red)[Tile<D>::DT][64], float (*s_m)[16],
                                                  float (*s_l)[16], int wave, int lane, int g, int col, int64_t hrow,
                                                  bool active) {
  using QS = typename Elem<QT>::storage;
  constexpr int DT = Tile<D>::DT;
  acc.reduce_max();
  if (acc.m_max != -INFINITY && acc.m_max != acc.m_run) {
    const float f = exp2f(acc.m_run - acc.m_max);
    acc.l_run *= f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc.o[dt] *= f;
    acc.m_run = acc.m_max;
  }
  const float l_col = column_sum(acc.l_run);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
    s_red[wave][dt][lane] = make_float4(acc.o[dt][0], acc.o[dt][1], acc.o[dt][2], acc.o[dt][3]);
  if (g == 0) {
    s_m[wave][col] = acc.m_run;
    s_l[wave][col] = l_col;
  }
  __syncthreads();
  if (!active) return;
  float M = s_m[0][col];
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, s_m[w][col]);
  const float mu = M == -INFINITY ? 0.f : M;
  float aw[NW];
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    aw[w] = exp2f(s_m[w][col] - mu);
    L += s_l[w][col] * aw[w];
  }
  const float inv = p.v_scale / (L + 1e-6f);
  QS* out = static_cast<QS*>(p.out) + hrow * D;
  for (int dt = wave; dt < DT; dt += NW) {
    const int d0 = tile_dim<D, ROWS>(dt, g);
    if (D % 16 != 0 && d0 >= D) continue;  // head sizes are multiples of 8
    float4 o = s_red[0][dt][lane];
    o.x *= aw[0];
    o.y *= aw[0];
    o.z *= aw[0];
    o.w *= aw[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
      const float4 x = s_red[w][dt][lane];
      o.x += aw[w] * x.x;
      o.y += aw[w] * x.y;
      o.z += aw[w] * x.z;
      o.w += aw[w] * x.w;
    }
    if constexpr (RowsWhole<D, ROWS>::value) {
      out[out_dim<D, ROWS>(dt, g, 0)] = from_f32<QT>(o.x * inv);
      out[out_dim<D, ROWS>(dt, g, 1)] = from_f32<QT>(o.y * inv);
      out[out_dim<D, ROWS>(dt, g, 2)] = from_f32<QT>(o.z * inv);
      out[out_dim<D, ROWS>(dt, g, 3)] = from_f32<QT>(o.w * inv);
    } else {
      store4<QT>(out + d0, o.x * inv, o.y * inv, o.z * inv, o.w * inv);
    }
  }
}

__device__ __forceinline__ void unit_heads(const DecodeParams& p, int unit, int& kvh, int& h0, int& nh) {
  kvh = unit / p.slices;
  const int slice = unit - kvh * p.slices;
  h0 = kvh * p.group + slice * 16;
  nh = min(16, p.group - slice * 16);
}

// ---------------------------------------------------------------------------
// The partition kernel's own merge.  Partition states cross workgroups inside
// one launch: each workgroup stores its state, then counts it on its
// (sequence, unit)'s arrival counter, and the workgroup whose state is the
// last to arrive merges.  gfx950's L2 caches are per XCD and not coherent
// with one another for ordinary accesses, so the states are written and read
// with agent-scope relaxed atomic accesses, which gfx950 issues as ordinary
// vector loads and stores carrying the SC1 cache-policy bit: each one is
// coherent at agent scope by itself, with no cache-wide write-back or
// invalidate.  A writer waits until its stores have completed (s_waitcnt
// vmcnt(0)) before its relaxed agent-scope atomic add on the counter, so a
// workgroup that sees the last count can only load states that are already
// at the coherence point.  The last arrival sets the counter back to zero
// for the next launch.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void store_agent2(float* p, float a, float b) {
  const uint64_t v = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_agent2(const float* p) {
  const uint64_t v =
      __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
}
// Waits until this wavefront's vector memory accesses so far have completed;
// the compiler fences keep every access on its side of the wait.
__device__ __forceinline__ void wait_stores() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt and lgkmcnt left at their maxima
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Counts one arrival; true for the expected-th, which resets the counter
// (every arrival of this launch has happened by then).
__device__ __forceinline__ bool arrive_last(int32_t* counter, int expected) {
  const bool last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == expected - 1;
  if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return last;
}

// Log-sum-exp merge of the `count` partition states (slots 0 .. count-1)
// of the nh rows row0 .. row0 + nh - 1, by the whole workgroup, and the rows
// written: thread t takes 4 dimensions (chunk t % (D/4)) of one row per
// pass and folds the states in slot order, so the result does not depend on
// which workgroup merges.  The weights are those of the merge kernel
// (paged_decode_reduce_kernel): sum * exp2(max - running max) per state,
// states whose max is -inf skipped; out = weighted sum / (weight sum +
// 1e-6).
template <class QT, int D, int NT>
__device__ __forceinline__ void merge_part_states(const DecodeParams& p, int64_t row0, int nh, int count) {
  using QS = typename Elem<QT>::storage;
  static_assert(D % 4 == 0, "head sizes are multiples of 8");
  constexpr int CH = D / 4;
  constexpr int RPP = NT / CH;  // rows per pass
  constexpr int U = kMergeGroup;
  const int t = threadIdx.x;
  const int c = t % CH, hr = t / CH;
  for (int hb = 0; hb < nh; hb += RPP) {
    const bool act = hr < RPP && hb + hr < nh;
    const int64_t row = row0 + (act ? hb + hr : 0);
    float m = -INFINITY, l = 0.f;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    float2 e[U];
    float4 o[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      e[u] = make_float2(-INFINITY, 0.f);
      o[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (act && u < count) {
        const int64_t slot = row * p.max_parts + u;
        e[u] = load_agent2(p.ws_ml + slot * 2);
        const float2 lo = load_agent2(p.ws_o + slot * D + 4 * c);
        const float2 hi = load_agent2(p.ws_o + slot * D + 4 * c + 2);
        o[u] = make_float4(lo.x, lo.y, hi.x, hi.y);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) m = fmaxf(m, e[u].x);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool use = e[u].x != -INFINITY;
      const float w = use ? e[u].y * exp2f(e[u].x - m) : 0.f;
      l += w;
      a.x += use ? w * o[u].x : 0.f;
      a.y += use ? w * o[u].y : 0.f;
      a.z += use ? w * o[u].z : 0.f;
      a.w += use ? w * o[u].w : 0.f;
    }
    if (act) {
      const float inv = 1.f / (l + 1e-6f);
      store4<QT>(static_cast<QS*>(p.out) + row * D + 4 * c, a.x * inv, a.y * inv, a.z * inv, a.w * inv);
    }
  }
}

// ---------------------------------------------------------------------------
// Partition kernel: one workgroup of NW wavefronts per (partition, sequence,
// unit).
// ---------------------------------------------------------------------------
template <class QT, class CT, int D, int BS, int NW>
__global__ __launch_bounds__(64 * NW) void paged_decode_part_kernel(DecodeParams p) {
  using QS = typename Elem<QT>::storage;
  constexpr int KSTEPS = Tile<D>::KSTEPS;
  constexpr int DT = Tile<D>::DT;
  constexpr bool SPLIT_Q = std::is_same<QT, F32>::value;
  constexpr int MAXT = kMaxPartition / kTile / NW;  // tiles per wavefront

  __shared__ float s_red[NW - 1][DT * 4][64];
  __shared__ float s_m[NW][16];
  __shared__ float s_l[NW][16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;

  const int unit = blockIdx.x % p.units;
  const int rest = blockIdx.x / p.units;
  const int seq = rest % p.num_seqs;
  const int part = rest / p.num_seqs;
  int kvh, h0, nh;
  unit_heads(p, unit, kvh, h0, nh);

  // Context lengths are read as unsigned, as the reference does.
  const uint32_t ctx = (uint32_t)p.context_lens[seq];
  if (ctx == 0 || ctx > (uint32_t)p.max_seq_len) {
    if (part == 0) {
      QS* out = static_cast<QS*>(p.out) + ((int64_t)seq * p.num_heads + h0) * D;
      for (int i = tid; i < nh * D; i += 64 * NW) out[i] = from_f32<QT>(0.f);
    }
    return;
  }
  const int nparts = ((int)ctx + p.partition - 1) / p.partition;
  if (part >= nparts) return;
  const int t0 = part * p.partition;
  const int t1 = min(t0 + p.partition, (int)ctx);
  const int lb0 = t0 / BS;
  const int nlb = (t1 + BS - 1) / BS - lb0;

  WaveBlocks<BS, MAXT> blk;
  blk.load(p.block_tables + (int64_t)seq * p.max_blocks_per_seq, p.num_blocks, nlb, lb0, t0, wave, NW, lane);
  uint4 qa[KSTEPS];
  uint4 qb[SPLIT_Q ? KSTEPS : 1];
  load_query<QT, typename MmaOf<QT, CT>::type, D, WideFp8<CT, D>::value>(p, seq, h0, nh, g, col, qa, qb);
  const float slope = (p.alibi != nullptr && col < nh) ? p.alibi[h0 + col] * kLog2e : 0.f;

  WaveAcc<D> acc;
  acc.init();
  using CS = typename Elem<CT>::storage;
  const CS* kbase = static_cast<const CS*>(p.k_cache) + (int64_t)kvh * p.k_head_stride;
  const CS* vbase = static_cast<const CS*>(p.v_cache) + (int64_t)kvh * p.v_head_stride;
  stream_tiles<QT, CT, D, BS, NW, MAXT, kPartBuffers>(p, kbase, vbase, blk, t0, t1, ctx, wave, g, col, qa, qb, slope,
                                                      acc);

  float M, L;
  merge_waves<D, NW>(acc, s_red, s_m, s_l, wave, lane, g, col, M, L);
  const int64_t hrow = (int64_t)seq * p.num_heads + h0 + col;
  if (nparts == 1) {
    if (wave == 0 && col < nh) write_output<QT, D>(p, hrow, acc, L, g);
    return;
  }
  const bool fused = p.counters != nullptr;
  if (wave == 0 && col < nh) {
    const int64_t slot = hrow * p.max_parts + part;
    const float invl = L > 0.f ? p.v_scale / L : 0.f;
    float* wo = p.ws_o + slot * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d = 16 * dt + 4 * g;
      if (D % 16 != 0 && d >= D) continue;
      const float x0 = acc.o[dt][0] * invl, x1 = acc.o[dt][1] * invl;
      const float x2 = acc.o[dt][2] * invl, x3 = acc.o[dt][3] * invl;
      if (fused) {
        store_agent2(wo + d, x0, x1);
        store_agent2(wo + d + 2, x2, x3);
      } else {
        *reinterpret_cast<float4*>(wo + d) = make_float4(x0, x1, x2, x3);
      }
    }
    if (g == 0) {
      if (fused)
        store_agent2(p.ws_ml + slot * 2, M, L);
      else
        *reinterpret_cast<float2*>(p.ws_ml + slot * 2) = make_float2(M, L);
    }
  }
  if (!fused) return;  // the merge kernel follows

  // Arrival: the workgroup whose state is the row's last merges them all.
  __shared__ int s_last;
  if (wave == 0) wait_stores();
  if (tid == 0) s_last = arrive_last(p.counters + (int64_t)seq * p.units + unit, nparts);
  __syncthreads();
  if (s_last) merge_part_states<QT, D, 64 * NW>(p, (int64_t)seq * p.num_heads + h0, nh, nparts);
}

// ---------------------------------------------------------------------------
// Token-row kernel: the partition kernel for the token-row layout.  The
// workgroup first stages the rows of its partition's tokens in LDS (from the
// block table and block size; -1 for tokens past the context or in blocks
// outside the pool), then streams tiles that gather those rows.
// ---------------------------------------------------------------------------
template <class QT, class CT, int D>
__global__ __launch_bounds__(64 * kPartWaves) void paged_decode_rows_kernel(DecodeParams p) {
  using QS = typename Elem<QT>::storage;
  constexpr int NW = kPartWaves;
  constexpr int KSTEPS = Tile<D>::KSTEPS;
  constexpr int DT = Tile<D>::DT;
  constexpr bool SPLIT_Q = std::is_same<QT, F32>::value;

  __shared__ float s_red[NW - 1][DT * 4][64];
  __shared__ float s_m[NW][16];
  __shared__ float s_l[NW][16];
  __shared__ __align__(16) int32_t s_rows[kMaxPartition];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;

  const int unit = blockIdx.x % p.units;
  const int rest = blockIdx.x / p.units;
  const int seq = rest % p.num_seqs;
  const int part = rest / p.num_seqs;
  int kvh, h0, nh;
  unit_heads(p, unit, kvh, h0, nh);

  const uint32_t ctx = (uint32_t)p.context_lens[seq];
  if (ctx == 0 || ctx > (uint32_t)p.max_seq_len) {
    if (part == 0) {
      QS* out = static_cast<QS*>(p.out) + ((int64_t)seq * p.num_heads + h0) * D;
      for (int i = tid; i < nh * D; i += 64 * NW) out[i] = from_f32<QT>(0.f);
    }
    return;
  }
  const int nparts = ((int)ctx + p.partition - 1) / p.partition;
  if (part >= nparts) return;
  const int t0 = part * p.partition;
  const int t1 = min(t0 + p.partition, (int)ctx);

  const int32_t* bt = p.block_tables + (int64_t)seq * p.max_blocks_per_seq;
  const int bs = p.block_size;
  const int span = (t1 - t0 + kTile - 1) / kTile * kTile;
  for (int i = tid; i < span; i += 64 * NW) {
    const int t = t0 + i;
    int r = -1;
    if (t < t1) {
      const int32_t b = bt[t / bs];
      if ((int64_t)(uint32_t)b < p.num_blocks) r = b * bs + t % bs;
    }
    s_rows[i] = r;
  }
  __syncthreads();

  uint4 qa[KSTEPS];
  uint4 qb[SPLIT_Q ? KSTEPS : 1];
  load_query<QT, typename MmaOf<QT, CT>::type, D, WideFp8<CT, D>::value>(p, seq, h0, nh, g, col, qa, qb);
  const float slope = (p.alibi != nullptr && col < nh) ? p.alibi[h0 + col] * kLog2e : 0.f;

  WaveAcc<D> acc;
  acc.init();
  using CS = typename Elem<CT>::storage;
  const CS* kbase = static_cast<const CS*>(p.k_cache) + (int64_t)kvh * p.k_head_stride;
  const CS* vbase = static_cast<const CS*>(p.v_cache) + (int64_t)kvh * p.v_head_stride;
  stream_tiles<QT, CT, D, kTile, NW, 1, 2, true, LdsRows>(p, kbase, vbase, LdsRows{s_rows}, t0, t1, ctx, wave, g, col,
                                                         qa, qb, slope, acc);

  float M, L;
  merge_waves<D, NW>(acc, s_red, s_m, s_l, wave, lane, g, col, M, L);
  if (wave != 0 || col >= nh) return;
  const int64_t hrow = (int64_t)seq * p.num_heads + h0 + col;
  if (nparts == 1) {
    write_output<QT, D, true>(p, hrow, acc, L, g);
    return;
  }
  const int64_t slot = hrow * p.max_parts + part;
  const float invl = L > 0.f ? p.v_scale / L : 0.f;
  float* wo = p.ws_o + slot * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    if constexpr (RowsWhole<D, true>::value) {
#pragma unroll
      for (int r = 0; r < 4; ++r) wo[out_dim<D, true>(dt, g, r)] = acc.o[dt][r] * invl;
    } else {
      const int d = tile_dim<D, true>(dt, g);
      if (D % 16 == 0 || d < D)
        *reinterpret_cast<float4*>(wo + d) =
            make_float4(acc.o[dt][0] * invl, acc.o[dt][1] * invl, acc.o[dt][2] * invl, acc.o[dt][3] * invl);
    }
  }
  if (g == 0) *reinterpret_cast<float2*>(p.ws_ml + slot * 2) = make_float2(M, L);
}

// ---------------------------------------------------------------------------
// Persistent kernel: one workgroup of NW wavefronts per CU works through
// whole (sequence, unit) items and produces their output rows without any
// partial results.  Items are ranked longest context first and dealt in a
// snake order (round k gives rank k*G + w to workgroup w, reversed on odd
// rounds), which balances the workgroups' total work.  Each item's context
// length, block ids and query are loaded at its start, after the previous
// item's merge (the reason is given at the item loop).
// ---------------------------------------------------------------------------
template <int D, bool ROWS = false, bool F8 = false> struct Persist {
  // Wavefronts per workgroup: two per SIMD while the register budget allows
  // (head sizes up to 128), one above.
  static constexpr int kWaves = D <= 128 ? 8 : 4;
  // Tile buffers per wavefront (one tile in flight beyond the consumed one:
  // with eight streaming wavefronts per CU, deeper rings measured no faster).
  static constexpr int kMaxBuf = 2;
};

// Rank of each of the first n entries of s_keys (distinct keys; the array
// is padded to a multiple of 16 bytes with keys that never count) among all
// of them, into s_order[rank] = index: DESC ranks larger keys first,
// otherwise smaller ones.  tp = the threads that share one entry's count
// (a power of two, at most 16), each counting a slice of the keys, read 16
// bytes per LDS load (the same address in every lane of the slice group, a
// broadcast); the partial counts meet through lane shuffles.  Every thread
// of the workgroup calls it; it ends with a workgroup barrier.
template <class K, bool DESC>
__device__ __forceinline__ void rank_keys(const K* s_keys, int n, int32_t* s_order, int tid, int nt) {
  constexpr int PER = 16 / sizeof(K);  // keys per 16-byte load
  const int nv = (n + PER - 1) / PER;  // 16-byte loads that cover the keys
  int tp = 1;
  while (tp < 16 && tp * 2 * n <= nt) tp *= 2;
  for (int base = 0; base < n * tp; base += nt) {
    const int t = base + tid;
    const int e = t / tp, part = t - e * tp;
    int r = 0;
    if (e < n) {
      const K k = s_keys[e];
      const int v0 = part * nv / tp, v1 = (part + 1) * nv / tp;
#pragma unroll 4
      for (int v = v0; v < v1; ++v) {
        if constexpr (sizeof(K) == 4) {
          const uint4 w = reinterpret_cast<const uint4*>(s_keys)[v];
          r += DESC ? (w.x > k) + (w.y > k) + (w.z > k) + (w.w > k) : (w.x < k) + (w.y < k) + (w.z < k) + (w.w < k);
        } else {
          const ulonglong2 w = reinterpret_cast<const ulonglong2*>(s_keys)[v];
          r += DESC ? (w.x > k) + (w.y > k) : (w.x < k) + (w.y < k);
        }
      }
    }
    for (int o = 1; o < tp; o <<= 1) r += __shfl_xor(r, o);
    if (e < n && part == 0) s_order[r] = e;
  }
  __syncthreads();
}

// Longest-first rank of the sequences (ties by index) into s_order, when
// there are at most kPersistMaxOrder of them (returns whether it did).
// Empty and over-long contexts (zero rows) count as length 0.  Every thread
// of the workgroup calls it.  Each sequence's key is its length above its
// inverted index, (len << 10) | (1023 - s), so that keys are distinct and
// one comparison orders two sequences; the padding to a multiple of 4
// entries holds 0, below every real key.
static_assert(kPersistMaxOrder == 1024 && kPersistMaxSeq < (1 << 22), "rank keys are (length << 10) | index");
__device__ __forceinline__ bool rank_sequences(const DecodeParams& p, uint32_t* s_key, int32_t* s_order, int tid,
                                               int nt) {
  const int B = p.num_seqs;
  if (B > kPersistMaxOrder) return false;
  const int B4 = (B + 3) & ~3;  // kPersistMaxOrder is a multiple of 4
  for (int s = tid; s < B4; s += nt) {
    uint32_t key = 0;
    if (s < B) {
      uint32_t c = (uint32_t)p.context_lens[s];
      c = c > (uint32_t)p.max_seq_len ? 0u : c;
      key = (c << 10) | (uint32_t)(kPersistMaxOrder - 1 - s);
    }
    s_key[s] = key;
  }
  __syncthreads();
  rank_keys<uint32_t, true>(s_key, B, s_order, tid, nt);
  return true;
}

struct PersistItem {
  int seq, kvh, h0, nh;
  uint32_t ctx;
  bool live;  // context in (0, max_seq_len]; otherwise the rows are zero
};

// BS = 0: token-row caches (any block size, p.block_size), with each
// wavefront's row ids in LDS (WaveRows); otherwise the paged layout.
template <class QT, class CT, int D, int BS>
__global__ __launch_bounds__(64 * (Persist<D, BS == 0>::kWaves)) void paged_decode_persist_kernel(DecodeParams p) {
  constexpr int NW = Persist<D, BS == 0>::kWaves;
  constexpr int NT = 64 * NW;
  constexpr int KSTEPS = Tile<D>::KSTEPS;
  constexpr int DT = Tile<D>::DT;
  constexpr bool SPLIT_Q = std::is_same<QT, F32>::value;
  constexpr bool ROWS = BS == 0;
  constexpr int TBS = ROWS ? kTile : BS;
  constexpr int MAXT = (ROWS ? persist_rows_max_seq(D) : kPersistMaxSeq) / kTile / NW;  // tiles per wavefront
  using Blocks = std::conditional_t<ROWS, WaveRows<MAXT>, WaveBlocks<TBS, MAXT>>;

  __shared__ float4 s_red[2][NW][DT][64];
  __shared__ float s_m[2][NW][16];
  __shared__ float s_l[2][NW][16];
  __shared__ __align__(16) uint32_t s_ctx[kPersistMaxOrder];
  __shared__ int32_t s_order[kPersistMaxOrder];
  // Token rows: each wavefront's row ids (WaveRows).
  constexpr int kRowIds = ROWS ? 64 * ((MAXT * kTile + 63) / 64) : 4;
  __shared__ __align__(16) int32_t s_rowids[NW][kRowIds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;
  const int B = p.num_seqs;
  const int total = B * p.units;
  const int G = gridDim.x;

  // With at most one item per workgroup the order balances nothing, so the
  // ranking (a context-length load and two barriers) is skipped and items
  // go in index order.
  const bool ordered = total > G && rank_sequences(p, s_ctx, s_order, tid, NT);
  // Rank of this workgroup's k-th item (>= total: none).
  auto rank_of = [&](int k) { return k * G + ((k & 1) ? G - 1 - (int)blockIdx.x : (int)blockIdx.x); };
  auto item_at = [&](int rank) {
    PersistItem it;
    const int sr = rank / p.units;
    const int unit = rank - sr * p.units;
    it.seq = ordered ? s_order[sr] : sr;
    unit_heads(p, unit, it.kvh, it.h0, it.nh);
    it.ctx = (uint32_t)p.context_lens[it.seq];
    it.live = it.ctx != 0 && it.ctx <= (uint32_t)p.max_seq_len;
    return it;
  };
  // Block ids of the wavefront's tiles of an item.  The bound comes from
  // max_seq_len rather than the item's context, so these loads do not wait
  // for it; entries past the context are never used.
  const int nlb_max = (p.max_seq_len + TBS - 1) / TBS;
  auto load_blocks = [&](int seq, Blocks& blk) {
    const int32_t* row = p.block_tables + (int64_t)seq * p.max_blocks_per_seq;
    if constexpr (ROWS)
      blk.load(row, __builtin_ctz((unsigned)p.block_size), p.num_blocks, p.max_seq_len, wave, NW, lane);
    else
      blk.load(row, p.num_blocks, nlb_max, 0, 0, wave, NW, lane);
  };

  // Each item's block ids, query and slope are loaded at its start, after
  // the previous item's merge.  Loading them one item ahead, while the
  // previous item streamed, measured 7 us slower at the Llama-3-8B layer
  // (113.4 against 106.3 us in one process): the registers they held (179
  // VGPRs against 158) cost more than the latency they hid behind the merge
  // barrier.
  int buf = 0;
  for (int k = 0;; ++k) {
    const int rank = rank_of(k);
    if (rank >= total) break;
    const PersistItem it = item_at(rank);
    Blocks blk;
    if constexpr (ROWS) blk.ids = s_rowids[wave];
    load_blocks(it.seq, blk);
    uint4 qa[KSTEPS];
    uint4 qb[SPLIT_Q ? KSTEPS : 1];
    load_query<QT, typename MmaOf<QT, CT>::type, D, WideFp8<CT, D>::value>(p, it.seq, it.h0, it.nh, g, col, qa, qb);
    const float slope = (p.alibi != nullptr && col < it.nh) ? p.alibi[it.h0 + col] * kLog2e : 0.f;

    WaveAcc<D> acc;
    acc.init();
    if (it.live) {
      using CS = typename Elem<CT>::storage;
      const CS* kbase = static_cast<const CS*>(p.k_cache) + (int64_t)it.kvh * p.k_head_stride;
      const CS* vbase = static_cast<const CS*>(p.v_cache) + (int64_t)it.kvh * p.v_head_stride;
      if constexpr (ROWS) {
        // Every head's rows end within k_rows_bytes (v_rows_bytes) of its base.
        blk.kr = __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)0, (int)p.k_rows_bytes, kBufferRsrcWord3);
        blk.vr = __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, (int)p.v_rows_bytes, kBufferRsrcWord3);
      }
      stream_tiles<QT, CT, D, TBS, NW, MAXT, Persist<D, ROWS, std::is_same<CT, FP8>::value>::kMaxBuf, ROWS, Blocks>(
          p, kbase, vbase, blk, 0, (int)it.ctx, it.ctx, wave, g, col, qa, qb, slope, acc);
    }
    // Every wavefront reads s_red[buf] right after this item's barrier and
    // before it reaches the next item's; s_red[buf] is written again only
    // after that one, two items later.
    merge_store_waves<QT, D, NW, ROWS>(p, acc, s_red[buf], s_m[buf], s_l[buf], wave, lane, g, col,
                                       (int64_t)it.seq * p.num_heads + it.h0 + col, col < it.nh);
    buf ^= 1;
  }
}

// ---------------------------------------------------------------------------
// Grouped persistent kernel (paged layout): each item is (S sequences whose
// longest-first ranks are ngroups apart, KV head), and the 16 MFMA columns
// hold the GQA query heads of all S sequences (S * group <= 16).  A
// wavefront walks its tiles w, w+NW, ... of the longest of the S contexts (in
// the order described at Job below); tile by tile:
//   * shared -- every live sequence of the item maps the tile to the same
//     block(s) and holds all 16 of its tokens: the tile is loaded once and
//     feeds all columns (a radix-shared prefix is read once per S sequences);
//   * otherwise each sequence whose context reaches the tile gets it as a
//     job of its own, with only its columns active.
// Jobs are streamed through two tile buffers, the next job's loads issued
// before the current one is consumed, so shared and private tiles follow
// each other without a pipeline refill.  A tile is never loaded more often
// than by the one-sequence kernels, and the MFMA count per loaded tile is the
// same; what sharing saves is loads.  Items are dealt like the persistent
// kernel's (snake order over the workgroups); the sequences of an item are
// taken S-strided from the longest-first order.
// ---------------------------------------------------------------------------
constexpr int kGroupSeqs = 4;       // sequences per item
constexpr int kGroupMaxSeq = 8192;  // longest context (block ids in registers)

template <int S> struct GroupItem {
  int kvh;
  int seq[S];       // -1: no sequence in this slot (last, partial group)
  uint32_t ctx[S];  // 0 unless live
};

// Wavefronts per workgroup and tile buffers per wavefront of the grouped
// kernel.  Measured on the radix-shared B256 workload (job iterator of the
// previous form, same process): eight wavefronts with two buffers 105 us;
// four wavefronts (one per SIMD, registers for a deeper ring) 157-160 us
// with 3, 4, 5 or 6 buffers alike.  More tiles in flight did not help; a
// second wavefront per SIMD to overlap each job's dependent instructions
// did.  Counters then showed 271 VALU and 128 SALU instructions per job
// against 82 and 48 per tile in the one-sequence kernel (same 12 MFMAs and
// 12 loads), which the per-item job list below removes.
constexpr int kGroupBuffers = 2;
// FP8 caches: two workgroups of four wavefronts per CU (the same eight
// wavefronts, two items in flight per CU, so one item's job-list build and
// merge overlap the other's stream): 66.7 against 70.4 us on the
// radix-shared B256 workload, same process.  16-bit caches keep one
// workgroup of eight (with four the kernel spills and times the same), and
// so do FP8 head sizes that are not multiples of 64 (they would spill).
template <class CT, int D> struct GroupShape {
  static constexpr bool kPairs = std::is_same<CT, FP8>::value && D % 64 == 0;
  static constexpr int kWaves = kPairs ? 4 : 8;
  static constexpr int kPerCu = kPairs ? 2 : 1;
};
// Longest context of the grouped kernel with NW wavefronts: each wavefront
// lists at most 64 tiles of an item (one per lane).
template <int NW> constexpr int group_max_seq() {
  return kGroupMaxSeq < 64 * kTile * NW ? kGroupMaxSeq : 64 * kTile * NW;
}


template <class QT, class CT, int D, int BS, int S, int NW, int NB>
__global__ __launch_bounds__(64 * NW, NW >= 8 ? 1 : 2) void paged_decode_group_kernel(DecodeParams p) {
  static_assert(NB >= 2, "the job pipeline needs at least two tile buffers");
  constexpr int NT = 64 * NW;
  constexpr int KSTEPS = Tile<D>::KSTEPS;
  constexpr int DT = Tile<D>::DT;
  constexpr bool SPLIT_Q = std::is_same<QT, F32>::value;
  constexpr bool F8 = std::is_same<CT, FP8>::value;
  constexpr int MAXT = group_max_seq<NW>() / kTile / NW;  // tiles per wavefront
  using Blocks = WaveBlocks<BS, MAXT>;
  constexpr int PT = Blocks::PER_TILE;
  using TileT = Tile<D, F8>;
  using CS = typename Elem<CT>::storage;
  using MT = typename MmaOf<QT, CT>::type;
  constexpr int LOADS = KSTEPS + DT;
  constexpr int AHEAD = (NB - 1) * LOADS;
  static_assert(AHEAD < 64, "vmcnt counts at most 63 outstanding loads");
  constexpr int kWaitAhead = (AHEAD & 15) | ((AHEAD >> 4) << 14) | (7 << 4) | (15 << 8);

  // Each wavefront's tiles of an item are its lanes (one tile per lane) when
  // the job list is built.
  static_assert(MAXT <= 64, "the job list takes one lane per tile of the wavefront");
  __shared__ float4 s_red[NW][DT][64];
  __shared__ float s_m[NW][16];
  __shared__ float s_l[NW][16];
  __shared__ __align__(16) uint32_t s_ctx[kPersistMaxOrder];
  __shared__ int32_t s_order[kPersistMaxOrder];
  // The item's job list, dealt to the wavefronts round-robin.  One-block
  // tiles (PT == 1) take (block, meta); two-block tiles (block, block, meta,
  // unused).  s_cnt: each wavefront's share of the list while it is built.
  using JobEntry = std::conditional_t<PT == 1, int2, int4>;
  __shared__ JobEntry s_jobs[NW * MAXT * S];
  __shared__ int s_cnt[NW];
  static_assert(NW * MAXT <= 1024 && S <= 14, "job meta holds tile < 1024 and slot + 1 < 15");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;
  const int B = p.num_seqs;
  const int grp = p.group;  // query heads per KV head; S * grp <= 16 (checked by the launcher)
  const int ngroups = (B + S - 1) / S;
  const int total = ngroups * p.num_kv_heads;
  const int G = gridDim.x;
  // The lane's column: sequence slot ci of the item, query head hc of its group.
  const int ci = col / grp;
  const int hc = col - ci * grp;
  const bool col_used = ci < S;

  const bool ordered = rank_sequences(p, s_ctx, s_order, tid, NT);
  auto rank_of = [&](int k) { return k * G + ((k & 1) ? G - 1 - (int)blockIdx.x : (int)blockIdx.x); };
  auto item_at = [&](int rank, GroupItem<S>& it) {
    const int gr = rank / p.num_kv_heads;
    it.kvh = rank - gr * p.num_kv_heads;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      // Ranks gr, gr + ngroups, ...: every item mixes long and short
      // contexts, so items are of like size and the snake order pairs them
      // evenly (89.6 against 90.3 us with ranks gr*S .. gr*S + S-1 on the
      // radix-shared B256 workload, mean of five same-process pairs).
      const int sr = gr + i * ngroups;
      it.seq[i] = sr < B ? (ordered ? s_order[sr] : sr) : -1;
      const uint32_t c = it.seq[i] >= 0 ? (uint32_t)p.context_lens[it.seq[i]] : 0u;
      it.ctx[i] = (c != 0 && c <= (uint32_t)p.max_seq_len) ? c : 0u;
    }
  };
  const int nlb_max = (p.max_seq_len + BS - 1) / BS;
  auto load_blocks = [&](const GroupItem<S>& it, Blocks (&blk)[S]) {
#pragma unroll
    for (int i = 0; i < S; ++i)
      blk[i].load(p.block_tables + (int64_t)(it.seq[i] >= 0 ? it.seq[i] : 0) * p.max_blocks_per_seq, p.num_blocks,
                  nlb_max, 0, 0, wave, NW, lane);
  };
  // Per-lane view of the item: the column's sequence, context and slope.
  auto lane_of = [&](const GroupItem<S>& it, int& seq, uint32_t& ctx) {
    seq = -1;
    ctx = 0;
#pragma unroll
    for (int i = 0; i < S; ++i)
      if (ci == i) {
        seq = it.seq[i];
        ctx = it.ctx[i];
      }
  };
  auto load_lane_query = [&](const GroupItem<S>& it, uint4 (&qa)[KSTEPS], uint4 (&qb)[SPLIT_Q ? KSTEPS : 1],
                             float& slope) {
    int seq;
    uint32_t ctx;
    lane_of(it, seq, ctx);
    const bool on = col_used && seq >= 0;
    const int head = it.kvh * grp + hc;
    load_query_lane<QT, MT, D, WideFp8<CT, D>::value>(p, seq, head, on, g, qa, qb);
    slope = (p.alibi != nullptr && on) ? p.alibi[head] * kLog2e : 0.f;
  };

  // Each item's block ids, queries and slopes are loaded at its start (as
  // in the one-sequence persistent kernel, where loading them an item ahead
  // measured slower).
  for (int k = 0;; ++k) {
    const int rank = rank_of(k);
    if (rank >= total) break;
    GroupItem<S> it;
    item_at(rank, it);
    Blocks blk[S];
    load_blocks(it, blk);
    uint4 qa[KSTEPS];
    uint4 qb[SPLIT_Q ? KSTEPS : 1];
    float slope;
    load_lane_query(it, qa, qb, slope);

    // ---- the item's jobs ----
    int nt[S];  // tiles per sequence (0: not live)
    int maxnt = 0;
    uint32_t minctx = 0xffffffffu;
    int first_live = -1;
    bool all_live = true;  // every sequence slot of the item holds a live sequence
#pragma unroll
    for (int i = 0; i < S; ++i) {
      nt[i] = ((int)it.ctx[i] + kTile - 1) / kTile;
      maxnt = max(maxnt, nt[i]);
      if (it.ctx[i] != 0) {
        minctx = min(minctx, it.ctx[i]);
        if (first_live < 0) first_live = i;
      } else {
        all_live = false;
      }
    }
    int lane_seq;
    uint32_t lane_ctx;
    lane_of(it, lane_seq, lane_ctx);
    const bool lane_live = col_used && lane_ctx != 0;
    const CS* kbase = static_cast<const CS*>(p.k_cache) + (int64_t)it.kvh * p.k_head_stride;
    const CS* vbase = static_cast<const CS*>(p.v_cache) + (int64_t)it.kvh * p.v_head_stride;

    // Job list of the item, built once: lane n of wavefront w describes
    // tile w + NW kk(n), kk taken from both ends in turn (0, K-1, 1, K-2,
    // ...), so that the shared prefix alternates with the private tails and
    // L2-served and HBM-served loads overlap.  A tile is
    //   * shared: every live sequence maps it to the same block(s) and holds
    //     all 16 of its tokens -- one job that feeds every column, so a
    //     radix-shared prefix is read once per S sequences;
    //   * otherwise one job per sequence that reaches it, with only that
    //     sequence's columns active.
    // A wave prefix sum of the lanes' job counts, offset by the earlier
    // wavefronts' counts, places each lane's jobs in the item's LDS list:
    // (block of tokens 0-7, block of tokens 8-15, tile | (sequence slot + 1,
    // 0 = shared) << 10 | valid tokens << 16).  Wavefront w then runs jobs
    // w, w + NW, ...: the item's jobs split within one per wavefront, where
    // whole tiles per wavefront left the first wavefronts up to one job per
    // sequence ahead (every sequence's last tile falls to them), and the
    // item's merge waits for the last.
    const int K = maxnt > wave ? (maxnt - 1 - wave) / NW + 1 : 0;  // tiles this wavefront lists
    int wjobs = 0, incl = 0, cnt = 0;
    int kk = 0, fb0 = 0, fb1 = 0;
    bool shared = false;
    int b0[S], b1[S];
    if (K > 0) {
      const bool has = lane < K;
      kk = (lane & 1) ? K - 1 - (lane >> 1) : (lane >> 1);
      const int tt0 = (wave + kk * NW) * kTile;
#pragma unroll
      for (int i = 0; i < S; ++i) {
        b0[i] = blk[i].fetch(kk * PT);
        b1[i] = PT == 2 ? blk[i].fetch(kk * PT + 1) : b0[i];
      }
      shared = tt0 + kTile <= (int)minctx;
#pragma unroll
      for (int i = 0; i < S; ++i) {
        if (it.ctx[i] == 0) continue;
        if (i == first_live) {
          fb0 = b0[i];
          fb1 = b1[i];
        } else {
          shared = shared && b0[i] == fb0 && b1[i] == fb1;
        }
      }
      if (has) {
        if (shared) {
          cnt = 1;
        } else {
#pragma unroll
          for (int i = 0; i < S; ++i) cnt += tt0 < (int)it.ctx[i];
        }
      }
      incl = cnt;  // inclusive prefix sum over the lanes
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        incl += lane >= o ? y : 0;
      }
      wjobs = __builtin_amdgcn_readlane(incl, 63);
    }
    if (lane == 0) s_cnt[wave] = wjobs;
    __syncthreads();
    int base = 0, item_jobs = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const int c = s_cnt[w];
      base += w < wave ? c : 0;
      item_jobs += c;
    }
    if (cnt > 0) {
      auto entry = [](int blk0, int blk1, int meta) {
        if constexpr (PT == 1)
          return make_int2(blk0, meta);
        else
          return make_int4(blk0, blk1, meta, 0);
      };
      const int tile = wave + kk * NW;
      const int tt0 = tile * kTile;
      int at = base + incl - cnt;
      if (shared) {
        s_jobs[at] = entry(fb0, fb1, tile | (kTile << 16));
      } else {
#pragma unroll
        for (int i = 0; i < S; ++i) {
          if (tt0 < (int)it.ctx[i]) {
            const int ntok = min(kTile, (int)it.ctx[i] - tt0);
            s_jobs[at++] = entry(b0[i], b1[i], tile | ((i + 1) << 10) | (ntok << 16));
          }
        }
      }
    }
    __syncthreads();
    const int njobs = item_jobs > wave ? (item_jobs - 1 - wave) / NW + 1 : 0;  // this wavefront's jobs
    struct Job {
      int b0, b1, tile, i, ntok;  // i = -1: shared
      bool pad;                   // past the wavefront's last job (see load_job)
    };
    // The wavefront's job j (item list entry wave + NW j) as read from LDS
    // (every lane reads the same entry), and as a wave-uniform job.  Past
    // the wavefront's last job: the item's first job, as padding.
    auto entry_at = [&](int j) -> JobEntry { return s_jobs[j < njobs ? wave + NW * j : 0]; };
    auto job_of = [&](int j, JobEntry e) -> Job {
      int b0, b1, meta;
      if constexpr (PT == 1) {
        b0 = e.x;
        b1 = e.x;
        meta = e.y;
      } else {
        b0 = e.x;
        b1 = e.y;
        meta = e.z;
      }
      meta = __builtin_amdgcn_readfirstlane(meta);
      return Job{__builtin_amdgcn_readfirstlane(b0), PT == 2 ? __builtin_amdgcn_readfirstlane(b1) : 0, meta & 0x3ff,
                 ((meta >> 10) & 0x3f) - 1, meta >> 16, j >= njobs};
    };
    // Every pipeline step issues one job's loads, padding past the last job
    // included, so that every step waits for the same count: a conditional
    // load makes the compiler wait for all outstanding loads (vmcnt(0))
    // before each tile is consumed, the next job's too, which left no load
    // in flight during the MFMA work (the one-sequence kernel's tile stream
    // pads the same way).  A padding load gets the zero-sized buffer
    // resource of a masked block with blocks of 16 and more (it reads
    // nothing); with smaller blocks it re-reads the item's first tile.
    // NT: the job's loads use the nontemporal policy (a private tile, read
    // once); shared tiles keep the default one, as the other items of their
    // KV head read them from L2.
    auto load_job = [&](TileT& t, const Job& j, auto NT) {
      int b0 = j.b0, b1 = PT == 2 ? j.b1 : j.b0;
      if constexpr (BS >= kTile) {
        if (j.pad) b0 = b1 = -1;
      }
      const int tt0 = j.tile * kTile;
      if constexpr (decltype(NT)::value) {
        if constexpr (F8)
          load_tile_fp8<D, BS, kStreamCpol>(t, kbase, vbase, p.k_block_stride, p.v_block_stride, b0, b1, tt0, g, col);
        else
          load_tile<D, BS, kStreamCpol>(t, kbase, vbase, p.k_block_stride, p.v_block_stride, b0, b1, tt0, g, col);
      } else {
        if constexpr (F8)
          load_tile_fp8<D, BS>(t, kbase, vbase, p.k_block_stride, p.v_block_stride, b0, b1, tt0, g, col);
        else
          load_tile<D, BS>(t, kbase, vbase, p.k_block_stride, p.v_block_stride, b0, b1, tt0, g, col);
      }
    };
    auto consume_job = [&](TileT& t, const Job& j, WaveAcc<D>& acc) {
      const int tt0 = j.tile * kTile;
      const int t1 = tt0 + j.ntok;
      const bool on = lane_live && (j.i < 0 || ci == j.i);
      // Columns that take no part in a job get p = 0, and 0 * inf is NaN:
      // such jobs check V for non-finite values (consume_tile); a shared
      // job of an item whose sequences are all live has every column on.
      const bool partial = j.i >= 0 || !all_live;
      // 16-bit caches: one code path for whole and partial tiles (the token
      // mask is built for every job).  With a second path the compiler moved
      // the accumulators between register sets at every join (64 more VGPRs
      // and 16 v_mov_b64 per job); one path measured 91.0 against 99.0 us on
      // the radix-shared B256 workload, same process.  FP8 tiles keep the
      // two paths: their masking comes after the dequantisation and costs
      // more than the moves (75.8 against 72.0 us).
      if constexpr (!F8) {
        consume_tile<QT, CT, D, BS, false, true, true>(p, t, tt0, t1, lane_ctx, g, col, qa, qb, slope, acc, on,
                                                       partial);
      } else if (j.ntok < kTile) {
        consume_tile<QT, CT, D, BS, false, true, true>(p, t, tt0, t1, lane_ctx, g, col, qa, qb, slope, acc, on, partial);
      } else {
        consume_tile<QT, CT, D, BS, false, false, true>(p, t, tt0, t1, lane_ctx, g, col, qa, qb, slope, acc, on,
                                                        partial);
      }
    };

    // Ring of NB tile buffers: the loads of the next NB - 1 jobs are in
    // flight while a job is consumed.  jb[b] is the job whose tile sits in
    // t[b] (padding past the wavefront's last job).  The LDS entry of the
    // job after the next one to load is read an iteration early, so its
    // latency stays off the path to the next load.  (Two LDS slots per
    // wavefront filled by buffer-to-LDS loads, for two jobs in flight during
    // each consume, measured slower: 108.2 against 101.6 us on the
    // radix-shared B256 workload.)
    WaveAcc<D> acc;
    acc.init();
    if (njobs > 0) {
      TileT t[NB];
      Job jb[NB];
#pragma unroll
      for (int b = 0; b < NB - 1; ++b) {
        jb[b] = job_of(b, entry_at(b));
        if (jb[b].i >= 0)
          load_job(t[b], jb[b], std::true_type{});
        else
          load_job(t[b], jb[b], std::false_type{});
      }
      JobEntry ahead = entry_at(NB - 1);
      int j = 0;
      bool more = true;
      while (more) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int sl = (b + NB - 1) % NB;
          jb[sl] = job_of(j + NB - 1, ahead);
          ahead = entry_at(j + NB);
          // Each branch issues its loads, waits and consumes: with the
          // loads alone in the branches the compiler saw a path with no loads
          // and waited for all of them (vmcnt(0)) before every tile.
          if (jb[sl].i >= 0) {
            load_job(t[sl], jb[sl], std::true_type{});
            __builtin_amdgcn_s_waitcnt(kWaitAhead);
            consume_job(t[b], jb[b], acc);
          } else {
            load_job(t[sl], jb[sl], std::false_type{});
            __builtin_amdgcn_s_waitcnt(kWaitAhead);
            consume_job(t[b], jb[b], acc);
          }
          ++j;
          if (j >= njobs) {
            more = false;
            break;
          }
        }
      }
    }
    // One merge buffer: every wavefront has read it (merge_store_waves)
    // before any writes it for the next item.
    merge_store_waves<QT, D, NW>(p, acc, s_red, s_m, s_l, wave, lane, g, col,
                                 (int64_t)lane_seq * p.num_heads + it.kvh * grp + hc, col_used && lane_seq >= 0);
    __syncthreads();
  }
}

// Log-sum-exp merge of the partitions of one (sequence, query head) per
// workgroup.  Rows whose sequence fits in one partition (or has an empty or
// over-long context) were finished by the partition kernel.  Wavefront w takes
// partitions w, w+NW, ..., U of them per step with their loads issued
// together, and keeps its own running maximum (so no separate pass finds the
// maximum first); the wavefronts' (max, sum, output) states are combined
// through LDS.  A row of P partitions costs about P / (NW*U) dependent memory
// round trips.
constexpr int kMergeWaves = 8;

template <class QT, int D>
__global__ __launch_bounds__(64 * kMergeWaves) void paged_decode_reduce_kernel(DecodeParams p) {
  using QS = typename Elem<QT>::storage;
  constexpr int NW = kMergeWaves;
  constexpr int NDL = (D + 63) / 64;  // dimensions per lane
  // Partitions per wavefront and step: 128 per step in all.  (32 per
  // wavefront, one step for the 512-token partitions of a 128K context,
  // measured 2-2.5 us slower on every Qwen2-7B long-context call.)
  constexpr int U = 16;
  __shared__ float s_acc[NW][NDL * 64];
  __shared__ float s_m[NW];
  __shared__ float s_s[NW];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = blockIdx.x;  // seq * Hq + head
  const int seq = (int)(blockIdx.x / (uint32_t)p.num_heads);
  const float2* ml = reinterpret_cast<const float2*>(p.ws_ml) + row * p.max_parts;
  const float* po = p.ws_o + row * p.max_parts * D;
  // Partitions i0 + u*NW of step i0, clamped to `lim` (in-range repeats of
  // i0 that the accumulation skips).
  float2 e[U];
  float ov[U][NDL];
  auto load_step = [&](int i0, int lim) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * NW < lim ? i0 + u * NW : i0;
      e[u] = ml[i];
#pragma unroll
      for (int k = 0; k < NDL; ++k) {
        const int d = lane + 64 * k;
        ov[u][k] = (D % 64 == 0 || d < D) ? po[(int64_t)i * D + d] : 0.f;
      }
    }
  };
  float mw = -INFINITY, sw = 0.f;
  float acc[NDL];
#pragma unroll
  for (int k = 0; k < NDL; ++k) acc[k] = 0.f;
  auto accumulate = [&](int i0, int nparts) {
    float gm = -INFINITY;
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + u * NW < nparts) gm = fmaxf(gm, e[u].x);
    if (gm > mw) {  // rescale onto the new running maximum
      const float f = mw == -INFINITY ? 0.f : exp2f(mw - gm);
      sw *= f;
#pragma unroll
      for (int k = 0; k < NDL; ++k) acc[k] *= f;
      mw = gm;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // A partition whose tokens were all masked has m = -inf and l = 0.
      // Entries past nparts are selected away rather than weighted by 0:
      // the first step reads them from workspace this call did not write,
      // which may hold inf or NaN.
      const bool use = i0 + u * NW < nparts && e[u].x != -INFINITY;
      const float w = use ? e[u].y * exp2f(e[u].x - mw) : 0.f;
      sw += w;
#pragma unroll
      for (int k = 0; k < NDL; ++k) acc[k] += use ? w * ov[u][k] : 0.f;
    }
  };
  // The first step's partials load together with the context length:
  // bounded by the workspace's max_parts instead of the row's partition
  // count, and accumulated (masked by that count) before any branch on it,
  // so that neither waits for the other.  Rows that need no merge (empty,
  // over-long or single-partition contexts) read and drop them.  A
  // wavefront past max_parts loads partition 0 (nparts <= max_parts always).
  const uint32_t ctx = (uint32_t)p.context_lens[seq];
  load_step(wave < p.max_parts ? wave : 0, p.max_parts);
  {
    // The asm needs every first-step value and the context length, so all
    // of those loads are issued before it (one round trip); without it the
    // compiler moves the partial loads past the branches on the context.
    float anchor = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      anchor += e[u].x + e[u].y;
#pragma unroll
      for (int k = 0; k < NDL; ++k) anchor += ov[u][k];
    }
    asm volatile("" ::"v"(anchor), "s"(ctx));
  }
  const bool live = ctx != 0 && ctx <= (uint32_t)p.max_seq_len;
  const int nparts = live ? ((int)ctx + p.partition - 1) / p.partition : 0;
  accumulate(wave, nparts);
  if (nparts <= 1) return;
  for (int i0 = wave + NW * U; i0 < nparts; i0 += NW * U) {
    load_step(i0, nparts);
    accumulate(i0, nparts);
  }
#pragma unroll
  for (int k = 0; k < NDL; ++k) s_acc[wave][lane + 64 * k] = acc[k];
  if (lane == 0) {
    s_m[wave] = mw;
    s_s[wave] = sw;
  }
  __syncthreads();
  const int d = threadIdx.x;
  if (d >= D) return;
  float M = s_m[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, s_m[w]);
  float num = 0.f, den = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float f = s_m[w] == -INFINITY ? 0.f : exp2f(s_m[w] - M);
    num += s_acc[w][d] * f;
    den += s_s[w] * f;
  }
  static_cast<QS*>(p.out)[row * D + d] = from_f32<QT>(num / (den + 1e-6f));
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

// Multiprocessor count of the current device, cached per device.
inline int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev] = n;
  }
  return cache[dev];
}

// Launches the persistent kernel (BS = 0: token rows) when the batch has
// enough items for it; *launched says whether it did.
// The grouped kernel when the batch fills it (at least two items of S
// sequences per CU), GQA groups fit S to the 16 columns and contexts fit its
// register-held block ids.
template <class QT, class CT, int D, int BS>
static hipError_t launch_grouped(const DecodeParams& p, hipStream_t stream, bool* launched) {
  *launched = false;
  constexpr int S = kGroupSeqs;
  constexpr int NW = GroupShape<CT, D>::kWaves, NB = kGroupBuffers;
  if (p.slices != 1 || p.group * S > 16 || p.max_seq_len > group_max_seq<NW>()) return hipSuccess;
  constexpr int NT = 64 * NW;
  static int per_cu = -1;
  if (per_cu < 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, paged_decode_group_kernel<QT, CT, D, BS, S, NW, NB>, NT, 0) !=
            hipSuccess ||
        n <= 0)
      n = 1;
    per_cu = n;
  }
  const int64_t items = (int64_t)((p.num_seqs + S - 1) / S) * p.num_kv_heads;
  const int64_t grid = (int64_t)device_cus() * std::min(per_cu, GroupShape<CT, D>::kPerCu);
  if (grid <= 0 || items < 2 * (int64_t)device_cus()) return hipSuccess;
  *launched = true;
  hipLaunchKernelGGL((paged_decode_group_kernel<QT, CT, D, BS, S, NW, NB>), dim3((unsigned)grid), dim3(NT), 0, stream,
                     p);
  return hipGetLastError();
}

template <class QT, class CT, int D, int BS>
static hipError_t launch_persistent(const DecodeParams& p, hipStream_t stream, bool* launched) {
  *launched = false;
  if (!p.persistent) return hipSuccess;
  // The grouped kernel's two job buffers leave no register room (it would
  // spill) above head size 128 and for 8-token blocks at 112 and above;
  // those keep the one-sequence kernel, as do float32 caches.
  constexpr bool kGroupable = BS > 0 && D <= 128 && !(BS == 8 && D >= 112) && !std::is_same<CT, F32>::value;
  if constexpr (kGroupable) {
    const hipError_t ge = launch_grouped<QT, CT, D, BS>(p, stream, launched);
    if (*launched || ge != hipSuccess) return ge;
  }
  constexpr int NT = 64 * Persist<D, BS == 0>::kWaves;
  static int per_cu = -1;  // resident workgroups per CU for this instantiation
  if (per_cu < 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, paged_decode_persist_kernel<QT, CT, D, BS>, NT, 0) !=
            hipSuccess ||
        n <= 0)
      n = 1;
    per_cu = n;
  }
  // Whole (sequence, unit) items, from one per resident workgroup; fewer,
  // longer items go to the partition path.  The grid never exceeds what is
  // resident at once, which the snake schedule assumes for its balance (not
  // for correctness).
  const int64_t items = (int64_t)p.num_seqs * p.units;
  const int64_t grid = (int64_t)device_cus() * per_cu;
  if (grid <= 0 || items < kPersistMinItemsPerWorkgroup * grid) return hipSuccess;
  *launched = true;
  hipLaunchKernelGGL((paged_decode_persist_kernel<QT, CT, D, BS>), dim3((unsigned)grid), dim3(NT), 0, stream, p);
  return hipGetLastError();
}

template <class QT, class CT, int D, int BS>
static hipError_t launch_one(const DecodeParams& p, hipStream_t stream) {
  bool launched = false;
  const hipError_t pe = launch_persistent<QT, CT, D, BS>(p, stream, &launched);
  if (launched || pe != hipSuccess) return pe;
  const int64_t nwg = (int64_t)p.max_parts * p.num_seqs * p.units;
  // Four wavefronts per workgroup at every grid size: eight for grids of
  // at most one workgroup per CU (one long sequence) measured no faster.
  hipLaunchKernelGGL((paged_decode_part_kernel<QT, CT, D, BS, kPartWaves>), dim3((unsigned)nwg), dim3(64 * kPartWaves),
                     0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.max_parts == 1 || p.counters != nullptr) return e;
  const int64_t rows = (int64_t)p.num_seqs * p.num_heads;
  hipLaunchKernelGGL((paged_decode_reduce_kernel<QT, D>), dim3((unsigned)rows), dim3(64 * kMergeWaves), 0, stream, p);
  return hipGetLastError();
}

template <class QT, class CT, int D>
static hipError_t launch_bs(const DecodeParams& p, int block_size, hipStream_t stream, bool* ok) {
  switch (block_size) {
    case 8: return launch_one<QT, CT, D, 8>(p, stream);
    case 16: return launch_one<QT, CT, D, 16>(p, stream);
    case 32: return launch_one<QT, CT, D, 32>(p, stream);
  }
  *ok = false;
  return hipErrorInvalidValue;
}

// Token-row layout: the persistent kernel in its token-row mode, else the
// token-row kernel plus the merge kernel when a sequence spans several
// partitions.
template <class QT, class CT, int D>
static hipError_t launch_rows(const DecodeParams& p, hipStream_t stream) {
  bool launched = false;
  const hipError_t pe = launch_persistent<QT, CT, D, 0>(p, stream, &launched);
  if (launched || pe != hipSuccess) return pe;
  const int64_t nwg = (int64_t)p.max_parts * p.num_seqs * p.units;
  hipLaunchKernelGGL((paged_decode_rows_kernel<QT, CT, D>), dim3((unsigned)nwg), dim3(64 * kPartWaves), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.max_parts == 1) return e;
  const int64_t rows = (int64_t)p.num_seqs * p.num_heads;
  hipLaunchKernelGGL((paged_decode_reduce_kernel<QT, D>), dim3((unsigned)rows), dim3(64 * kMergeWaves), 0, stream, p);
  return hipGetLastError();
}

// FP8 caches: paged 5-D layout only, head sizes that are multiples of x = 16.
// Float32 caches: paged 5-D layout only.
template <class QT, class CT, int D>
static hipError_t launch_layout(const DecodeParams& p, int block_size, hipStream_t stream, bool* ok) {
  if constexpr (std::is_same<CT, FP8>::value) {
    if constexpr (D % 16 != 0) {
      *ok = false;
      return hipErrorInvalidValue;
    } else {
      if (p.rows) {
        *ok = false;
        return hipErrorInvalidValue;
      }
      return launch_bs<QT, CT, D>(p, block_size, stream, ok);
    }
  } else if constexpr (std::is_same<CT, F32>::value) {
    if (p.rows) {  // float32 caches: paged layout only
      *ok = false;
      return hipErrorInvalidValue;
    }
    return launch_bs<QT, CT, D>(p, block_size, stream, ok);
  } else {
    if (p.rows) return launch_rows<QT, CT, D>(p, stream);
    return launch_bs<QT, CT, D>(p, block_size, stream, ok);
  }
}

template <class QT, class CT>
hipError_t launch_decode_typed(const DecodeParams& p, int head_size, int block_size, hipStream_t stream,
                               bool* ok) {
  switch (head_size) {
    case 32: return launch_layout<QT, CT, 32>(p, block_size, stream, ok);
    case 64: return launch_layout<QT, CT, 64>(p, block_size, stream, ok);
    case 80: return launch_layout<QT, CT, 80>(p, block_size, stream, ok);
    case 96: return launch_layout<QT, CT, 96>(p, block_size, stream, ok);
    case 112: return launch_layout<QT, CT, 112>(p, block_size, stream, ok);
    case 120: return launch_layout<QT, CT, 120>(p, block_size, stream, ok);
    case 128: return launch_layout<QT, CT, 128>(p, block_size, stream, ok);
    case 192: return launch_layout<QT, CT, 192>(p, block_size, stream, ok);
    case 256: return launch_layout<QT, CT, 256>(p, block_size, stream, ok);
  }
  *ok = false;
  return hipErrorInvalidValue;
}

}  // namespace pkv
