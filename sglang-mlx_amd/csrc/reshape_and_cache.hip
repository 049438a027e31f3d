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
//    token-minor, so one token's stores cannot be wider than one element).
//    Tokens that together fill a whole block in order (a prefill) instead
//    write slices of the block's regions as whole lines (below).
//  * FP8 caches (E4M3 codes of x / scale, either layout): see below.
//  * token-major (MHATokenPool / flash): K and V [num_slots, H, D].  A token's
//    K row and V row are each one contiguous H*D run in both source and
//    destination, so every lane moves 16-byte vectors and every wavefront
//    covers 1 KiB of one row.  Rows of at least 64 vectors go one token per
//    wavefront with nontemporal stores; shorter rows one token per
//    workgroup.
#include "pkv_fp8.h"
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

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// ---- paged 5-D layout, whole-block runs ------------------------------------------
// When bs consecutive batch tokens write slots blk*bs .. blk*bs + bs - 1 in
// order (a prefill writing whole blocks), the (block, head) region's K
// ([D/8][bs][8]) and V ([D][bs]) are each one contiguous run of D*bs
// elements that these tokens fill completely.  The wavefront of the run's
// token at offset `off` then writes slice `off` of each region: elements
// off*D .. off*D + D - 1, i.e. 16-byte units off*D/8 .. off*D/8 + D/8 - 1,
// gathered from the run's source rows.  Every unit is written once and
// whole, and the bs wavefronts of a run cover the region.  K unit u holds
// dimensions 8c .. 8c+7 of token t (u = c*bs + t); V unit u holds tokens
// 8g .. 8g+7 of dimension d (u = d*bs/8 + g).  The per-token path instead
// writes a token's V as single 2-byte elements 2*bs bytes apart, each a
// partial write of its line.  2-byte cache types (the kernel's ALIGNED
// case).
//
// The slices' stores are nontemporal: each store instruction writes whole
// lines that nothing in the launch reads back.  Measured on MI355X (same
// box, one library per policy): the radix-shared workload's first decode
// after its churn appends 84.0 -> 77.3 us per launch (the appends' lines no
// longer linger in the caches), the reference's fp16 append at 1024
// consecutive slots 4.33 -> 4.03 us, the churn append itself unchanged
// (26.9 us).  The per-token path keeps default stores: its 2-byte V stores
// rely on the L2 to combine them into lines (nontemporal, they made the
// churn append 4.5x slower).
template <class KT, class CT, int BS>
__device__ __forceinline__ void rac_run_slice(const RacParams& p, int64_t first, int off, int head, int64_t blk,
                                              int lane) {
  using KS = typename Elem<KT>::storage;
  using CS = typename Elem<CT>::storage;
  static_assert(Elem<CT>::kBytes == 2 && BS % 8 == 0, "16-byte units of 2-byte elements");
  constexpr int X = 8;
  const int D = p.head_size;
  const int per = D / X;  // units per wavefront and region
  const int64_t slice = (blk * p.num_heads + head) * (int64_t)D * BS + (int64_t)off * per * X;
  const int64_t hoff = (int64_t)head * D;
  const KS* key = static_cast<const KS*>(p.key);
  const KS* val = static_cast<const KS*>(p.value);
  // Each lane moves two neighbouring elements of the slice: one store
  // instruction writes 256 contiguous bytes of each region.
  for (int i = 2 * lane; i < D; i += 128) {
    const int u = off * per + i / X, e = i % X;
    // K: dimensions 8c + e, +1 of token t.
    const int c = u / BS, t = u % BS;
    const KS* ks = key + (first + t) * p.key_stride + hoff + X * c + e;
    // V: tokens 8g + e, +1 of dimension d.
    const int d = u / (BS / X), g = u % (BS / X);
    const KS* vs = val + (first + X * g + e) * p.value_stride + hoff + d;
    const uint32_t kw = pack2(convert_elem<KT, CT>(ks[0]), convert_elem<KT, CT>(ks[1]));
    const uint32_t vw = pack2(convert_elem<KT, CT>(vs[0]), convert_elem<KT, CT>(vs[p.value_stride]));
    __builtin_nontemporal_store(kw, reinterpret_cast<uint32_t*>(static_cast<CS*>(p.key_cache) + slice + i));
    __builtin_nontemporal_store(vw, reinterpret_cast<uint32_t*>(static_cast<CS*>(p.value_cache) + slice + i));
  }
}

// True when the token at batch position tok (slot `slot`, offset `off` in
// its block) lies in a whole-block run: positions tok - off .. tok - off +
// bs - 1 hold slots slot - off .. slot - off + bs - 1.  Wave-uniform; lanes
// 0 .. bs-1 each check one entry.
__device__ __forceinline__ bool rac_whole_block(const RacParams& p, int64_t tok, int32_t slot, int off, int lane) {
  const int bs = p.block_size;
  const int64_t first = tok - off;
  if (first < 0 || first + bs > p.num_tokens) return false;
  bool ok = true;
  if (lane < bs) ok = p.slot_mapping[first + lane] == slot - off + lane;
  return __all(ok);
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
  if constexpr (ALIGNED && Elem<CT>::kBytes == 2) {
    const int bs = p.block_size;
    // (Head sizes that are multiples of 8: whole 16-byte units per slice.)
    if ((bs == 8 || bs == 16 || bs == 32) && p.head_size % 8 == 0 && rac_whole_block(p, tok, slot, off, lane)) {
      if (bs == 8) rac_run_slice<KT, CT, 8>(p, tok - off, off, head, blk, lane);
      else if (bs == 16) rac_run_slice<KT, CT, 16>(p, tok - off, off, head, blk, lane);
      else rac_run_slice<KT, CT, 32>(p, tok - off, off, head, blk, lane);
      return;
    }
  }
  const int D = p.head_size;
  const KS* ksrc = static_cast<const KS*>(p.key) + tok * p.key_stride + (int64_t)head * D;
  const KS* vsrc = static_cast<const KS*>(p.value) + tok * p.value_stride + (int64_t)head * D;
  const int64_t region = ((int64_t)blk * p.num_heads + head) * (int64_t)D * p.block_size;
  CS* kdst = static_cast<CS*>(p.key_cache) + region;    // [D/X][bs][X]
  CS* vdst = static_cast<CS*>(p.value_cache) + region;  // [D][bs]
  const int nchunk = D / X;
  // K chunks of a large call are stored nontemporally (p.stream_k): a
  // token's 16-byte chunks sit bs*16 bytes apart, one per line, and a call
  // writing more K than one XCD's L2 holds (4 MiB) has its lines evicted
  // before a later token fills their neighbours.  Measured on MI355X at
  // 4096 random slots (8 MiB of K): 76.4 -> 65.0 us.  A small call keeps
  // default stores (the reference's append of 8 tokens, rewritten back to
  // back: 2.45 us default, 3.1 us nontemporal).  V's 2-byte stores keep
  // default stores: the L2 combines the tokens of a block into lines.
  if (ALIGNED && p.stream_k) {
    for (int c = lane; c < nchunk; c += 64)
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, load_vec16<KT, CT>(ksrc + c * X)),
                                  reinterpret_cast<u32x4_t*>(kdst + ((int64_t)c * p.block_size + off) * X));
  } else {
    for (int c = lane; c < nchunk; c += 64)
      convert_run<KT, CT, X, ALIGNED>(ksrc + c * X, kdst + ((int64_t)c * p.block_size + off) * X);
  }
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
// The source rows are loaded with the nontemporal policy when no conversion
// is needed: each is read once.

// Measured at 4096 tokens x 8 heads x D 128, bf16, 65,536 slots (median of
// interleaved runs, one process per variant): one token per wavefront, four
// wavefronts per workgroup, default-policy source loads 6.64 us; with
// nontemporal source loads (each source row is read once) 6.29 us; two or
// eight wavefronts per workgroup 6.62 / 6.60 us; two tokens per wavefront
// 6.85 us; one wavefront per (token, head) 9.68 us.
constexpr int kRacWaves = 4;  // wavefronts (tokens) per workgroup

template <class KT, class CT>
__device__ __forceinline__ uint4 load_src16(const typename Elem<KT>::storage* src) {
  if constexpr (std::is_same<KT, CT>::value) {
    return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src)));
  } else {
    return load_vec16<KT, CT>(src);
  }
}

template <class KT, class CT, int NV>
__global__ __launch_bounds__(64 * kRacWaves) void rac_token_major_wave_kernel(RacParams p) {
  using KS = typename Elem<KT>::storage;
  using CS = typename Elem<CT>::storage;
  constexpr int VE = 16 / Elem<CT>::kBytes;  // elements per 16-byte cache vector
  constexpr int TPW = 1;  // tokens per wavefront
  const int lane = threadIdx.x & 63;
  const int tok0 = ((int)blockIdx.x * kRacWaves + (int)(threadIdx.x >> 6)) * TPW;
  const int row = p.num_heads * p.head_size;
  const int nvec = row / VE;  // 64 * (NV/2) < nvec <= 64 * NV
  uint4 kx[TPW][NV], vx[TPW][NV];
  int32_t slot[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int tok = tok0 + u;
    // Wavefronts past the last token stay for the barrier and move nothing.
    const bool live = tok < p.num_tokens;
    slot[u] = live ? p.slot_mapping[tok] : -1;
    const KS* ksrc = static_cast<const KS*>(p.key) + (int64_t)tok * p.key_stride;
    const KS* vsrc = static_cast<const KS*>(p.value) + (int64_t)tok * p.value_stride;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
      const int i = 64 * c + lane;
      const bool ok = live && i < nvec;
      kx[u][c] = ok ? load_src16<KT, CT>(ksrc + i * VE) : make_uint4(0, 0, 0, 0);
      vx[u][c] = ok ? load_src16<KT, CT>(vsrc + i * VE) : make_uint4(0, 0, 0, 0);
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    if (slot[u] >= 0 && (int64_t)slot[u] < p.num_slots) {
      CS* kdst = static_cast<CS*>(p.key_cache) + (int64_t)slot[u] * row;
      CS* vdst = static_cast<CS*>(p.value_cache) + (int64_t)slot[u] * row;
#pragma unroll
      for (int c = 0; c < NV; ++c) {
        const int i = 64 * c + lane;
        if (i < nvec) {
          __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, kx[u][c]), reinterpret_cast<u32x4_t*>(kdst + i * VE));
          __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, vx[u][c]), reinterpret_cast<u32x4_t*>(vdst + i * VE));
        }
      }
    }
  }
}

// ---- FP8 caches -------------------------------------------------------------------
// E4M3 codes of x / scale (pkv_fp8.h).  Token-major: one wavefront per
// token, each lane turning 8 source elements into 8 code bytes per step of
// the K row and of the V row.  Paged 5-D (x = 16): one wavefront per
// (token, head), K as 16-byte chunks, V as single bytes (token-minor layout).
__device__ __forceinline__ float fp8_scaled(float x, float scale, float inv, bool pow2) {
  return pow2 ? x * inv : __fdiv_rn(x, scale);
}

template <class KT>
__device__ __forceinline__ uint2 encode8(const typename Elem<KT>::storage* __restrict__ src, float scale, float inv,
                                         bool pow2) {
  float v[8];
  if constexpr (std::is_same<KT, F32>::value) {
    const float4 a = reinterpret_cast<const float4*>(src)[0], b = reinterpret_cast<const float4*>(src)[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  } else {
    const uint4 w = *reinterpret_cast<const uint4*>(src);
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = to_f32<KT>((uint16_t)(u[i] & 0xffffu));
      v[2 * i + 1] = to_f32<KT>((uint16_t)(u[i] >> 16));
    }
  }
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo |= fp8_e4m3_encode(fp8_scaled(v[i], scale, inv, pow2)) << (8 * i);
    hi |= fp8_e4m3_encode(fp8_scaled(v[4 + i], scale, inv, pow2)) << (8 * i);
  }
  return make_uint2(lo, hi);
}

template <class KT>
__global__ __launch_bounds__(256) void rac_fp8_token_major_kernel(RacParams p) {
  using KS = typename Elem<KT>::storage;
  const int lane = threadIdx.x & 63;
  const int64_t tok = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= p.num_tokens) return;
  const int32_t slot = p.slot_mapping[tok];
  if (slot < 0 || (int64_t)slot >= p.num_slots) return;
  const int row = p.num_heads * p.head_size;  // a multiple of 8
  const int n8 = row / 8;
  const bool pow2 = p.scales_pow2 != 0;
  const KS* ksrc = static_cast<const KS*>(p.key) + tok * p.key_stride;
  const KS* vsrc = static_cast<const KS*>(p.value) + tok * p.value_stride;
  uint8_t* kdst = static_cast<uint8_t*>(p.key_cache) + (int64_t)slot * row;
  uint8_t* vdst = static_cast<uint8_t*>(p.value_cache) + (int64_t)slot * row;
  for (int i = lane; i < n8; i += 64) {
    const uint2 k = encode8<KT>(ksrc + 8 * i, p.k_scale, p.k_inv, pow2);
    const uint2 v = encode8<KT>(vsrc + 8 * i, p.v_scale, p.v_inv, pow2);
    __builtin_nontemporal_store(k.x, reinterpret_cast<uint32_t*>(kdst + 8 * i));
    __builtin_nontemporal_store(k.y, reinterpret_cast<uint32_t*>(kdst + 8 * i) + 1);
    __builtin_nontemporal_store(v.x, reinterpret_cast<uint32_t*>(vdst + 8 * i));
    __builtin_nontemporal_store(v.y, reinterpret_cast<uint32_t*>(vdst + 8 * i) + 1);
  }
}

// Whole-block runs over FP8 caches (block sizes 16 and 32): as
// rac_run_slice, with 16-byte units of 16 codes -- K unit u = c*bs + t
// (dimensions 16c .. 16c+15 of token t), V unit u = d*bs/16 + g (tokens
// 16g .. 16g+15 of dimension d); D/16 units (D bytes) per wavefront and
// region.  Each lane encodes two neighbouring codes of the slice, so one
// store instruction writes D/64 x 128 contiguous bytes and the encodes
// spread over the whole wavefront.
template <class KT, int BS>
__device__ __forceinline__ void rac_fp8_run_slice(const RacParams& p, int64_t first, int off, int head, int64_t blk,
                                                  int lane) {
  using KS = typename Elem<KT>::storage;
  static_assert(BS % 16 == 0, "16-byte units of 16 codes");
  const int D = p.head_size;
  const int per = D / 16;
  const bool pow2 = p.scales_pow2 != 0;
  const int64_t region = (blk * p.num_heads + head) * (int64_t)D * BS;
  const int64_t slice = region + (int64_t)off * per * 16;
  const int64_t hoff = (int64_t)head * D;
  const KS* key = static_cast<const KS*>(p.key);
  const KS* val = static_cast<const KS*>(p.value);
  for (int i = 2 * lane; i < D; i += 128) {
    const int u = off * per + i / 16, b = i % 16;
    // K: dimensions 16c + b, +1 of token t.
    const int c = u / BS, t = u % BS;
    const KS* ks = key + (first + t) * p.key_stride + hoff + 16 * c + b;
    const uint32_t k0 = fp8_e4m3_encode(fp8_scaled(to_f32<KT>(ks[0]), p.k_scale, p.k_inv, pow2));
    const uint32_t k1 = fp8_e4m3_encode(fp8_scaled(to_f32<KT>(ks[1]), p.k_scale, p.k_inv, pow2));
    // V: tokens 16g + b, +1 of dimension d.
    const int d = u / (BS / 16), g = u % (BS / 16);
    const KS* vs = val + (first + 16 * g + b) * p.value_stride + hoff + d;
    const uint32_t v0 = fp8_e4m3_encode(fp8_scaled(to_f32<KT>(vs[0]), p.v_scale, p.v_inv, pow2));
    const uint32_t v1 = fp8_e4m3_encode(fp8_scaled(to_f32<KT>(vs[p.value_stride]), p.v_scale, p.v_inv, pow2));
    __builtin_nontemporal_store((uint16_t)(k0 | (k1 << 8)),
                                reinterpret_cast<uint16_t*>(static_cast<uint8_t*>(p.key_cache) + slice + i));
    __builtin_nontemporal_store((uint16_t)(v0 | (v1 << 8)),
                                reinterpret_cast<uint16_t*>(static_cast<uint8_t*>(p.value_cache) + slice + i));
  }
}

template <class KT>
__global__ __launch_bounds__(256) void rac_fp8_paged5d_kernel(RacParams p) {
  using KS = typename Elem<KT>::storage;
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= p.num_tokens * p.num_heads) return;
  const int64_t tok = wid / p.num_heads;
  const int head = (int)(wid - tok * p.num_heads);
  const int32_t slot = p.slot_mapping[tok];
  if (slot < 0 || (int64_t)slot >= p.num_slots) return;
  const int64_t blk = slot / p.block_size;
  const int off = slot - (int)blk * p.block_size;
  const int D = p.head_size;  // a multiple of 16
  if ((p.block_size == 16 || p.block_size == 32) && rac_whole_block(p, tok, slot, off, lane)) {
    if (p.block_size == 16) rac_fp8_run_slice<KT, 16>(p, tok - off, off, head, blk, lane);
    else rac_fp8_run_slice<KT, 32>(p, tok - off, off, head, blk, lane);
    return;
  }
  const bool pow2 = p.scales_pow2 != 0;
  const KS* ksrc = static_cast<const KS*>(p.key) + tok * p.key_stride + (int64_t)head * D;
  const KS* vsrc = static_cast<const KS*>(p.value) + tok * p.value_stride + (int64_t)head * D;
  const int64_t region = ((int64_t)blk * p.num_heads + head) * (int64_t)D * p.block_size;
  uint8_t* kdst = static_cast<uint8_t*>(p.key_cache) + region;    // [D/16][bs][16]
  uint8_t* vdst = static_cast<uint8_t*>(p.value_cache) + region;  // [D][bs]
  for (int c = lane; c < D / 8; c += 64) {  // 8-element halves of the 16-byte chunks
    const uint2 k = encode8<KT>(ksrc + 8 * c, p.k_scale, p.k_inv, pow2);
    *reinterpret_cast<uint2*>(kdst + ((int64_t)(c >> 1) * p.block_size + off) * 16 + (c & 1) * 8) = k;
  }
  for (int d = lane; d < D; d += 64)
    vdst[(int64_t)d * p.block_size + off] =
        (uint8_t)fp8_e4m3_encode(fp8_scaled(to_f32<KT>(vsrc[d]), p.v_scale, p.v_inv, pow2));
}

template <class KT>
static hipError_t launch_rac_fp8(const RacParams& p, hipStream_t stream) {
  if (p.layout == 0) {
    const int64_t waves = p.num_tokens * p.num_heads;
    hipLaunchKernelGGL((rac_fp8_paged5d_kernel<KT>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream, p);
  } else {
    hipLaunchKernelGGL((rac_fp8_token_major_kernel<KT>), dim3((unsigned)((p.num_tokens + 3) / 4)), dim3(256), 0,
                       stream, p);
  }
  return hipGetLastError();
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
    // The one-wavefront-per-token kernels index tokens with 32-bit ints
    // (a workgroup covers at most 64 tokens).
    const int nvec = (vec && p.num_tokens <= INT32_MAX - 64) ? row / VE : 0;
    const dim3 wgrid((unsigned)((p.num_tokens + kRacWaves - 1) / kRacWaves));
    if (vec && nvec > 64 && nvec <= 128)
      hipLaunchKernelGGL((rac_token_major_wave_kernel<KT, CT, 2>), wgrid, dim3(64 * kRacWaves), 0, stream, p);
    else if (vec && nvec > 128 && nvec <= 256)
      hipLaunchKernelGGL((rac_token_major_wave_kernel<KT, CT, 4>), wgrid, dim3(64 * kRacWaves), 0, stream, p);
    else if (vec && nvec > 256 && nvec <= 512)
      hipLaunchKernelGGL((rac_token_major_wave_kernel<KT, CT, 8>), wgrid, dim3(64 * kRacWaves), 0, stream, p);
    else if (vec && nvec > 512 && nvec <= 1024)
      hipLaunchKernelGGL((rac_token_major_wave_kernel<KT, CT, 16>), wgrid, dim3(64 * kRacWaves), 0, stream, p);
    else if (vec)
      hipLaunchKernelGGL((rac_token_major_kernel<KT, CT, VE, true>), grid, dim3(threads), 0, stream, p);
    else
      hipLaunchKernelGGL((rac_token_major_kernel<KT, CT, 1, false>), grid, dim3(threads), 0, stream, p);
  }
  return hipGetLastError();
}

hipError_t launch_reshape_and_cache(const RacParams& params, bool aligned, hipStream_t stream) {
  if (params.num_tokens == 0) return hipSuccess;
  RacParams p = params;
  const int64_t cache_elem = p.cache_dtype == kF32 ? 4 : p.cache_dtype == kFP8 ? 1 : 2;
  p.stream_k = p.num_tokens * p.num_heads * p.head_size * cache_elem >= kRacStreamKBytes;
  const int kt = p.kv_dtype, ct = p.cache_dtype;
  if (kt == kF32 && ct == kF32) return launch_rac_typed<F32, F32>(p, aligned, stream);
  if (kt == kF16 && ct == kF16) return launch_rac_typed<F16, F16>(p, aligned, stream);
  if (kt == kBF16 && ct == kBF16) return launch_rac_typed<BF16, BF16>(p, aligned, stream);
  if (kt == kF32 && ct == kF16) return launch_rac_typed<F32, F16>(p, aligned, stream);
  if (kt == kF32 && ct == kBF16) return launch_rac_typed<F32, BF16>(p, aligned, stream);
  if (ct == kFP8) {
    if (!aligned) return hipErrorInvalidValue;  // the ABI checks alignment first
    if (kt == kF32) return launch_rac_fp8<F32>(p, stream);
    if (kt == kF16) return launch_rac_fp8<F16>(p, stream);
    if (kt == kBF16) return launch_rac_fp8<BF16>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace pkv
