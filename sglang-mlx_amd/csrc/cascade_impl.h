// Shared-prefix (cascade) decode attention for gfx950, paged 5-D layout.
//
// Semantics are those of paged_attention_v1 (paged_attention_kernels.metal:
// 37-168 of the reference): per (sequence, query head), softmax over the
// first ctx tokens of scale * q.k (+ alibi), weighted sum of V, denominator
// sum + 1e-6, zero rows for ctx == 0 or ctx > max_seq_len.  The cascade only
// changes where the work is done.  Sequences whose block tables begin with
// the same blocks (a radix-shared prefix) are listed by the host in a plan
// (CascadeParams), and two kernels run:
//
// paged_cascade_kernel -- workgroups of 4 wavefronts in two roles, sized so
//   that one of each shares a CU (LDS below half a CU's, at most 256 VGPRs
//   per wavefront): the compute-bound prefix work and the HBM-bound tail
//   work overlap.
//   * Prefix role (workgroups 0 .. plan tiles x KV heads - 1): one plan
//     tile's query rows (members x GQA heads, up to 128; each wavefront 32
//     rows as two 16-column MFMA query sets held in registers) against one
//     chunk of the group's prefix.  The chunk's K and V are staged through
//     LDS two tiles of 16 tokens at a time (16-bit caches: four buffers,
//     the scores of the next pair computed while the current pair's
//     softmax runs) by direct-to-LDS buffer loads, in the order the MFMA
//     operands want; every K/V byte is read from HBM (or L2) once per
//     workgroup and from LDS once per wavefront, and feeds 32 query rows
//     there.  FP8 codes are dequantised once per stage into a 16-bit LDS
//     image.  Scores S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_16x16x32
//     over tile pairs, online softmax in the log2 domain; each row's
//     partial state (max, sum, unnormalised output) goes to the workspace
//     slot of its (sequence, head, chunk).
//   * Tail role (the rest): one wavefront per (tail partition, KV head)
//     item, longest partition first: the partition's tokens (after the
//     sequence's prefix) through the one-sequence tile pipeline.  A
//     sequence with no prefix and a single partition gets its output row
//     written here; otherwise the partition's state goes to the workspace.
// paged_cascade_merge_kernel -- sixteen lanes per row (D/16 dimensions
//   each) of the rows the tail role did not write: the row's tail
//   partitions' and prefix chunks' states folded by log-sum-exp in that
//   fixed order, the row written.  States cross workgroups here, so they
//   meet at the launch boundary rather than inside the first kernel, where
//   the merge's dependent loads would queue behind the tail's streaming.
//
// The log-sum-exp merge of partial states is an identity with one softmax
// over all tokens (the final denominator is taken against the true maximum,
// as the reference's), so the cascade returns paged_attention_v1's result
// within floating-point rounding.
#pragma once

#include "paged_decode_impl.h"

namespace pkv {

constexpr int kCascadeWaves = 4;                               // wavefronts per workgroup, both roles
constexpr int kPrefixSets = 2;                                 // 16-column query sets per wavefront
constexpr int kPrefixRows = kCascadeWaves * kPrefixSets * 16;  // query rows per prefix workgroup
constexpr int kPrefixStageTiles = 2;                           // 16-token tiles per LDS stage (one pair)
// LDS stage buffers of 16-bit caches: four, so that a step can read the
// next stage's K for its look-ahead scores while two later stages load
// (67.6 KB of LDS per workgroup, two workgroups per CU).  FP8 caches stage
// through two code buffers and two 16-bit images instead.
constexpr int kPrefixBuffers = 4;
constexpr int kTailBuffers = 2;                                // tile buffers per tail wavefront

// Largest block-table span of one prefix chunk (8-token blocks).
constexpr int kPrefixMaxBlocks = kMaxPrefixChunk / 8;

// LDS image of one staged 16-token tile, in 16-byte units.
//   16-bit caches: K unit c8 * 16 + t = dimensions 8 c8 .. +7 of token t;
//                  V unit 2d + h     = tokens 8h .. 8h+7 of dimension d.
//   FP8 caches (codes): K unit c16 * 16 + t = dimensions 16 c16 .. +15 of
//                  token t; V unit d = tokens 0 .. 15 of dimension d.
// Every 64 consecutive units come from one (block, head) region of the
// cache (one block with blocks of 16 and more; a half tile's block, by lane,
// with 8-token blocks), so a wavefront stages a tile with direct-to-LDS
// buffer loads, lane l of a load writing unit l of its 64.
template <class CT, int D> struct PrefixTile {
  static constexpr bool kF8 = std::is_same<CT, FP8>::value;
  static constexpr int kKUnits = kF8 ? D : 2 * D;
  static constexpr int kVUnits = kF8 ? D : 2 * D;
  static constexpr int kUnits = kKUnits + kVUnits;
  static_assert(kKUnits % 64 == 0 && kVUnits % 64 == 0, "whole 64-unit loads");
};

// A lane's MFMA operands of a staged tile pair (A, B) (16-bit caches as
// loaded; FP8 codes dequantised exactly into MT):
//   ka / kb[j]: K operand of k-step j (token col, dimensions 32j + 8g .. +7);
//   v[dt]:      the PV operand of dimension tile dt over the pair's 32
//               tokens, k-index 8g + e = token 4g + e of A (e < 4) and of B
//               (e >= 4): dimension 16dt + col.
template <class CT, class MT, int D> struct PrefixOperands {
  uint4 ka[Tile<D>::KSTEPS], kb[Tile<D>::KSTEPS];
  uint4 v[Tile<D>::DT];
};

template <class CT, class MT, int D>
__device__ __forceinline__ void read_pair(PrefixOperands<CT, MT, D>& op, const uint4* ta, const uint4* tb, int lane,
                                          int g, int col) {
  using PT = PrefixTile<CT, D>;
  constexpr int KSTEPS = Tile<D>::KSTEPS, DT = Tile<D>::DT;
  if constexpr (!PT::kF8) {
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) {
      op.ka[j] = ta[64 * j + lane];
      op.kb[j] = tb[64 * j + lane];
    }
    const char* va = reinterpret_cast<const char*>(ta + PT::kKUnits);
    const char* vb = reinterpret_cast<const char*>(tb + PT::kKUnits);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int o = (16 * dt + col) * 32 + 8 * g;
      const uint2 x = *reinterpret_cast<const uint2*>(va + o), y = *reinterpret_cast<const uint2*>(vb + o);
      op.v[dt] = make_uint4(x.x, x.y, y.x, y.y);
    }
  } else {
    uint2 ka8[KSTEPS], kb8[KSTEPS];
    uint32_t va8[DT], vb8[DT];
    const char* ka_ = reinterpret_cast<const char*>(ta);
    const char* kb_ = reinterpret_cast<const char*>(tb);
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) {
      const int o = ((2 * j + (g >> 1)) * 16 + col) * 16 + (g & 1) * 8;
      ka8[j] = *reinterpret_cast<const uint2*>(ka_ + o);
      kb8[j] = *reinterpret_cast<const uint2*>(kb_ + o);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int o = PT::kKUnits * 16 + (16 * dt + col) * 16 + 4 * g;
      va8[dt] = *reinterpret_cast<const uint32_t*>(ka_ + o);
      vb8[dt] = *reinterpret_cast<const uint32_t*>(kb_ + o);
    }
    // Exponent-15 codes (the reference's inf / NaN) take the exact path;
    // one wave-wide test for the pair.
    uint32_t probe = 0;
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) probe |= fp8x4_special(ka8[j].x) | fp8x4_special(ka8[j].y) |
                                              fp8x4_special(kb8[j].x) | fp8x4_special(kb8[j].y);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) probe |= fp8x4_special(va8[dt]) | fp8x4_special(vb8[dt]);
    const bool special = __any(probe != 0u);
    auto cvt = [&](uint32_t w) { return special ? fp8x4_exact<MT>(w) : fp8x4_cvt<MT>(w); };
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) {
      uint2 lo = cvt(ka8[j].x), hi = cvt(ka8[j].y);
      op.ka[j] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      lo = cvt(kb8[j].x), hi = cvt(kb8[j].y);
      op.kb[j] = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint2 x = cvt(va8[dt]), y = cvt(vb8[dt]);
      op.v[dt] = make_uint4(x.x, x.y, y.x, y.y);
    }
  }
}

// Stages part PART (0: the K units, 1: the V units) of tokens tt0 ..
// tt0+15 of the (block, head) regions at `base` into the LDS tile `dst`:
// b0 is the block of tokens 0 .. 7 and b1 of 8 .. 15 (equal with blocks of
// 16 and more; -1: outside the pool or past the chunk).  A block of -1 gets
// a zero-sized buffer resource, so its units read as zeros.  Returns the
// tile's live-token mask (bit i = token i).
template <class CT, int D, int BS, int PART>
__device__ __forceinline__ uint32_t stage_part(uint4* dst, const typename Elem<CT>::storage* base, int64_t block_stride,
                                               int b0, int b1, int tt0, int lane) {
  using PT = PrefixTile<CT, D>;
  constexpr int EB = Elem<CT>::kBytes;
  constexpr int REGION = D * BS * EB;  // bytes of one (block, head) region of K (and of V)
  typedef __attribute__((address_space(3))) void* lds_ptr;
  auto rsrc = [&](int b) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)(base + (int64_t)(b < 0 ? 0 : b) * block_stride), (short)0,
                                             b < 0 ? 0 : REGION, kBufferRsrcWord3);
  };
  const int hi = lane >> 4, t = lane & 15;
  uint4* out = dst + (PART == 0 ? 0 : PT::kKUnits);
  constexpr int LOADS = (PART == 0 ? PT::kKUnits : PT::kVUnits) / 64;
  if constexpr (BS >= kTile) {
    const int off = tt0 % BS;
    const __amdgpu_buffer_rsrc_t r = rsrc(b0);
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      if constexpr (PART == 0)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(out + 64 * j), 16, ((4 * j + hi) * BS + t) * 16, off * 16,
                                                 0, 0);
      else if constexpr (PT::kF8)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(out + 64 * j), 16, (64 * j + lane) * BS, off, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)(out + 64 * j), 16,
                                                 ((32 * j + (lane >> 1)) * BS + 8 * (lane & 1)) * 2, off * 2, 0, 0);
    }
  } else {
    static_assert(!PT::kF8, "FP8 caches with 8-token blocks are not staged");
    // 8-token blocks: each load goes out twice, to the lanes of each half
    // tile with that half's block.
    const __amdgpu_buffer_rsrc_t r0 = rsrc(b0), r1 = rsrc(b1);
    const bool first = PART == 0 ? t < 8 : (lane & 1) == 0;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int vo = PART == 0 ? ((4 * j + hi) * BS + (t & 7)) * 16 : (32 * j + (lane >> 1)) * BS * 2;
      if (first)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r0, (lds_ptr)(out + 64 * j), 16, vo, 0, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r1, (lds_ptr)(out + 64 * j), 16, vo, 0, 0, 0);
    }
  }
  return (b0 >= 0 ? 0x00ffu : 0u) | (b1 >= 0 ? 0xff00u : 0u);
}


// The merge kernel's per-lane state: its row's running maximum and weight
// sum (the same in each of the row's lanes, so no lane exchange is needed)
// and the unnormalised output of the lane's NC four-dimension chunks
// (dimensions 4 (e + 16 k) .. +3 for chunk k of lane e of the row).
constexpr int kMergeLanesPerRow = 16;
template <int D> struct MergeAcc {
  static_assert(D % (4 * kMergeLanesPerRow) == 0, "whole four-dimension chunks per lane");
  static constexpr int NC = D / (4 * kMergeLanesPerRow);
  float m, l;
  float4 o[NC];
};

// Folds one partial state (maximum m, weight sum l against it, the lane's
// chunks o of the unnormalised output) into acc, whose m is its true
// maximum: acc rescaled onto max(acc.m, m), then the state added with
// weight exp2(m - acc.m).  States whose maximum is -inf hold no tokens.
template <int D>
__device__ __forceinline__ void fold_partial(MergeAcc<D>& acc, float m, float l, const float4 (&o)[MergeAcc<D>::NC]) {
  if (m == -INFINITY) return;
  if (m > acc.m) {
    const float f = acc.m == -INFINITY ? 0.f : exp2f(acc.m - m);
    acc.l *= f;
#pragma unroll
    for (int k = 0; k < MergeAcc<D>::NC; ++k) {
      acc.o[k].x *= f;
      acc.o[k].y *= f;
      acc.o[k].z *= f;
      acc.o[k].w *= f;
    }
    acc.m = m;
  }
  const float w = exp2f(m - acc.m);
#pragma unroll
  for (int k = 0; k < MergeAcc<D>::NC; ++k) {
    acc.o[k].x += w * o[k].x;
    acc.o[k].y += w * o[k].y;
    acc.o[k].z += w * o[k].z;
    acc.o[k].w += w * o[k].w;
  }
  acc.l += w * l;
}

// The lane's chunks of state slot `slot` of a workspace (ml: maxima and
// sums, o: unnormalised outputs).
template <int D>
__device__ __forceinline__ void load_state(const float* ml, const float* o, int64_t slot, int e, float2& st_ml,
                                           float4 (&st_o)[MergeAcc<D>::NC]) {
  st_ml = *reinterpret_cast<const float2*>(ml + slot * 2);
#pragma unroll
  for (int k = 0; k < MergeAcc<D>::NC; ++k)
    st_o[k] = *reinterpret_cast<const float4*>(o + slot * D + 4 * (e + kMergeLanesPerRow * k));
}

// Folds the n states of one row into acc, in order: tail partitions 0 ..
// np-1 (ws_tail_*, slots tail0 + k), then prefix chunks (ws_*, slots
// chunk0 + j); n = 0 on lanes without a row.  NB states' loads are in
// flight at a time.
template <int D, int NB>
__device__ __forceinline__ void fold_states(MergeAcc<D>& acc, const CascadeParams& c, int64_t tail0, int np,
                                            int64_t chunk0, int n, int e) {
  constexpr int NC = MergeAcc<D>::NC;
  for (int j0 = 0; j0 < n; j0 += NB) {
    float2 ml[NB];
    float4 o[NB][NC];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      ml[b] = make_float2(-INFINITY, 0.f);
#pragma unroll
      for (int k = 0; k < NC; ++k) o[b][k] = make_float4(0.f, 0.f, 0.f, 0.f);
      const int j = j0 + b;
      if (j < n) {
        const bool tail = j < np;
        load_state<D>(tail ? c.ws_tail_ml : c.ws_ml, tail ? c.ws_tail_o : c.ws_o, tail ? tail0 + j : chunk0 + (j - np),
                      e, ml[b], o[b]);
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) fold_partial<D>(acc, ml[b].x, ml[b].y, o[b]);
  }
}


// The prefix length a sequence's rows take from the plan: 0 when the
// sequence is not live, has no prefix, or the plan's value cannot be used
// (not a multiple of the tile alignment, or beyond the workspace's chunks);
// the context is then streamed whole.  The tail and merge kernels decide
// alike.
template <int BS>
__device__ __forceinline__ int usable_prefix_of(const CascadeParams& c, int plan_len, bool live) {
  constexpr int ALIGN = BS < kTile ? BS : kTile;  // a tail starts on a tile boundary of its blocks
  const int pre = live ? plan_len : 0;
  return (pre < 0 || pre % ALIGN != 0 || pre > c.max_chunks * c.chunk) ? 0 : pre;
}
template <int BS>
__device__ __forceinline__ int usable_prefix(const CascadeParams& c, int seq, bool live) {
  return usable_prefix_of<BS>(c, live ? c.prefix_lens[seq] : 0, live);
}

// Tail partitions of a sequence whose tail (tokens after the prefix) is
// `tail` tokens long: at least one, so that every sequence's row is written.
__device__ __forceinline__ int tail_parts(const CascadeParams& c, int tail) {
  return tail <= c.part_tokens ? 1 : (tail + c.part_tokens - 1) / c.part_tokens;
}

// FP8 stages are dequantised once, by the whole workgroup, into a 16-bit
// image of the stage in MT's layout (PrefixTile<MT, D>) that every
// wavefront then reads as it would a 16-bit cache's stage: thread t takes
// code units t, t + NT, ... of the stage's two tiles (K unit c16 * 16 + tk ->
// image units (2 c16) * 16 + tk and (2 c16 + 1) * 16 + tk; V unit d -> image
// units 2 d and 2 d + 1).  Exponent-15 codes take the exact path (one
// wave-wide test).  Conversion per wavefront and tile pair drops to a quarter
// of what reading the codes in every wavefront costs.
template <class MT, int D, int NT>
__device__ __forceinline__ void convert_stage(const uint4 (*codes)[PrefixTile<FP8, D>::kUnits],
                                              uint4 (*img)[PrefixTile<MT, D>::kUnits], int tid) {
  constexpr int CU = PrefixTile<FP8, D>::kUnits;  // code units per tile: D of K, D of V
  constexpr int IK = PrefixTile<MT, D>::kKUnits;  // image K units per tile (2 D)
  static_assert((kPrefixStageTiles * CU) % NT == 0, "whole code units per thread");
#pragma unroll
  for (int u0 = 0; u0 < kPrefixStageTiles * CU; u0 += NT) {
    const int u = u0 + tid;
    const int tile = u / CU, r = u - tile * CU;
    const uint4 w = codes[tile][r];
    const uint32_t probe = fp8x4_special(w.x) | fp8x4_special(w.y) | fp8x4_special(w.z) | fp8x4_special(w.w);
    const bool special = __any(probe != 0u);
    auto cvt = [&](uint32_t x) __attribute__((always_inline)) {
      return special ? fp8x4_exact_inline<MT>(x) : fp8x4_cvt<MT>(x);
    };
    const uint2 a = cvt(w.x), b = cvt(w.y), c = cvt(w.z), d = cvt(w.w);
    int i0, i1;
    if (r < D) {  // K: dimensions 16 c16 .. +15 of token tk
      const int c16 = r >> 4, tk = r & 15;
      i0 = (2 * c16) * 16 + tk;
      i1 = i0 + 16;
    } else {      // V: tokens 0 .. 15 of dimension r - D
      i0 = IK + 2 * (r - D);
      i1 = i0 + 1;
    }
    img[tile][i0] = make_uint4(a.x, a.y, b.x, b.y);
    img[tile][i1] = make_uint4(c.x, c.y, d.x, d.y);
  }
}

// Prefix role: plan tile `wi`, KV head `kvh` (see the file comment).
template <class QT, class CT, int D, int BS>
__device__ __forceinline__ void prefix_role(const DecodeParams& p, const CascadeParams& c, int wi, int kvh,
                                            uint4 (*s_buf0)[PrefixTile<CT, D>::kUnits],
                                            uint4 (*s_buf1)[PrefixTile<CT, D>::kUnits],
                                            uint4 (*s_buf2)[PrefixTile<CT, D>::kUnits],
                                            uint4 (*s_buf3)[PrefixTile<CT, D>::kUnits],
                                            uint4 (*s_img0)[PrefixTile<typename MmaOf<QT, CT>::type, D>::kUnits],
                                            uint4 (*s_img1)[PrefixTile<typename MmaOf<QT, CT>::type, D>::kUnits],
                                            int32_t* s_blk, uint32_t (*s_live)[kPrefixStageTiles],
                                            uint32_t (*s_ilive)[kPrefixStageTiles]) {
  using MT = typename MmaOf<QT, CT>::type;
  using CS = typename Elem<CT>::storage;
  using PT = PrefixTile<CT, D>;
  constexpr int NW = kCascadeWaves, NS = kPrefixSets, ST = kPrefixStageTiles;
  constexpr int NT = 64 * NW;
  constexpr int KSTEPS = Tile<D>::KSTEPS;
  constexpr int DT = Tile<D>::DT;
  static_assert(ST == 2 && NW == 2 * ST, "wavefront w stages part w % 2 of tile w / 2; one pair per stage");
  static_assert(PT::kKUnits == PT::kVUnits, "K and V parts stage alike");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, col = lane & 15;
  const int4 e = c.tiles[wi];
  const int mb = e.x, mc = e.y, t0 = e.z;
  // A malformed tile (the host builds them) is skipped, never read past.
  const int tcap = p.max_blocks_per_seq * BS;
  const int t1 = min(e.w, tcap);
  if (mb < 0 || mc <= 0 || mb > c.num_members - mc || mc * p.group > kPrefixRows || t0 < 0 || t0 >= t1 ||
      t1 - t0 > c.chunk || t0 % c.chunk != 0 || t0 / c.chunk >= c.max_chunks)
    return;
  const int chunk_idx = t0 / c.chunk;
  const int seq0 = c.members[mb];
  if (seq0 < 0 || seq0 >= p.num_seqs) return;

  // Block ids of the chunk (from the first member's table): -1 outside the
  // pool.  Blocks only partly inside [t0, t1) count as outside: a chunk
  // ends on a block boundary (the plan's prefixes are whole blocks).
  const int lb0 = t0 / BS;
  const int nlb = t1 / BS - lb0;
  {
    const int32_t* row = p.block_tables + (int64_t)seq0 * p.max_blocks_per_seq;
    for (int i = tid; i < nlb; i += NT) {
      const int b = row[lb0 + i];
      s_blk[i] = (int64_t)(uint32_t)b < p.num_blocks ? b : -1;
    }
  }
  // The lane's query rows: set s, row (wave * NS + s) * 16 + col = (member
  // r / group, head kvh * group + r % group).
  int seqs[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int r = (wave * NS + s) * 16 + col;
    const int m = r / p.group;
    const int sq = m < mc ? c.members[mb + m] : -1;
    seqs[s] = (sq >= 0 && sq < p.num_seqs) ? sq : -1;
  }
  __syncthreads();  // s_blk

  const CS* kbase = static_cast<const CS*>(p.k_cache) + (int64_t)kvh * p.k_head_stride;
  const CS* vbase = static_cast<const CS*>(p.v_cache) + (int64_t)kvh * p.v_head_stride;
  const int ntiles = (t1 - t0 + kTile - 1) / kTile;
  const int nstages = (ntiles + ST - 1) / ST;
  auto buffer = [&](auto k) __attribute__((always_inline)) -> uint4 (*)[PT::kUnits] {
    if constexpr (decltype(k)::value == 0) return s_buf0;
    else if constexpr (decltype(k)::value == 1) return s_buf1;
    else if constexpr (decltype(k)::value == 2) return s_buf2;
    else return s_buf3;
  };
  // Wavefront w stages part w % 2 (K, V) of tile w / 2 of a stage.
  const int my_tile = wave >> 1, my_part = wave & 1;
  auto stage = [&](auto k, int st) __attribute__((always_inline)) {
    const int tt0 = t0 + (st * ST + my_tile) * kTile;
    auto blk_of = [&](int tok) __attribute__((always_inline)) {
      const int lb = tok / BS - lb0;
      return (tok < t1 && lb < nlb) ? __builtin_amdgcn_readfirstlane(s_blk[lb]) : -1;
    };
    const int b0 = blk_of(tt0);
    const int b1 = BS >= kTile ? b0 : blk_of(tt0 + 8);
    uint4* dst = buffer(k)[my_tile];
    if (my_part == 0) {
      const uint32_t live = stage_part<CT, D, BS, 0>(dst, kbase, p.k_block_stride, b0, b1, tt0, lane);
      if (lane == 0) s_live[decltype(k)::value][my_tile] = live;
    } else {
      stage_part<CT, D, BS, 1>(dst, vbase, p.v_block_stride, b0, b1, tt0, lane);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  constexpr int NB = kPrefixBuffers;
  static_assert(NB == 3 || NB == 4, "three or four stage buffers");
  stage(I0{}, 0);
  if (1 < nstages) stage(I1{}, 1);
  if constexpr (NB == 4 && !PT::kF8)  // FP8 stages through two code buffers
    if (2 < nstages) stage(I2{}, 2);

  // Scores are scale * q.k in the log2 domain.  A negative scale is folded
  // into the query's sign bits (exact), so the softmax sees scale >= 0 and
  // the largest raw score is the largest scaled one.
  const float cs = fabsf(p.scale_log2);
  const uint32_t qsign = p.scale_log2 < 0.f ? 0x80008000u : 0u;
  uint4 qa[NS][KSTEPS];
  uint4 qdummy[1];
  int lim[NS], ctxs[NS];
  int64_t slot[NS];
  float slope[NS];
  bool on[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int r = (wave * NS + s) * 16 + col;
    const int head = kvh * p.group + (r % p.group);
    const int seq = seqs[s];
    const uint32_t ctx = (uint32_t)p.context_lens[seq < 0 ? 0 : seq];
    const bool live = seq >= 0 && ctx != 0 && ctx <= (uint32_t)p.max_seq_len;
    on[s] = live;
    ctxs[s] = live ? (int)ctx : 0;
    lim[s] = live ? min((int)ctx, t1) : t0;
    slot[s] = live ? (((int64_t)seq * p.num_heads + head) * c.max_chunks + chunk_idx) : 0;
    load_query_lane<QT, MT, D, false>(p, seq, head, seq >= 0, g, qa[s], qdummy);
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j)
      qa[s][j] = make_uint4(qa[s][j].x ^ qsign, qa[s][j].y ^ qsign, qa[s][j].z ^ qsign, qa[s][j].w ^ qsign);
    slope[s] = p.alibi != nullptr ? p.alibi[head] * kLog2e : 0.f;
  }
  // The plain softmax step (no ALiBi, scale > 0): max over raw scores,
  // weights exp2(fma(s, scale, -m)); otherwise scaled scores first.
  const bool plain = p.alibi == nullptr && cs > 0.f;

  WaveAcc<D> acc[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) acc[s].init();

  // The softmax step and PV product of one tile pair, given its scores (sa:
  // tile A, sb: tile B, per query set) and its PV operands.  Per set: the
  // softmax step, then its PV product, so that set s+1's softmax runs while
  // set s's PV MFMAs execute.
  auto softmax_pv = [&](const f32x4 (&sa)[NS], const f32x4 (&sb)[NS], const uint4 (&v)[DT], uint32_t live_a,
                        uint32_t live_b, int tok_a) __attribute__((always_inline)) {
    const int va = tok_a + 4 * g, vb = va + kTile;
    // Token liveness of the lane's 4 + 4 tokens; the context bound per set.
    const uint32_t la = (live_a >> (4 * g)) & 15u, lb = (live_b >> (4 * g)) & 15u;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      float sc[8];
      const bool whole = la == 15u && lb == 15u && vb + 3 < lim[s];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float xa = sa[s][r], xb = sb[s][r];
        if (!plain) {
          xa *= cs;
          xb *= cs;
          if (p.alibi != nullptr) {
            xa += slope[s] * (float)(va + r - ctxs[s] + 1);
            xb += slope[s] * (float)(vb + r - ctxs[s] + 1);
          }
        }
        sc[r] = xa;
        sc[4 + r] = xb;
      }
      if (!__all(whole)) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[r] = (((la >> r) & 1u) && va + r < lim[s]) ? sc[r] : -INFINITY;
          sc[4 + r] = (((lb >> r) & 1u) && vb + r < lim[s]) ? sc[4 + r] : -INFINITY;
        }
      }
      // The lane's maximum in log2 units (scaling by cs >= 0 commutes with
      // the maximum exactly).  Over FP8 caches the column's is taken only
      // when some lane passes the slack, off the path from the scores to the
      // weights (radix-shared FP8 cascade 49.0 -> 48.2 us); over 16-bit
      // caches in every pair, where the deferred form measured 0.6 us slower
      // (67.5 against 68.1 us).  Either way reduce_max() at the end gives
      // the column's maximum.
      float ml =
          fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])), fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
      if constexpr (!PT::kF8) ml = column_max(ml);
      ml *= plain ? cs : 1.f;
      WaveAcc<D>& a = acc[s];
      a.m_max = fmaxf(a.m_max, ml);
      if (__any(ml > a.m_run + kRescaleSlack)) {
        const float m_new = fmaxf(a.m_run, PT::kF8 ? column_max(ml) : ml);
        const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(a.m_run - m_new);
        a.l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) a.o[dt] *= alpha;
        a.m_run = m_new;
      }
      const float m_use = a.m_run == -INFINITY ? 0.f : a.m_run;
      const float cm = plain ? cs : 1.f;
      float pr[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) pr[r] = fast_exp2(__builtin_fmaf(sc[r], cm, -m_use));
      a.l_run += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
      const uint4 pp = make_uint4(pack_p<MT>(pr[0], pr[1]), pack_p<MT>(pr[2], pr[3]), pack_p<MT>(pr[4], pr[5]),
                                  pack_p<MT>(pr[6], pr[7]));
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) a.o[dt] = Mma<MT>::k32(v[dt], pp, a.o[dt]);
    }
  };
  auto scores_of = [&](const uint4 (&ka)[KSTEPS], const uint4 (&kb)[KSTEPS], f32x4 (&sa)[NS], f32x4 (&sb)[NS])
                       __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < NS; ++s) sa[s] = sb[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int j = 0; j < KSTEPS; ++j) {
        sa[s] = Mma<MT>::k32(ka[j], qa[s][j], sa[s]);
        sb[s] = Mma<MT>::k32(kb[j], qa[s][j], sb[s]);
      }
  };
  // One tile pair as one step (the FP8 path): scores of both tiles per query
  // set (all sets first, so that set 0's softmax runs while set 1's score
  // MFMAs execute), then softmax_pv.  img: the pair is a 16-bit image of an
  // FP8 stage (MT's layout) rather than the stage as loaded.  Measured on the
  // radix-shared B256 workload (16-bit caches, one pair per step): 70.1 ->
  // 68.4 us per launch against running each phase for both sets before the
  // next; scores one stage ahead (below) then 68.3 -> 67.6 us.
  auto consume_pair = [&](auto img, const uint4* ta, const uint4* tb, uint32_t live_a, uint32_t live_b,
                          int tok_a) __attribute__((always_inline)) {
    using OT = std::conditional_t<decltype(img)::value, MT, CT>;
    PrefixOperands<OT, MT, D> op;
    read_pair<OT, MT, D>(op, ta, tb, lane, g, col);
    f32x4 sa[NS], sb[NS];
    scores_of(op.ka, op.kb, sa, sb);
    softmax_pv(sa, sb, op.v, live_a, live_b, tok_a);
  };
  // Direct-to-LDS loads a wavefront issues per stage; s_waitcnt immediates
  // (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt in 6:4 left at its
  // maximum, lgkmcnt 0) that leave 0 or 1 later stage's loads in flight.
  constexpr int LPS = PT::kKUnits / 64 * (BS >= kTile ? 1 : 2);
  static_assert(LPS < 64, "vmcnt counts at most 63 loads");
  constexpr int kWait0 = (7 << 4);
  constexpr int kWait1 = (LPS & 15) | ((LPS >> 4) << 14) | (7 << 4);
  // The workgroup meets at a bare s_barrier (a __syncthreads, or any
  // workgroup fence that covers LDS, waits for every outstanding
  // direct-to-LDS load, the stages in flight included).  Each wavefront
  // first waits explicitly for its own loads of the next stage and its LDS
  // writes (the kWait* immediates); the asm's memory clobber keeps the
  // compiler from moving memory accesses across the barrier.
  auto barrier = [] __attribute__((always_inline)) { asm volatile("s_barrier" ::: "memory"); };
  // lgkmcnt(0) alone: this wavefront's LDS writes done, its loads in flight
  // left so.
  constexpr int kWaitLds = 15 | (7 << 4) | (3 << 14);
  __builtin_amdgcn_s_waitcnt(kWait0);  // the first stages, and the queries
  barrier();
  if constexpr (PT::kF8) {
    // Two code buffers and two images: step st consumes image st % 2, issues
    // stage st + 2 into code buffer st % 2 (its codes became image st % 2 a
    // step earlier), waits for stage st + 1, and the workgroup converts it
    // into the other image.  Each image carries its stage's live-token masks
    // (s_ilive), since the next stage issued into a code buffer rewrites
    // that buffer's masks before the image is consumed.
    auto img = [&](auto k) __attribute__((always_inline)) -> uint4 (*)[PrefixTile<MT, D>::kUnits] {
      if constexpr (decltype(k)::value == 0) return s_img0;
      else return s_img1;
    };
    auto convert = [&](auto k) __attribute__((always_inline)) {
      convert_stage<MT, D, NT>(buffer(k), img(k), tid);
      if (tid < ST) s_ilive[decltype(k)::value][tid] = s_live[decltype(k)::value][tid];
      __builtin_amdgcn_s_waitcnt(kWaitLds);
      barrier();
    };
    convert(I0{});
    auto fstep = [&](auto k, int st) __attribute__((always_inline)) {
      constexpr int K = decltype(k)::value;
      using KN = std::integral_constant<int, K ^ 1>;
      if (st + 2 < nstages) stage(k, st + 2);
      consume_pair(std::true_type{}, img(k)[0], img(k)[1], s_ilive[K][0], s_ilive[K][1], t0 + st * ST * kTile);
      if (st + 2 < nstages)
        __builtin_amdgcn_s_waitcnt(kWait1);
      else
        __builtin_amdgcn_s_waitcnt(kWait0);
      barrier();
      if (st + 1 < nstages) convert(KN{});
    };
    for (int st = 0; st < nstages; st += 2) {
      fstep(I0{}, st);
      if (st + 1 >= nstages) break;
      fstep(I1{}, st + 1);
    }
  } else {

  // Scores one stage ahead.  Step st (buffer k) issues stage st + 3 into
  // the buffer stage st - 1 used, reads stage st's V and stage st + 1's K,
  // issues stage st + 1's score MFMAs and then runs stage st's softmax and
  // PV product on the scores the previous step computed: the score MFMAs
  // of one pair execute under the softmax VALU work of the one before.  It
  // then waits for stage st + 2 (whose K the next step reads; stage st + 3
  // may stay in flight) and meets the workgroup at a barrier.  The last
  // step's look-ahead reads a buffer it never uses.
  static_assert(NB == 4, "scores one stage ahead need four stage buffers");
  auto read_k = [&](auto k, uint4 (&ka)[KSTEPS], uint4 (&kb)[KSTEPS]) __attribute__((always_inline)) {
    const uint4* ta = buffer(k)[0];
    const uint4* tb = buffer(k)[1];
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) {
      ka[j] = ta[64 * j + lane];
      kb[j] = tb[64 * j + lane];
    }
  };
  auto read_v = [&](auto k, uint4 (&v)[DT]) __attribute__((always_inline)) {
    const char* va = reinterpret_cast<const char*>(buffer(k)[0] + PT::kKUnits);
    const char* vb = reinterpret_cast<const char*>(buffer(k)[1] + PT::kKUnits);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int o = (16 * dt + col) * 32 + 8 * g;
      const uint2 x = *reinterpret_cast<const uint2*>(va + o), y = *reinterpret_cast<const uint2*>(vb + o);
      v[dt] = make_uint4(x.x, x.y, y.x, y.y);
    }
  };
  f32x4 sa[NS], sb[NS];
  {
    uint4 ka[KSTEPS], kb[KSTEPS];
    read_k(I0{}, ka, kb);
    scores_of(ka, kb, sa, sb);
  }
  auto step = [&](auto k, int st) __attribute__((always_inline)) {
    constexpr int K = decltype(k)::value;
    if (st + 3 < nstages) stage(std::integral_constant<int, (K + 3) % NB>{}, st + 3);
    uint4 v[DT];
    read_v(k, v);
    f32x4 na[NS], nb[NS];
    {
      uint4 ka[KSTEPS], kb[KSTEPS];
      read_k(std::integral_constant<int, (K + 1) % NB>{}, ka, kb);
      scores_of(ka, kb, na, nb);
    }
    softmax_pv(sa, sb, v, s_live[K][0], s_live[K][1], t0 + st * ST * kTile);
#pragma unroll
    for (int s2 = 0; s2 < NS; ++s2) {
      sa[s2] = na[s2];
      sb[s2] = nb[s2];
    }
    if (st + 3 < nstages)
      __builtin_amdgcn_s_waitcnt(kWait1);
    else
      __builtin_amdgcn_s_waitcnt(kWait0);
    barrier();
  };
  for (int st = 0; st < nstages; st += NB) {
    step(I0{}, st);
    if (st + 1 >= nstages) break;
    step(I1{}, st + 1);
    if (st + 2 >= nstages) break;
    step(I2{}, st + 2);
    if (st + 3 >= nstages) break;
    step(I3{}, st + 3);
  }
  }

  // Partial states: each row's true maximum, its weight sum against it and
  // the unnormalised output.
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    WaveAcc<D>& a = acc[s];
    a.reduce_max();
    if (a.m_max != -INFINITY && a.m_max != a.m_run) {
      const float f = exp2f(a.m_run - a.m_max);
      a.l_run *= f;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) a.o[dt] *= f;
      a.m_run = a.m_max;
    }
    const float l_col = column_sum(a.l_run);
    if (!on[s]) continue;
    float* wo = c.ws_o + slot[s] * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<float4*>(wo + 16 * dt + 4 * g) = make_float4(a.o[dt][0], a.o[dt][1], a.o[dt][2], a.o[dt][3]);
    if (g == 0) *reinterpret_cast<float2*>(c.ws_ml + slot[s] * 2) = make_float2(a.m_max, l_col);
  }
}

// Tail role: tail wavefront `tw` of `tws` takes items tw, tw + tws, ... of
// (tail partition, KV head unit), partitions longest first.
template <class QT, class CT, int D, int BS>
__device__ __forceinline__ void tail_role(const DecodeParams& p, const CascadeParams& c, int tw, int tws) {
  using QS = typename Elem<QT>::storage;
  using CS = typename Elem<CT>::storage;
  using MT = typename MmaOf<QT, CT>::type;
  constexpr int KSTEPS = Tile<D>::KSTEPS;
  constexpr int DT = Tile<D>::DT;
  constexpr int MAXT = kMaxTailPart / kTile;
  using Blocks = WaveBlocks<BS, MAXT>;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, col = lane & 15;
  const int total = c.num_parts * p.units;
  for (int rank = tw; rank < total; rank += tws) {
    const int pi = rank / p.units;
    const int unit = rank - pi * p.units;
    const int2 part = c.parts[pi];
    const int seq = part.x, k = part.y;
    if (seq < 0 || seq >= p.num_seqs) continue;  // malformed entry: nothing is written
    int kvh, h0, nh;
    unit_heads(p, unit, kvh, h0, nh);
    const uint32_t ctx = (uint32_t)p.context_lens[seq];
    const bool live = ctx != 0 && ctx <= (uint32_t)p.max_seq_len;
    const int pre = usable_prefix<BS>(c, seq, live);
    const int tstart = live ? min(pre, (int)ctx) : 0;
    const int np = tail_parts(c, live ? (int)ctx - tstart : 0);
    if (k < 0 || k >= np || k >= c.max_parts) continue;
    const int t0 = tstart + k * c.part_tokens;
    const int t1 = live ? min((int)ctx, t0 + c.part_tokens) : t0;
    const bool direct = pre == 0 && np == 1;  // the row is this partition's

    Blocks blk;
    const int lb0 = t0 / BS;
    blk.load(p.block_tables + (int64_t)seq * p.max_blocks_per_seq, p.num_blocks,
             t1 > t0 ? (t1 + BS - 1) / BS - lb0 : 0, lb0, t0, 0, 1, lane);
    uint4 qa[KSTEPS];
    uint4 qb[1];
    load_query<QT, MT, D, WideFp8<CT, D>::value>(p, seq, h0, nh, g, col, qa, qb);
    const float slope = (p.alibi != nullptr && col < nh) ? p.alibi[h0 + col] * kLog2e : 0.f;

    WaveAcc<D> acc;
    acc.init();
    if (t1 > t0) {
      const CS* kbase = static_cast<const CS*>(p.k_cache) + (int64_t)kvh * p.k_head_stride;
      const CS* vbase = static_cast<const CS*>(p.v_cache) + (int64_t)kvh * p.v_head_stride;
      stream_tiles<QT, CT, D, BS, 1, MAXT, kTailBuffers>(p, kbase, vbase, blk, t0, t1, ctx, 0, g, col, qa, qb, slope,
                                                         acc);
    }
    acc.reduce_max();
    if (acc.m_max != -INFINITY && acc.m_max != acc.m_run) {
      const float f = exp2f(acc.m_run - acc.m_max);
      acc.l_run *= f;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc.o[dt] *= f;
    }
    const float L = column_sum(acc.l_run);
    const int64_t row = (int64_t)seq * p.num_heads + h0 + col;
    if (direct) {
      if (col >= nh) continue;
      const float inv = live ? p.v_scale / (L + 1e-6f) : 0.f;
      QS* out = static_cast<QS*>(p.out) + row * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        store4<QT>(out + 16 * dt + 4 * g, acc.o[dt][0] * inv, acc.o[dt][1] * inv, acc.o[dt][2] * inv,
                   acc.o[dt][3] * inv);
      continue;
    }
    // This partition's state, for the merge kernel.
    if (col >= nh) continue;
    const int64_t slot = row * c.max_parts + k;
    float* wo = c.ws_tail_o + slot * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<float4*>(wo + 16 * dt + 4 * g) =
          make_float4(acc.o[dt][0], acc.o[dt][1], acc.o[dt][2], acc.o[dt][3]);
    if (g == 0) *reinterpret_cast<float2*>(c.ws_tail_ml + slot * 2) = make_float2(acc.m_max, L);
  }
}

// Prefix and tail roles in one launch (see the file comment).
template <class QT, class CT, int D, int BS>
__global__ __launch_bounds__(64 * kCascadeWaves, 2) void paged_cascade_kernel(DecodeParams p, CascadeParams c) {
  using PT = PrefixTile<CT, D>;
  static_assert(D % 64 == 0, "head sizes 64 and 128");
  static_assert(!std::is_same<QT, F32>::value, "the cascade takes a 16-bit query");
  using IT = PrefixTile<typename MmaOf<QT, CT>::type, D>;
  // Stage buffers: three (or four) of the stages as loaded for 16-bit
  // caches; for FP8 two of codes plus two 16-bit images.
  __shared__ uint4 s_buf0[kPrefixStageTiles][PT::kUnits];
  __shared__ uint4 s_buf1[kPrefixStageTiles][PT::kUnits];
  uint4 (*s_buf2p)[PT::kUnits] = s_buf1;
  uint4 (*s_buf3p)[PT::kUnits] = s_buf1;  // unused unless four buffers
  uint4 (*s_img0p)[IT::kUnits] = nullptr;
  uint4 (*s_img1p)[IT::kUnits] = nullptr;
  if constexpr (PT::kF8) {
    __shared__ uint4 s_img0[kPrefixStageTiles][IT::kUnits];
    __shared__ uint4 s_img1[kPrefixStageTiles][IT::kUnits];
    s_img0p = s_img0;
    s_img1p = s_img1;
  } else {
    __shared__ uint4 s_buf2[kPrefixStageTiles][PT::kUnits];
    s_buf2p = s_buf2;
    if constexpr (kPrefixBuffers == 4) {
      __shared__ uint4 s_buf3[kPrefixStageTiles][PT::kUnits];
      s_buf3p = s_buf3;
    }
  }
  __shared__ uint32_t s_ilive[2][kPrefixStageTiles];
  __shared__ int32_t s_blk[kPrefixMaxBlocks];
  __shared__ uint32_t s_live[kPrefixBuffers][kPrefixStageTiles];
  const int prefix_wgs = c.num_tiles * p.num_kv_heads;
  if ((int)blockIdx.x < prefix_wgs) {
    // The prefix role is compute-bound and sets the launch's length; its
    // wavefronts take issue priority over the memory-bound tail wavefronts
    // sharing their SIMDs.
    __builtin_amdgcn_s_setprio(3);
    prefix_role<QT, CT, D, BS>(p, c, (int)blockIdx.x / p.num_kv_heads, (int)blockIdx.x % p.num_kv_heads, s_buf0,
                               s_buf1, s_buf2p, s_buf3p, s_img0p, s_img1p, s_blk, s_live, s_ilive);
  } else {
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int tail_wgs = (int)gridDim.x - prefix_wgs;
    tail_role<QT, CT, D, BS>(p, c, ((int)blockIdx.x - prefix_wgs) * kCascadeWaves + wave, tail_wgs * kCascadeWaves);
  }
}

// Four rows per wavefront (lane 16 rs + e: chunks of row rs), kMergeRowWaves
// wavefronts per workgroup (with a quarter of the head dimension per lane,
// two measured 0.8 us faster on the FP8 radix-shared workload than one, and
// the same over 16-bit caches; four were slower).
constexpr int kMergeRowWaves = 2;
constexpr int kMergeRowsPerWave = 64 / kMergeLanesPerRow;
template <class QT, int D, int BS>
__global__ __launch_bounds__(64 * kMergeRowWaves) void paged_cascade_merge_kernel(DecodeParams p, CascadeParams c) {
  using QS = typename Elem<QT>::storage;
  constexpr int NC = MergeAcc<D>::NC;
  // States whose loads are in flight together after the early ones.
  constexpr int kMoreStates = 4;
  const int lane = threadIdx.x & 63;
  // Lane e of a row reads 16 bytes at 16 (e + 16 k) of each state's output:
  // one load instruction covers 256 contiguous bytes of each of its rows.
  // Sixteen lanes per row (122 VGPRs, four wavefronts per SIMD) against a
  // quarter of the head dimension per lane (256 VGPRs plus AGPR copies, one
  // wavefront per SIMD, and half the wavefronts): radix-shared FP8 cascade
  // 47.4 -> 46.7 us, bf16 67.7 -> 67.5 us (eight lanes per row: 46.8 and
  // 67.7 us), same process.  Each lane folds with the same operations in
  // the same order as the quarter-per-lane form did (whose weight sums were
  // summed over four lanes, three of them zero).
  const int e = lane % kMergeLanesPerRow, rs = lane / kMergeLanesPerRow;
  // Rows go in KV-head-major order (KV head, sequence, head of the group).
  // Workgroups are dealt to the 8 XCDs round-robin by index, and the prefix
  // role's workgroup for (tile, KV head h) has index = h mod 8 when there
  // are 8 KV heads, so XCD h wrote KV head h's prefix states.  With 8 KV
  // heads and a grid that is a multiple of 8, workgroup b takes row block
  // (b mod 8) * grid/8 + b/8, so that XCD h merges KV head h's rows.
  // Measured in one process against the plain order: radix-shared FP8
  // cascade 48.2 -> 47.4 us, bf16 68.3 -> 68.0 us per launch.  The merge
  // kernel's L2 hit rate stays at 29% (per-XCD counters), so the gain is not
  // its own L2 hits; where it comes from is not established.  (Dealing the
  // tail workgroups the same way measured 0.8 us slower on bf16.)  Any other
  // shape keeps the plain order; both are bijections onto the rows, and each
  // row's fold order is the same.
  const int nblk = (int)gridDim.x, b = (int)blockIdx.x;
  const int lb = (p.num_kv_heads == 8 && nblk % 8 == 0) ? (b % 8) * (nblk / 8) + b / 8 : b;
  const int64_t r = ((int64_t)lb * kMergeRowWaves + (threadIdx.x >> 6)) * kMergeRowsPerWave + rs;
  bool on = r < (int64_t)p.num_seqs * p.num_heads;
  const int64_t per_kvh = (int64_t)p.num_seqs * p.group;  // rows per KV head
  const int64_t rr = on ? r : 0;
  const int kvh_of = (int)(rr / per_kvh);
  const int64_t in_kvh = rr - kvh_of * per_kvh;  // seq * group + head of the group
  const int seq = (int)(in_kvh / p.group);
  const int64_t row = (int64_t)seq * p.num_heads + (int64_t)kvh_of * p.group + (in_kvh - (int64_t)seq * p.group);
  // The row's first tail-partition state and its first kEarly prefix-chunk
  // states are loaded together with its context and prefix lengths, in one
  // round trip: those slots exist for every row (chunk slots past the
  // workspace's max_chunks are replaced by slot 0 and never used), and each
  // is folded below only if the row has it (a slot this call did not write
  // may hold inf or NaN).  The fold order is unchanged: tail partitions,
  // then chunks.  (A 2048-token prefix in 512-token chunks, as the plan
  // picks to fill the CUs, gives a row 4 chunk states and 1 tail state.)
  constexpr int kEarly = 4;
  const uint32_t ctx = (uint32_t)p.context_lens[seq];
  const int plan_len = c.prefix_lens[seq];
  float2 ml_e[1 + kEarly];
  float4 o_e[1 + kEarly][NC];
  {
    load_state<D>(c.ws_tail_ml, c.ws_tail_o, row * c.max_parts, e, ml_e[0], o_e[0]);
#pragma unroll
    for (int j = 1; j <= kEarly; ++j)
      load_state<D>(c.ws_ml, c.ws_o, row * c.max_chunks + (j - 1 < c.max_chunks ? j - 1 : 0), e, ml_e[j], o_e[j]);
    // No load may move past this asm (it may write memory), so all of them
    // are issued before the branches on the lengths; without it the
    // compiler moves the state loads into those branches.  It uses no
    // value, so nothing waits here.
    asm volatile("" ::: "memory");
  }
  const bool live = ctx != 0 && ctx <= (uint32_t)p.max_seq_len;
  const int pre = usable_prefix_of<BS>(c, plan_len, live);
  const int np = tail_parts(c, live ? (int)ctx - min(pre, (int)ctx) : 0);
  on = on && !(pre == 0 && np == 1);  // rows the tail role wrote
  const int nt = min(np, c.max_parts);  // >= 1
  const int nch = pre > 0 ? (pre + c.chunk - 1) / c.chunk : 0;  // <= max_chunks
  MergeAcc<D> acc;
  acc.m = -INFINITY;
  acc.l = 0.f;
#pragma unroll
  for (int k = 0; k < NC; ++k) acc.o[k] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (on) fold_partial<D>(acc, ml_e[0].x, ml_e[0].y, o_e[0]);
  fold_states<D, kMoreStates>(acc, c, row * c.max_parts + 1, nt - 1, 0, on ? nt - 1 : 0, e);
#pragma unroll
  for (int j = 1; j <= kEarly; ++j)
    if (on && j - 1 < nch) fold_partial<D>(acc, ml_e[j].x, ml_e[j].y, o_e[j]);
  fold_states<D, kMoreStates>(acc, c, 0, 0, row * c.max_chunks + kEarly, on ? nch - kEarly : 0, e);
  if (!on) return;
  const float inv = p.v_scale / (acc.l + 1e-6f);
  QS* out = static_cast<QS*>(p.out) + row * D;
#pragma unroll
  for (int k = 0; k < NC; ++k)
    store4<QT>(out + 4 * (e + kMergeLanesPerRow * k), acc.o[k].x * inv, acc.o[k].y * inv, acc.o[k].z * inv, acc.o[k].w * inv);
}

template <class QT, class CT, int D, int BS>
static hipError_t launch_cascade_bs(const DecodeParams& p, const CascadeParams& c, hipStream_t stream) {
  const int64_t prefix_wgs = (int64_t)c.num_tiles * p.num_kv_heads;
  // One tail wavefront per (partition, unit) item; the hardware deals the
  // tail workgroups to CUs as slots free up, longest partitions first.
  const int64_t tail_wgs = ((int64_t)c.num_parts * p.units + kCascadeWaves - 1) / kCascadeWaves;
  hipLaunchKernelGGL((paged_cascade_kernel<QT, CT, D, BS>), dim3((unsigned)(prefix_wgs + tail_wgs)),
                     dim3(64 * kCascadeWaves), 0, stream, p, c);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t rows = (int64_t)p.num_seqs * p.num_heads;
  constexpr int kRowsPerGroup = kMergeRowsPerWave * kMergeRowWaves;
  hipLaunchKernelGGL((paged_cascade_merge_kernel<QT, D, BS>), dim3((unsigned)((rows + kRowsPerGroup - 1) / kRowsPerGroup)),
                     dim3(64 * kMergeRowWaves), 0, stream,
                     p, c);
  return hipGetLastError();
}

template <class QT, class CT, int D>
static hipError_t launch_cascade_d(const DecodeParams& p, const CascadeParams& c, int block_size, hipStream_t stream,
                                   bool* ok) {
  switch (block_size) {
    case 8:
      // FP8 V tiles of 8-token blocks are 8 bytes per dimension, below the
      // 16-byte direct-to-LDS unit: the one-pass decode takes them.
      if constexpr (std::is_same<CT, FP8>::value) break;
      else return launch_cascade_bs<QT, CT, D, 8>(p, c, stream);
    case 16: return launch_cascade_bs<QT, CT, D, 16>(p, c, stream);
    case 32: return launch_cascade_bs<QT, CT, D, 32>(p, c, stream);
  }
  *ok = false;
  return hipErrorInvalidValue;
}

template <class QT, class CT>
hipError_t launch_cascade_typed(const DecodeParams& p, const CascadeParams& c, int head_size, int block_size,
                                hipStream_t stream, bool* ok) {
  // Query sets of 16 columns: the GQA group of a KV head fits one set.
  if (p.slices != 1 || p.rows) {
    *ok = false;
    return hipErrorInvalidValue;
  }
  switch (head_size) {
    case 64: return launch_cascade_d<QT, CT, 64>(p, c, block_size, stream, ok);
    case 128: return launch_cascade_d<QT, CT, 128>(p, c, block_size, stream, ok);
  }
  *ok = false;
  return hipErrorInvalidValue;
}

}  // namespace pkv
