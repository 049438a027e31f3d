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

#include "pkv_device.h"
#include "pkv_launch.h"

namespace pkv {

constexpr int kWaves = 4;
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

// Two probabilities -> packed 16-bit MFMA operand word.
template <class CT> __device__ __forceinline__ uint32_t pack_p(float a, float b);
template <> __device__ __forceinline__ uint32_t pack_p<BF16>(float a, float b) {
  return pack2(f32_to_bf16_bits(a), f32_to_bf16_bits(b));
}
template <> __device__ __forceinline__ uint32_t pack_p<F16>(float a, float b) {
  return pack2(f32_to_f16_bits(a), f32_to_f16_bits(b));
}

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

// One wavefront's 16-token tile in registers.
template <int D> struct Tile {
  static constexpr int KSTEPS = (D + 31) / 32;  // 16x16x32 k-steps over the head dimension
  static constexpr int DT = (D + 15) / 16;      // 16-wide dimension tiles of the output
  uint4 k[KSTEPS];
  uint2 v[DT];
  int vpb;  // block of this lane's 4 V tokens, -1 if masked out
};

// Issues the loads of tile `tile` (tokens tt0 .. tt0+15).  Block ids that are
// masked out (past the partition's blocks or outside the pool) read block 0
// instead -- always in bounds -- and are discarded by the caller, so the
// number of loads per tile is fixed and the next tile's loads can stay in
// flight while the current one is consumed.
template <int D, int BS>
__device__ __forceinline__ void load_tile(Tile<D>& t, const uint16_t* kbase, const uint16_t* vbase,
                                          int64_t k_block_stride, int64_t v_block_stride,
                                          const int32_t* s_blk, int nlb, int lb0, int tt0, int g, int col) {
  constexpr int NCHUNK = D / 8;  // 16-byte K chunks per token
  const int ktok = tt0 + col;
  const int klb = ktok / BS - lb0;
  const int kpb = klb < nlb ? s_blk[klb] : -1;
  const uint16_t* kp = kbase + (int64_t)(kpb < 0 ? 0 : kpb) * k_block_stride + (ktok % BS) * 8;
#pragma unroll
  for (int j = 0; j < Tile<D>::KSTEPS; ++j) {
    const int c = 4 * j + g;
    if (NCHUNK % 4 == 0 || c < NCHUNK)
      t.k[j] = *reinterpret_cast<const uint4*>(kp + c * (BS * 8));
    else
      t.k[j] = make_uint4(0, 0, 0, 0);
  }
  const int vtok = tt0 + 4 * g;
  const int vlb = vtok / BS - lb0;
  const int vpb = vlb < nlb ? s_blk[vlb] : -1;
  t.vpb = vpb;
  const uint16_t* vp = vbase + (int64_t)(vpb < 0 ? 0 : vpb) * v_block_stride + (vtok % BS);
#pragma unroll
  for (int dt = 0; dt < Tile<D>::DT; ++dt) {
    const int d = 16 * dt + col;
    if (D % 16 == 0 || d < D)
      t.v[dt] = *reinterpret_cast<const uint2*>(vp + d * BS);
    else
      t.v[dt] = make_uint2(0, 0);
  }
}

template <class QT, class CT, int D, int BS>
__global__ __launch_bounds__(256) void paged_decode_part_kernel(DecodeParams p) {
  using QS = typename Elem<QT>::storage;
  constexpr int KSTEPS = Tile<D>::KSTEPS;
  constexpr int DT = Tile<D>::DT;
  constexpr bool SPLIT_Q = std::is_same<QT, F32>::value;

  __shared__ int32_t s_blk[kMaxPartition / BS];
  __shared__ float s_red[kWaves - 1][DT * 4][64];
  __shared__ float s_m[kWaves][16];
  __shared__ float s_l[kWaves][16];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, col = lane & 15;

  const int unit = blockIdx.x % p.units;
  const int rest = blockIdx.x / p.units;
  const int seq = rest % p.num_seqs;
  const int part = rest / p.num_seqs;
  const int kvh = unit / p.slices;
  const int slice = unit - kvh * p.slices;
  const int h0 = kvh * p.group + slice * 16;
  const int nh = min(16, p.group - slice * 16);

  // Context lengths are read as unsigned, as the reference does.
  const uint32_t ctx = (uint32_t)p.context_lens[seq];
  if (ctx == 0 || ctx > (uint32_t)p.max_seq_len) {
    if (part == 0) {
      QS* out = static_cast<QS*>(p.out) + ((int64_t)seq * p.num_heads + h0) * D;
      for (int i = tid; i < nh * D; i += 256) out[i] = from_f32<QT>(0.f);
    }
    return;
  }
  const int nparts = ((int)ctx + p.partition - 1) / p.partition;
  if (part >= nparts) return;
  const int t0 = part * p.partition;
  const int t1 = min(t0 + p.partition, (int)ctx);
  const int lb0 = t0 / BS;
  const int nlb = (t1 + BS - 1) / BS - lb0;

  // Block-table slice of this partition -> LDS (one coalesced read).
  {
    const int32_t* bt = p.block_tables + (int64_t)seq * p.max_blocks_per_seq + lb0;
    for (int i = tid; i < nlb; i += 256) {
      const int32_t b = bt[i];
      s_blk[i] = ((int64_t)(uint32_t)b < p.num_blocks) ? b : -1;
    }
  }

  // Query group -> B operand registers (head = col, dims 32j + 8g .. +8).
  uint4 qa[KSTEPS];
  uint4 qb[SPLIT_Q ? KSTEPS : 1];
  {
    const QS* qrow = static_cast<const QS*>(p.q) + (int64_t)seq * p.q_stride + (int64_t)(h0 + col) * D;
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) {
      const int d0 = 32 * j + 8 * g;
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
  const float slope = (p.alibi != nullptr && col < nh) ? p.alibi[h0 + col] * kLog2e : 0.f;
  __syncthreads();

  f32x4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  const uint16_t* kbase = static_cast<const uint16_t*>(p.k_cache) + (int64_t)kvh * p.k_head_stride;
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v_cache) + (int64_t)kvh * p.v_head_stride;
  const int ntiles = (t1 - t0 + kTile - 1) / kTile;

  // Consumes one loaded tile starting at token tt0.
  auto consume = [&](Tile<D>& t, int tt0) {
    const int vtok = tt0 + 4 * g;
    // Tokens at or past the end of the partition, and tokens of masked-out
    // blocks, contribute nothing: zero their V (the slots may hold anything,
    // including NaN) and their scores.
    if (t.vpb < 0) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) t.v[dt] = make_uint2(0, 0);
    } else if (tt0 + kTile > t1) {
      const uint32_t m01 = (vtok + 0 < t1 ? 0x0000ffffu : 0u) | (vtok + 1 < t1 ? 0xffff0000u : 0u);
      const uint32_t m23 = (vtok + 2 < t1 ? 0x0000ffffu : 0u) | (vtok + 3 < t1 ? 0xffff0000u : 0u);
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
      sacc = Mma<CT>::k32(t.k[j], qa[j], sacc);
      if constexpr (SPLIT_Q) sacc = Mma<CT>::k32(t.k[j], qb[j], sacc);
    }
    // ---- online softmax (log2 domain) ----
    float sc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tok = vtok + r;
      float x = sacc[r] * p.scale_log2;
      if (p.alibi != nullptr) x += slope * (float)(tok - (int)ctx + 1);
      sc[r] = (tok < t1 && t.vpb >= 0) ? x : -INFINITY;
    }
    const float mt = column_max(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
    const float m_new = fmaxf(m_run, mt);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = exp2f(sc[r] - m_use);
    l_run = l_run * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
    // ---- O^T += V^T * P^T ----
    const uint2 pp = make_uint2(pack_p<CT>(pr[0], pr[1]), pack_p<CT>(pr[2], pr[3]));
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = Mma<CT>::k16(t.v[dt], pp, o[dt]);
  };

  // Two register sets: the loads of tile i+4 are issued before tile i is
  // consumed.  Past the last tile the prefetch re-reads the current tile
  // (in bounds, served by L2) so that every iteration issues the same loads.
  if (wave < ntiles) {
    Tile<D> ta, tb;
    int tile = wave;
    load_tile<D, BS>(ta, kbase, vbase, p.k_block_stride, p.v_block_stride, s_blk, nlb, lb0, t0 + tile * kTile,
                     g, col);
    while (true) {
      int nt = tile + kWaves < ntiles ? tile + kWaves : tile;
      load_tile<D, BS>(tb, kbase, vbase, p.k_block_stride, p.v_block_stride, s_blk, nlb, lb0, t0 + nt * kTile,
                       g, col);
      consume(ta, t0 + tile * kTile);
      tile += kWaves;
      if (tile >= ntiles) break;
      nt = tile + kWaves < ntiles ? tile + kWaves : tile;
      load_tile<D, BS>(ta, kbase, vbase, p.k_block_stride, p.v_block_stride, s_blk, nlb, lb0, t0 + nt * kTile,
                       g, col);
      consume(tb, t0 + tile * kTile);
      tile += kWaves;
      if (tile >= ntiles) break;
    }
  }

  // ---- merge the four wavefronts of the workgroup ----
  const float l_col = column_sum(l_run);
  if (wave > 0) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) s_red[wave - 1][dt * 4 + r][lane] = o[dt][r];
  }
  if (g == 0) {
    s_m[wave][col] = m_run;
    s_l[wave][col] = l_col;
  }
  __syncthreads();
  if (wave != 0) return;
  float M = m_run;
#pragma unroll
  for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w][col]);
  const float mu = M == -INFINITY ? 0.f : M;
  const float a0 = exp2f(m_run - mu);
  float L = l_col * a0;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] *= a0;
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    const float aw = exp2f(s_m[w][col] - mu);
    L += s_l[w][col] * aw;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[dt][r] += aw * s_red[w - 1][dt * 4 + r][lane];
  }
  if (col >= nh) return;
  const int64_t hrow = (int64_t)seq * p.num_heads + h0 + col;
  if (nparts == 1) {
    const float inv = 1.f / (L + 1e-6f);
    QS* out = static_cast<QS*>(p.out) + hrow * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 16 * dt + 4 * g + r;
        if (D % 16 == 0 || d < D) out[d] = from_f32<QT>(o[dt][r] * inv);
      }
    return;
  }
  const int64_t slot = hrow * p.max_parts + part;
  const float invl = L > 0.f ? 1.f / L : 0.f;
  float* wo = p.ws_o + slot * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const int d = 16 * dt + 4 * g;
    if (D % 16 == 0 || d < D)
      *reinterpret_cast<float4*>(wo + d) =
          make_float4(o[dt][0] * invl, o[dt][1] * invl, o[dt][2] * invl, o[dt][3] * invl);
  }
  if (g == 0) *reinterpret_cast<float2*>(p.ws_ml + slot * 2) = make_float2(M, L);
}

// Log-sum-exp merge of the partitions of one (sequence, query head) per
// wavefront.  Rows whose sequence fits in one partition (or has an empty or
// over-long context) were finished by the partition kernel.
template <class QT, int D>
__global__ __launch_bounds__(256) void paged_decode_reduce_kernel(DecodeParams p) {
  using QS = typename Elem<QT>::storage;
  constexpr int NDL = (D + 63) / 64;  // dimensions per lane
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);  // seq * Hq + head
  if (row >= (int64_t)p.num_seqs * p.num_heads) return;
  const int seq = (int)(row / p.num_heads);
  const uint32_t ctx = (uint32_t)p.context_lens[seq];
  if (ctx == 0 || ctx > (uint32_t)p.max_seq_len) return;
  const int nparts = ((int)ctx + p.partition - 1) / p.partition;
  if (nparts == 1) return;
  const float* ml = p.ws_ml + row * p.max_parts * 2;
  const float* po = p.ws_o + row * p.max_parts * D;
  float mx = -INFINITY;
  for (int i = lane; i < nparts; i += 64) mx = fmaxf(mx, ml[2 * i]);
  mx = wave_max(mx);
  const float mu = mx == -INFINITY ? 0.f : mx;
  float acc[NDL];
#pragma unroll
  for (int i = 0; i < NDL; ++i) acc[i] = 0.f;
  float sum = 0.f;
  for (int i = 0; i < nparts; ++i) {
    const float2 e = *reinterpret_cast<const float2*>(ml + 2 * i);
    const float w = e.y * exp2f(e.x - mu);
    sum += w;
#pragma unroll
    for (int k = 0; k < NDL; ++k) {
      const int d = lane + 64 * k;
      if (D % 64 == 0 || d < D) acc[k] += w * po[(int64_t)i * D + d];
    }
  }
  const float inv = 1.f / (sum + 1e-6f);
  QS* out = static_cast<QS*>(p.out) + row * D;
#pragma unroll
  for (int k = 0; k < NDL; ++k) {
    const int d = lane + 64 * k;
    if (D % 64 == 0 || d < D) out[d] = from_f32<QT>(acc[k] * inv);
  }
}

template <class QT, class CT, int D, int BS>
static hipError_t launch_one(const DecodeParams& p, hipStream_t stream) {
  const int64_t nwg = (int64_t)p.max_parts * p.num_seqs * p.units;
  hipLaunchKernelGGL((paged_decode_part_kernel<QT, CT, D, BS>), dim3((unsigned)nwg), dim3(256), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.max_parts == 1) return e;
  const int64_t rows = (int64_t)p.num_seqs * p.num_heads;
  hipLaunchKernelGGL((paged_decode_reduce_kernel<QT, D>), dim3((unsigned)((rows + kWaves - 1) / kWaves)), dim3(256),
                     0, stream, p);
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

template <class QT, class CT>
hipError_t launch_decode_typed(const DecodeParams& p, int head_size, int block_size, hipStream_t stream,
                               bool* ok) {
  switch (head_size) {
    case 32: return launch_bs<QT, CT, 32>(p, block_size, stream, ok);
    case 64: return launch_bs<QT, CT, 64>(p, block_size, stream, ok);
    case 80: return launch_bs<QT, CT, 80>(p, block_size, stream, ok);
    case 96: return launch_bs<QT, CT, 96>(p, block_size, stream, ok);
    case 112: return launch_bs<QT, CT, 112>(p, block_size, stream, ok);
    case 120: return launch_bs<QT, CT, 120>(p, block_size, stream, ok);
    case 128: return launch_bs<QT, CT, 128>(p, block_size, stream, ok);
    case 192: return launch_bs<QT, CT, 192>(p, block_size, stream, ok);
    case 256: return launch_bs<QT, CT, 256>(p, block_size, stream, ok);
  }
  *ok = false;
  return hipErrorInvalidValue;
}

}  // namespace pkv
