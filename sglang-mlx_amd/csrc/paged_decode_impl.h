// Block-table decode attention for gfx950 (paged 5-D KV layout).
//
// Semantics: paged_attention_kernels.metal:37-168 of the reference --
// per (sequence s, query head h), softmax over the first ctx tokens of
// scale * q.k (+ alibi[h] * (t - ctx + 1)), weighted sum of V, denominator
// (sum + 1e-6), fp32 accumulation, zero output when ctx == 0 or
// ctx > max_seq_len.  GQA: kv_head = h / (Hq / Hkv).
//
// Work decomposition (one workgroup = 4 wavefronts):
//   unit      = (KV head, slice of at most 16 query heads of its GQA group)
//   workgroup = (partition, sequence, unit); the unit index varies fastest so
//               that, with 8 KV heads, every XCD sees one KV head only.
//   wavefront = every 4th 16-token tile of the partition.
// Per tile the wavefront computes S^T[16 tok x 16 heads] with
// v_mfma_f32_16x16x32_{bf16,f16}: the A operand is the K tile straight from
// HBM -- in the paged 5-D layout lane l reading the 16 bytes at
// (64*j + l) * 16 of the (block, head) region is exactly row l%16, k-group
// l/16 of step j, so each k-step is one contiguous 1 KiB load -- and the B
// operand is the query group, held in registers for the whole partition.
// The output layout of that MFMA (lane l, register r = token 4*(l/16)+r,
// head l%16) is the B-operand layout of v_mfma_f32_16x16x16, so the softmax
// probabilities feed P*V without leaving registers; V^T tiles are 8-byte
// loads of 4 consecutive tokens of one dimension (contiguous in the V layout).
// The softmax runs online in the log2 domain.
//
// Partitions of one (sequence, unit) are merged by the last workgroup to
// arrive (device-scope counter in the workspace): groups of up to 16
// partitions are merged first, then the group results, so the merge work is
// spread over many workgroups when the context is long.  Counters are reset
// by the workgroup that consumed them.
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

// Merge `cnt` partials of the unit's heads, taken from partition slots
// first, first+stride, ...  If `final`, write the attention output; else
// write a normalised partial into slot `first`.  Executed by a whole
// workgroup.
template <class QT, int D>
__device__ void merge_partials(const DecodeParams& p, int seq, int h0, int nh, int first, int stride,
                               int cnt, bool final, float (*s_w)[kMaxGroups], float* s_mu,
                               float* s_sum) {
  using QS = typename Elem<QT>::storage;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int hh = wave; hh < nh; hh += kWaves) {
    const int64_t row = ((int64_t)seq * p.num_heads + h0 + hh) * p.max_parts;
    const float m = lane < cnt ? p.ws_ml[(row + first + (int64_t)lane * stride) * 2] : -INFINITY;
    const float l = lane < cnt ? p.ws_ml[(row + first + (int64_t)lane * stride) * 2 + 1] : 0.f;
    const float mx = wave_max(m);
    const float mu = mx == -INFINITY ? 0.f : mx;
    const float w = l * exp2f(m - mu);
    if (lane < cnt) s_w[hh][lane] = w;
    const float sum = wave_sum(w);
    if (lane == 0) {
      s_mu[hh] = mx;
      s_sum[hh] = sum;
    }
  }
  __syncthreads();
  for (int i = tid; i < nh * D; i += 256) {
    const int hh = i / D, d = i - (i / D) * D;
    const int64_t row = ((int64_t)seq * p.num_heads + h0 + hh) * p.max_parts;
    float acc = 0.f;
    for (int k = 0; k < cnt; ++k) acc += s_w[hh][k] * p.ws_o[(row + first + (int64_t)k * stride) * D + d];
    if (final) {
      QS* out = static_cast<QS*>(p.out) + ((int64_t)seq * p.num_heads + h0 + hh) * D;
      out[d] = from_f32<QT>(acc / (s_sum[hh] + 1e-6f));
    } else {
      const float s = s_sum[hh];
      p.ws_o[(row + first) * D + d] = s > 0.f ? acc / s : 0.f;
    }
  }
  if (!final && tid < nh) {
    const int64_t row = ((int64_t)seq * p.num_heads + h0 + tid) * p.max_parts;
    p.ws_ml[(row + first) * 2] = s_mu[tid];
    p.ws_ml[(row + first) * 2 + 1] = s_sum[tid];
  }
}

// Arrival: returns true in every thread of the workgroup that arrived last.
__device__ __forceinline__ bool arrive_last(int32_t* counter, int expected, int* s_flag) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(counter, 1);
    *s_flag = (prev == expected - 1);
  }
  __syncthreads();
  const bool last = *s_flag;
  if (last) __threadfence();
  return last;
}

template <class QT, class CT, int D, int BS>
__global__ __launch_bounds__(256) void paged_decode_kernel(DecodeParams p) {
  using QS = typename Elem<QT>::storage;
  using CS = uint16_t;
  constexpr int KSTEPS = (D + 31) / 32;  // 16x16x32 k-steps over the head dimension
  constexpr int DT = (D + 15) / 16;      // 16-wide dimension tiles of the output
  constexpr int NCHUNK = D / 8;          // 16-byte K chunks per token
  constexpr bool SPLIT_Q = std::is_same<QT, F32>::value;

  __shared__ int32_t s_blk[kMaxPartition / BS];
  __shared__ float s_red[kWaves - 1][DT * 4][64];
  __shared__ float s_m[kWaves][16];
  __shared__ float s_l[kWaves][16];
  __shared__ float s_w[16][kMaxGroups];
  __shared__ float s_mu[16], s_sum[16];
  __shared__ int s_flag;

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

  const CS* kbase = static_cast<const CS*>(p.k_cache) + (int64_t)kvh * p.k_head_stride;
  const CS* vbase = static_cast<const CS*>(p.v_cache) + (int64_t)kvh * p.v_head_stride;
  const int ntiles = (t1 - t0 + kTile - 1) / kTile;

  for (int tile = wave; tile < ntiles; tile += kWaves) {
    const int tt0 = t0 + tile * kTile;
    // ---- K tile: row = token tt0 + col ----
    const int ktok = tt0 + col;
    const int klb = ktok / BS - lb0;
    const int kpb = klb < nlb ? s_blk[klb] : -1;
    uint4 kv[KSTEPS];
    {
      const CS* kp = kbase + (int64_t)(kpb < 0 ? 0 : kpb) * p.k_block_stride + (ktok % BS) * 8;
#pragma unroll
      for (int j = 0; j < KSTEPS; ++j) {
        const int c = 4 * j + g;
        kv[j] = make_uint4(0, 0, 0, 0);
        if (kpb >= 0 && (NCHUNK % 4 == 0 || c < NCHUNK))
          kv[j] = *reinterpret_cast<const uint4*>(kp + c * (BS * 8));
      }
    }
    // ---- V^T tile: tokens tt0 + 4g .. +3 (one block), dim 16*dt + col ----
    const int vtok = tt0 + 4 * g;
    const int vlb = vtok / BS - lb0;
    const int vpb = vlb < nlb ? s_blk[vlb] : -1;
    uint2 vv[DT];
    {
      const CS* vp = vbase + (int64_t)(vpb < 0 ? 0 : vpb) * p.v_block_stride + (vtok % BS);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d = 16 * dt + col;
        vv[dt] = make_uint2(0, 0);
        if (vpb >= 0 && (D % 16 == 0 || d < D)) vv[dt] = *reinterpret_cast<const uint2*>(vp + d * BS);
      }
    }
    // Tokens at or past the end of the partition are masked: zero their V
    // (the slots may hold anything, including NaN) and their scores.
    if (tt0 + kTile > t1) {
      const uint32_t m01 = (vtok + 0 < t1 ? 0x0000ffffu : 0u) | (vtok + 1 < t1 ? 0xffff0000u : 0u);
      const uint32_t m23 = (vtok + 2 < t1 ? 0x0000ffffu : 0u) | (vtok + 3 < t1 ? 0xffff0000u : 0u);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        vv[dt].x &= m01;
        vv[dt].y &= m23;
      }
    }
    // ---- S^T = K * Q^T ----
    f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) {
      sacc = Mma<CT>::k32(kv[j], qa[j], sacc);
      if constexpr (SPLIT_Q) sacc = Mma<CT>::k32(kv[j], qb[j], sacc);
    }
    // ---- online softmax (log2 domain) ----
    float sc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = vtok + r;
      float x = sacc[r] * p.scale_log2;
      if (p.alibi != nullptr) x += slope * (float)(t - (int)ctx + 1);
      sc[r] = (t < t1 && vpb >= 0) ? x : -INFINITY;
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
    for (int dt = 0; dt < DT; ++dt) o[dt] = Mma<CT>::k16(vv[dt], pp, o[dt]);
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
  if (wave == 0) {
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
    if (col < nh) {
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
      } else {
        const int64_t slot = hrow * p.max_parts + part;
        const float invl = L > 0.f ? 1.f / L : 0.f;
        float* wo = p.ws_o + slot * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int d = 16 * dt + 4 * g + r;
            if (D % 16 == 0 || d < D) wo[d] = o[dt][r] * invl;
          }
        if (g == 0) {
          p.ws_ml[slot * 2] = M;
          p.ws_ml[slot * 2 + 1] = L;
        }
      }
    }
  }
  if (nparts == 1) return;

  // ---- cross-partition log-sum-exp merge, last arrival does the work ----
  const int ngroups = (nparts + kGroup - 1) / kGroup;
  int32_t* counters = p.ws_count + ((int64_t)seq * p.units + unit) * (1 + kMaxGroups);
  if (ngroups == 1) {
    if (!arrive_last(&counters[0], nparts, &s_flag)) return;
    merge_partials<QT, D>(p, seq, h0, nh, 0, 1, nparts, true, s_w, s_mu, s_sum);
    if (tid == 0) counters[0] = 0;
    return;
  }
  const int grp = part / kGroup;
  const int gcnt = min(kGroup, nparts - grp * kGroup);
  if (!arrive_last(&counters[1 + grp], gcnt, &s_flag)) return;
  merge_partials<QT, D>(p, seq, h0, nh, grp * kGroup, 1, gcnt, false, s_w, s_mu, s_sum);
  if (tid == 0) counters[1 + grp] = 0;
  if (!arrive_last(&counters[0], ngroups, &s_flag)) return;
  merge_partials<QT, D>(p, seq, h0, nh, 0, kGroup, ngroups, true, s_w, s_mu, s_sum);
  if (tid == 0) counters[0] = 0;
}

template <class QT, class CT, int D, int BS>
static hipError_t launch_one(const DecodeParams& p, hipStream_t stream) {
  const int64_t nwg = (int64_t)p.max_parts * p.num_seqs * p.units;
  hipLaunchKernelGGL((paged_decode_kernel<QT, CT, D, BS>), dim3((unsigned)nwg), dim3(256), 0, stream, p);
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
