// Parameter blocks and launcher declarations shared by the kernels and the
// C-ABI entry points (pkv_abi.hip).  Kernels receive these structs by value
// as kernel arguments.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

namespace pkv {

enum { kF32 = 0, kF16 = 1, kBF16 = 2, kFP8 = 3 };

// Largest partition (tokens) of the partition kernel, for the internal v1
// choice and for paged_attention_v2 callers alike; the tile height of the
// decode kernels; the most partitions one sequence may be split into.
constexpr int kMaxPartition = 4096;
constexpr int kTile = 16;
constexpr int kMaxParts = 65536;
// Limits of the persistent decode kernel: longest context (its block ids sit
// in LDS) and the most sequences it orders longest-first.
constexpr int kPersistMaxSeq = 16384;
constexpr int kPersistMaxOrder = 1024;
// Token-row caches keep each wavefront's row ids of an item in its own LDS
// region (512 ids, 2 KiB), so their persistent path stops at 4096 tokens
// with eight wavefronts per workgroup (head sizes up to 128) and at 2048
// with four.
constexpr int persist_rows_max_seq(int head_size) { return head_size > 128 ? 2048 : 4096; }

struct RacParams {
  const void* key;
  const void* value;
  void* key_cache;
  void* value_cache;
  const int32_t* slot_mapping;
  int64_t num_tokens;
  int64_t key_stride;
  int64_t value_stride;
  int64_t num_slots;
  int32_t num_heads;
  int32_t head_size;
  int32_t block_size;
  int32_t layout;  // 0 = paged 5-D, 1 = token-major
  int32_t kv_dtype;
  int32_t cache_dtype;
  // FP8 caches store encode(x / scale); a power-of-two scale multiplies by
  // its exact reciprocal instead (the same result, without a division).
  float k_scale, v_scale;
  float k_inv, v_inv;
  int32_t scales_pow2;
  // Set by launch_reshape_and_cache: the call writes at least
  // kRacStreamKBytes of K, so the paged layout's per-token K stores are
  // nontemporal (reshape_and_cache.hip).
  int32_t stream_k;
};

constexpr int64_t kRacStreamKBytes = int64_t(4) << 20;

hipError_t launch_reshape_and_cache(const RacParams& p, bool aligned, hipStream_t stream);

// Element-wise conversion with a scale between the element types kF32,
// kF16, kBF16 and kFP8 (E4M3 codes), convert_fp8.hip.
hipError_t launch_convert_fp8(void* dst, const void* src, int64_t n, float scale, int src_dtype, int dst_dtype,
                              hipStream_t stream);

struct DecodeParams {
  void* out;                  // [B, Hq, D], query dtype
  const void* q;              // [B, Hq, D], row stride q_stride
  const void* k_cache;        // paged 5-D K, or token rows (see rows)
  const void* v_cache;        // paged 5-D V, or token rows
  const int32_t* block_tables;
  const int32_t* context_lens;
  const float* alibi;         // [Hq] or null
  float* ws_ml;               // [B, Hq, max_parts, 2]: (max, sum) per partition, log2 domain
  float* ws_o;                // [B, Hq, max_parts, D]: normalised partition outputs
  int64_t num_blocks;
  int64_t q_stride;
  int64_t k_block_stride, k_head_stride;
  int64_t v_block_stride, v_head_stride;
  float scale_log2;           // scale * log2(e)
  int32_t num_seqs;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t group;              // num_heads / num_kv_heads
  int32_t slices;             // ceil(group / 16): 16-head slices per KV head
  int32_t units;              // num_kv_heads * slices
  int32_t max_blocks_per_seq;
  int32_t max_seq_len;
  int32_t partition;          // tokens per partition (multiple of 16 and block_size)
  int32_t max_parts;          // ceil(max_seq_len / partition)
  int32_t persistent;         // 1: the persistent kernel may be used (v1 semantics, short enough contexts)
  // Token-row layout ([blocks, block_size, Hkv, D], block_size 1 being
  // MHATokenPool's [rows, Hkv, D]): k/v_block_stride then hold the row
  // stride (elements from one token's row to the next) and block_size the
  // tokens per block; token t of a sequence sits at row
  // block_tables[t / block_size] * block_size + t % block_size.
  int32_t rows;
  int32_t block_size;
  // Token rows, persistent path: bytes of K and V reachable from any head's
  // base, (rows - 1) * row bytes + head_size * element bytes; the persistent
  // kernel addresses rows with 32-bit buffer offsets, so it is used only when
  // both fit in 32 bits.
  uint32_t k_rows_bytes, v_rows_bytes;
  // Output scale: v_scale for FP8 caches (whose k_scale is folded into
  // scale_log2), 1 otherwise.
  float v_scale;
  // Arrival counters of the partition kernel's own merge (null: the merge
  // kernel runs after it): one per (sequence, unit), zero before a launch
  // and left zero by it.
  int32_t* counters;
};

// The partition kernel merges its own partitions (the workgroup whose state
// arrives last folds them all) when a row has at most kMergeGroup of them;
// deeper rows are merged by the merge kernel, whose many workgroups fetch
// the states faster than one workgroup's dependent loads would.
constexpr int kMergeGroup = 8;
// Bytes at the start of every decode workspace that hold those counters.
constexpr int64_t kCounterBytes = 65536;

// Shared-prefix (cascade) decode plan, device arrays built on the host from
// the block tables (see include/pagedkv.h, pkv_cascade_plan):
//   prefix_lens[s]: leading tokens of sequence s that the prefix pass covers
//                   (0: none), a multiple of the block size and of 16;
//   members[i]:     sequence ids, the members of each prefix group adjacent;
//   tiles[w]:       (member_begin, member_count, token_begin, token_end) of
//                   prefix-pass work unit w: members[member_begin ..
//                   +member_count) share the blocks of the first one's table
//                   over tokens [0, token_end), and the unit covers tokens
//                   [token_begin, token_end) = chunk token_begin / chunk;
//   parts[r]:       (sequence, k) of tail partition r, longest first:
//                   partition k of a sequence covers tokens
//                   [pre + k * part_tokens, min(ctx, pre + (k + 1) *
//                   part_tokens)) after its prefix pre, and a sequence has
//                   max(1, ceil((ctx - pre) / part_tokens)) of them.
// Partial softmax states of the prefix pass, per (sequence, query head,
// chunk): (max, sum) in ws_ml and the unnormalised output in ws_o; of the
// tail pass, per (sequence, query head, partition), in ws_tail_ml /
// ws_tail_o.  A sequence with no prefix and one partition has its rows
// written by the tail pass; the merge kernel writes the others.
struct CascadeParams {
  const int32_t* prefix_lens;
  const int32_t* members;
  const int4* tiles;
  const int2* parts;
  float* ws_ml;       // [B, Hq, max_chunks, 2]
  float* ws_o;        // [B, Hq, max_chunks, D]
  float* ws_tail_ml;  // [B, Hq, max_parts, 2]
  float* ws_tail_o;   // [B, Hq, max_parts, D]
  int32_t num_members;
  int32_t num_tiles;
  int32_t num_parts;
  int32_t chunk;       // tokens per chunk: a multiple of 16 and of the block size, at most kMaxPrefixChunk
  int32_t max_chunks;  // chunk slots per (sequence, query head) in the workspace
  int32_t part_tokens; // tokens per tail partition: a multiple of 16 and of the block size, at most kMaxTailPart
  int32_t max_parts;   // partition slots per (sequence, query head) in the workspace
};
constexpr int kMaxPrefixChunk = 4096;
// Longest tail partition: each wavefront keeps its partition's block ids in
// registers.
constexpr int kMaxTailPart = 1024;
// Defined in cascade_impl.h for the (query, cache) pairs (BF16, BF16),
// (F16, F16), (BF16, FP8) and (F16, FP8); *ok is cleared for a shape the
// cascade kernels do not cover (the caller then runs the one-pass decode).
template <class QT, class CT>
hipError_t launch_cascade_typed(const DecodeParams& p, const CascadeParams& c, int head_size, int block_size,
                                hipStream_t stream, bool* ok);
struct CascadeWorkspace {
  size_t ml_bytes, o_bytes, tail_ml_bytes, tail_o_bytes, total;
};
CascadeWorkspace cascade_workspace_layout(int32_t num_seqs, int32_t num_heads, int32_t head_size,
                                          int32_t max_chunks, int32_t max_parts);

// Scratch carve-up shared by the size query and the launcher: per-partition
// (max, sum) pairs, then per-partition outputs.
struct DecodeWorkspace {
  size_t ml_bytes, o_bytes, total;
};
DecodeWorkspace decode_workspace_layout(int32_t num_seqs, int32_t num_heads, int32_t head_size,
                                        int32_t max_parts);

// Whole-block copies (copy_blocks.hip): plane i copies block src of src[i]
// to block dst of dst[i] for every pair of the device int64 mapping.
constexpr int kMaxCopyPlanes = 64;
struct BlockCopyParams {
  const int64_t* mapping;  // [num_pairs][2] = (src block, dst block)
  int64_t num_pairs;
  int64_t src_blocks;      // blocks in each source plane
  int64_t dst_blocks;      // blocks in each destination plane
  int64_t block_bytes;
  int32_t num_planes;      // at most kMaxCopyPlanes per launch
  const char* src[kMaxCopyPlanes];
  char* dst[kMaxCopyPlanes];
};
hipError_t launch_copy_blocks(const BlockCopyParams& p, bool aligned, hipStream_t stream);
// Most pairs one launch can take for this block size.
int64_t copy_blocks_max_grid_pairs(int64_t block_bytes, bool aligned);

struct F32;
struct F16;
struct BF16;
struct FP8;
// Defined in paged_decode_impl.h, instantiated once per (query, cache) type
// pair in decode_<q>_<cache>.hip.  *ok is cleared for an unsupported
// head_size / block_size.
template <class QT, class CT>
hipError_t launch_decode_typed(const DecodeParams& p, int head_size, int block_size, hipStream_t stream,
                               bool* ok);

}  // namespace pkv
