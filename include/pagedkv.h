/*
 * pagedkv.h - C ABI of the MI355X (gfx950) paged-KV hot path.
 *
 * The library (libpagedkv_gfx950.so) replaces the reference's nanobind module
 * `sglang_mlx._ext` (bindings.cpp:37-134) and the MLX host ops behind it
 * (paged_attention/mlx_paged_attention.cpp, paged_attention/mlx_cache.cpp,
 * paged_attention/mlx_device.cpp).  Every entry point takes plain device
 * pointers, sizes and strides; no framework types cross this boundary.
 *
 * Conventions shared by all entry points
 *   - Return value: PKV_OK (0) on success, otherwise a PKV_ERR_* code; the
 *     message of the last failure on the calling thread is returned by
 *     pkv_last_error().  Argument checks run before any HIP call, so a
 *     rejected call has no side effect.  A HIP error status describes this
 *     call only: an error left pending on the thread by earlier HIP calls of
 *     other code is cleared before launching, and a HIP call of the library
 *     that fails leaves no pending error behind.
 *   - Launches are asynchronous on `stream` (a hipStream_t passed as void*;
 *     NULL = the legacy default stream).  Nothing synchronises.
 *   - The library allocates no device memory.  Output buffers and the
 *     attention workspace belong to the caller.
 *   - Strides are in elements, not bytes.
 *   - Block tables, context lengths and slot mappings are 32-bit integers.
 */
#ifndef PAGEDKV_H
#define PAGEDKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  PKV_ERR_INVALID and PKV_ERR_UNSUPPORTED map to Python
 * ValueError (the reference raises std::invalid_argument for both,
 * mlx_paged_attention.cpp:156-199); PKV_ERR_HIP maps to RuntimeError. */
enum {
  PKV_OK = 0,
  PKV_ERR_INVALID = 1,
  PKV_ERR_UNSUPPORTED = 2,
  PKV_ERR_HIP = 3
};

/* Element types (reference dtypeStr, mlx_paged_attention.cpp:30-37), and
 * PKV_FP8_E4M3: one-byte E4M3 codes in the reference's format
 * (float8.metal:13-124: bias 7, exponent 15 = +-inf / NaN, so finite values
 * reach 240; not OCP E4M3FN), encoded by its algorithm bit for bit. */
enum { PKV_F32 = 0, PKV_F16 = 1, PKV_BF16 = 2, PKV_FP8_E4M3 = 3 };

/* KV cache layouts.
 *   PKV_LAYOUT_PAGED5D    : K [num_blocks, Hkv, D/x, block_size, x],
 *                           V [num_blocks, Hkv, D, block_size],
 *                           x = 16 / sizeof(cache element)
 *                           (reshape_and_cache.metal:20-23).
 *   PKV_LAYOUT_TOKEN_MAJOR: K and V [num_slots, Hkv, D] with
 *                           slot = block * block_size + offset; this is both
 *                           the MHATokenPool buffer (memory_pool.py:102-108)
 *                           and the flash layout [num_blocks, block_size,
 *                           Hkv, D] (reshape_and_cache.metal:104-107). */
enum { PKV_LAYOUT_PAGED5D = 0, PKV_LAYOUT_TOKEN_MAJOR = 1 };

/* Library identification string (build flags and target). */
const char* pkv_version(void);

/* Message describing the last non-zero status returned on this thread. */
const char* pkv_last_error(void);

/*
 * Slot-mapped KV append.
 * Replaces ReshapeAndCache (mlx_cache.cpp:40-97, :256-278) for
 * PKV_LAYOUT_PAGED5D and ReshapeAndCacheFlash (mlx_cache.cpp:101-153,
 * :280-300) for PKV_LAYOUT_TOKEN_MAJOR; kernel semantics follow
 * reshape_and_cache.metal:35-69 and :115-136.
 *
 * key/value   : [num_tokens, num_kv_heads, head_size], row stride
 *               key_stride / value_stride; the inner [Hkv, D] is contiguous.
 * slot_mapping: [num_tokens]; a negative slot skips the token
 *               (reshape_and_cache.metal:36-39).  Slots >= num_slots are
 *               skipped as well (the reference does not check them).
 * block_size/x: used by PKV_LAYOUT_PAGED5D only; x must be
 *               16 / sizeof(cache element).
 * num_slots   : num_blocks * block_size (PAGED5D) or the first dimension of
 *               the token-major buffers.
 * kv_dtype -> cache_dtype pairs: equal types, or F32 -> F16 / F32 -> BF16
 *               (round to nearest even; NaN -> 0x7FC0 for BF16), or any of
 *               F32 / F16 / BF16 -> PKV_FP8_E4M3.
 * k_scale, v_scale: FP8 caches store encode(x / k_scale) for keys and
 *               encode(x / v_scale) for values (the quantisation of
 *               convert_fp8.metal:33-35; both finite and nonzero; a
 *               power-of-two scale multiplies by its exact reciprocal, which
 *               is the same result).  FP8 caches need 16-byte aligned
 *               key/value rows and caches, and x = 16 in the paged layout.
 *               Ignored for other caches (the reference has no FP8 append).
 */
int pkv_reshape_and_cache(const void* key, const void* value,
                          void* key_cache, void* value_cache,
                          const int32_t* slot_mapping, int64_t num_tokens,
                          int32_t num_kv_heads, int32_t head_size,
                          int64_t key_stride, int64_t value_stride,
                          int32_t layout, int32_t block_size, int32_t x,
                          int64_t num_slots, int32_t kv_dtype,
                          int32_t cache_dtype, float k_scale, float v_scale,
                          void* stream);

/*
 * Workspace bytes that pkv_paged_attention needs for these sizes:
 * PKV_COUNTER_BYTES of arrival counters, then per-partition (max, sum)
 * pairs and per-partition outputs (float32).  partition_size = 0 selects
 * the single-pass (v1) semantics; the library then chooses its own
 * schedule.  Zero-fill a workspace once, when it is allocated: its first
 * PKV_COUNTER_BYTES count the partitions of each (sequence, KV head) as
 * their workgroups finish, and every call leaves them zero again; the rest
 * needs no initialisation (each launch reads only what it wrote).  Calls
 * ordered on one stream may share one workspace, also with
 * pkv_paged_attention_cascade; calls that overlap in time must not.
 * Returns 0 for invalid sizes.
 */
#define PKV_COUNTER_BYTES 65536
size_t pkv_paged_attention_workspace_size(int32_t num_seqs, int32_t num_heads,
                                          int32_t num_kv_heads,
                                          int32_t head_size,
                                          int32_t max_seq_len,
                                          int32_t partition_size);

/*
 * Block-table decode attention.
 * Replaces PagedAttentionV1 (mlx_paged_attention.cpp:93-144, :150-213);
 * semantics follow paged_attention_kernels.metal:37-168:
 *   out[s,h,:] = sum_t softmax_t(scale * q[s,h].k_t + alibi[h]*(t-ctx+1)) v_t
 * with the GQA map kv_head = h / (num_heads / num_kv_heads), the softmax
 * denominator (sum + 1e-6), fp32 accumulation, and a zero output row when
 * context_lens[s] == 0 or context_lens[s] > max_seq_len.
 *
 * partition_size = 0 : paged_attention_v1 semantics (one softmax over the
 *                      whole context; the split is an internal detail).
 * partition_size > 0 : split-K (paged_attention_v2): partitions of
 *                      partition_size tokens, merged by log-sum-exp.  Must be
 *                      a multiple of 16 and of block_size, at most 4096.  A
 *                      workgroup takes a run of consecutive partitions (as
 *                      many as keep one workgroup per CU) and merges them as
 *                      it streams; the result is the same log-sum-exp merge.
 * Launches (all on `stream`): for partition_size = 0, contexts of at most
 * 16384 tokens and at least one (sequence, KV head) item per resident
 * workgroup, one persistent kernel that gives each item to one workgroup,
 * longest contexts first (with two or more items per CU, GQA groups of at
 * most 4 and contexts of at most 8192 tokens -- 4096 over FP8 caches at
 * head sizes 64 and 128 -- items of four sequences that share the MFMA
 * columns, so that tiles the four map to the same block are read once);
 * otherwise a partition kernel.  When a sequence has more than one
 * partition: with at most 8 partitions per sequence (paged layout, and
 * num_seqs * num_kv_heads counters within the counter region), the
 * workgroup that finishes a sequence's last partition merges them (log-sum-
 * exp, in partition order: results do not depend on which workgroup
 * merges); otherwise a log-sum-exp merge kernel follows.
 * query   : [num_seqs, num_heads, head_size], row stride q_stride.
 * out     : [num_seqs, num_heads, head_size] contiguous, same dtype as
 *           query, 16-byte aligned.
 * block_tables: [num_seqs, max_num_blocks_per_seq]; entries past
 *               ceil(ctx / block_size) are never read.  Entries outside
 *               [0, num_blocks) mask their tokens out.
 * alibi_slopes: [num_heads] float32 or NULL.
 * Cache layouts and strides (elements):
 *   PAGED5D     K [num_blocks, Hkv, D/x, block_size, x], V [num_blocks, Hkv,
 *               D, block_size]; k_block_stride/k_head_stride (and v_*) are
 *               the strides of the block and head dimensions.
 *   TOKEN_MAJOR K and V [num_blocks, block_size, Hkv, D] (the flash layout;
 *               block_size 1 is MHATokenPool's [rows, Hkv, D] with the
 *               block table holding slots).  k_block_stride is the stride
 *               between blocks and a multiple of block_size; the rows of a
 *               block are k_block_stride / block_size apart, and each must
 *               hold (Hkv - 1) * k_head_stride + D elements, k_head_stride
 *               >= D being the head offset inside a row; the D elements of
 *               one head are contiguous (likewise v_*).  block_size may
 *               also be 1.  The persistent path covers max_seq_len up to
 *               4096 here (2048 for head sizes above 128; 16384 for
 *               PAGED5D).
 *               (The reference decodes the paged layout only; this is the
 *               gather-free path its pool asks for, memory_pool.py:110-112.)
 * (q_dtype, cache_dtype): (BF16,BF16), (F16,F16), (F32,BF16), (F32,F16),
 *   (F32,F32) in the paged layout (x = 4; scores and PV on float32 MFMA, so
 *   nothing is rounded to 16 bits; the V base and strides then need 16-byte
 *   alignment), and (BF16|F16|F32, FP8_E4M3): FP8 caches in the paged layout (x = 16,
 *   head_size a multiple of 16) hold codes of K / k_scale and V / v_scale
 *   (pkv_reshape_and_cache); attention runs on decode(code) * scale, i.e.
 *   scores scale * k_scale * (q . decode(k)) and output v_scale *
 *   sum p decode(v) / (sum p + 1e-6).  The codes are dequantised exactly
 *   into the query's 16-bit type (float16 for a float32 query).  k_scale and
 *   v_scale are ignored for other caches.
 * head_size in {32,64,80,96,112,120,128,192,256}; block_size in {8,16,32}
 * (isValidConfig, mlx_paged_attention.cpp:52-59), or 1 with TOKEN_MAJOR.
 */
int pkv_paged_attention(void* out, const void* query, const void* key_cache,
                        const void* value_cache, const int32_t* block_tables,
                        const int32_t* context_lens,
                        const float* alibi_slopes, int32_t num_seqs,
                        int32_t num_heads, int32_t num_kv_heads,
                        int32_t head_size, int32_t block_size,
                        int32_t max_num_blocks_per_seq, int32_t max_seq_len,
                        int64_t num_blocks, float scale, int64_t q_stride,
                        int64_t k_block_stride, int64_t k_head_stride,
                        int64_t v_block_stride, int64_t v_head_stride,
                        int32_t layout, int32_t partition_size,
                        void* workspace, size_t workspace_bytes,
                        int32_t q_dtype, int32_t cache_dtype,
                        float k_scale, float v_scale, void* stream);

/*
 * Shared-prefix plan of pkv_paged_attention_cascade, built on the host from
 * the block tables and context lengths
 * (sglang_mlx_amd.srt.mem_cache.build_cascade_plan).  All arrays are int32
 * device buffers.
 *   prefix_lens [num_seqs]: leading tokens of each sequence that the prefix
 *                pass covers, 0 for none; a multiple of block_size and of 16
 *                (of 8 for 8-token blocks), at most the sequence's context.
 *   members     [num_members]: sequence ids, each prefix group's members
 *                adjacent.
 *   tiles       [num_tiles][4] (16-byte aligned): (member_begin,
 *                member_count, token_begin, token_end) of one prefix-pass
 *                unit.  members[member_begin .. +member_count) map tokens
 *                [0, token_end) to the same blocks as the first of them and
 *                have prefix_lens >= token_end; member_count * (num_heads /
 *                num_kv_heads) <= 128; token_begin is a multiple of
 *                chunk_tokens and token_end - token_begin <= chunk_tokens.
 *                The units of a group cover its prefix [0, prefix_len)
 *                chunk by chunk, and every member sits in the units of its
 *                group.
 *   parts       [num_parts][2] (8-byte aligned): (sequence, k) of each tail
 *                partition, the order the tail pass takes them in (longest
 *                first balances the launch).  Partition k of a sequence
 *                covers tokens [pre + k * part_tokens, min(context, pre +
 *                (k + 1) * part_tokens)) after its prefix pre; every
 *                sequence, whatever its context, has max(1, ceil((context
 *                - pre) / part_tokens)) partitions, each listed once.
 *   chunk_tokens: a multiple of 16 and of block_size, at most 4096.
 *   max_chunks  : at least ceil(prefix_lens[s] / chunk_tokens) for every s.
 *   part_tokens : a multiple of 16 and of block_size, at most 1024.
 *   max_parts   : at least the partitions of every sequence.
 * A plan that breaks these rules never makes a kernel read or write outside
 * its buffers, but the rows it concerns are then undefined.
 */
typedef struct pkv_cascade_plan {
  const int32_t* prefix_lens;
  const int32_t* members;
  const int32_t* tiles;
  const int32_t* parts;
  int32_t num_members;
  int32_t num_tiles;
  int32_t num_parts;
  int32_t chunk_tokens;
  int32_t max_chunks;
  int32_t part_tokens;
  int32_t max_parts;
} pkv_cascade_plan;

/*
 * Workspace bytes of pkv_paged_attention_cascade: the larger of the one-pass
 * decode's (pkv_paged_attention_workspace_size with partition_size 0) and
 * the counter region plus the partial states' (num_seqs * num_heads *
 * (max_chunks + max_parts) * (head_size + 2) float32, in four parts each
 * 256-byte aligned).  Zero-filled once when allocated, as for
 * pkv_paged_attention (the cascade leaves the counter region untouched).
 * Returns 0 for invalid sizes.
 */
size_t pkv_paged_attention_cascade_workspace_size(int32_t num_seqs,
                                                  int32_t num_heads,
                                                  int32_t num_kv_heads,
                                                  int32_t head_size,
                                                  int32_t max_seq_len,
                                                  int32_t max_chunks,
                                                  int32_t max_parts);

/*
 * Decode attention with radix-shared prefixes computed once per group
 * (cascade).  No counterpart in the reference, whose radix cache shares
 * token slots but whose kernel reads every sequence's context in full
 * (paged_attention_kernels.metal:37-168); the result is
 * pkv_paged_attention's with partition_size 0 (paged_attention_v1), to
 * within floating-point rounding, for any plan that follows the rules of
 * pkv_cascade_plan.  Arguments as pkv_paged_attention, PAGED5D layout.
 * Launches two kernels on `stream`.  The first has two kinds of
 * workgroups, running side by side: prefix work (one workgroup per (plan
 * tile, KV head): the tile's query rows against one chunk of the shared
 * prefix, K/V staged through LDS, partial softmax states to the workspace)
 * and tail work (one wavefront per (tail partition, KV head): the
 * partition's tokens streamed, its partial state to the workspace, or the
 * output row when the sequence has no prefix and one partition).  The
 * second merges each remaining row's states by log-sum-exp, in a fixed
 * order, and writes the row.  The cascade kernels take 16-bit queries over
 * caches of the same type or FP8 (FP8 with blocks of 16 and 32 tokens),
 * head sizes 64 and 128, GQA groups of at most 16 and V rows aligned for
 * 16-byte loads; other shapes run the one-pass decode of
 * pkv_paged_attention (the plan is then unused).
 */
int pkv_paged_attention_cascade(void* out, const void* query,
                                const void* key_cache,
                                const void* value_cache,
                                const int32_t* block_tables,
                                const int32_t* context_lens,
                                const float* alibi_slopes,
                                const pkv_cascade_plan* plan,
                                int32_t num_seqs, int32_t num_heads,
                                int32_t num_kv_heads, int32_t head_size,
                                int32_t block_size,
                                int32_t max_num_blocks_per_seq,
                                int32_t max_seq_len, int64_t num_blocks,
                                float scale, int64_t q_stride,
                                int64_t k_block_stride, int64_t k_head_stride,
                                int64_t v_block_stride, int64_t v_head_stride,
                                void* workspace, size_t workspace_bytes,
                                int32_t q_dtype, int32_t cache_dtype,
                                float k_scale, float v_scale, void* stream);

/*
 * Block-table decode attention that allocates nothing and takes no
 * workspace.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Arguments, semantics and results are
 * those of pkv_paged_attention without its workspace / workspace_bytes.
 * The partials of the split-K path live in a static device array of
 * PKV_NOALLOC_SCRATCH_BYTES per GPU, which the library holds from its first
 * call on that GPU until the process ends; a call whose sizes need more
 * (pkv_paged_attention_workspace_size) fails with PKV_ERR_UNSUPPORTED
 * before any HIP call, whether or not the launch would use it.  The array
 * is laid out as a workspace and starts zeroed, so its counter region is
 * zero as pkv_paged_attention requires (every call leaves it zero); the rest
 * is read only where the same call wrote it, so stale contents from an
 * earlier call do not matter.  Every call on one GPU shares that GPU's array: calls that
 * overlap in time on one GPU (different streams, or threads) race and give
 * undefined results; order them on one stream.  The first call on a GPU
 * looks the array's address up with hipGetSymbolAddress (no allocation).
 */
#define PKV_NOALLOC_SCRATCH_BYTES (32u << 20) /* 32 MiB per GPU */
int pkv_paged_attention_noalloc(void* out, const void* query, const void* key_cache,
                                const void* value_cache, const int32_t* block_tables,
                                const int32_t* context_lens,
                                const float* alibi_slopes, int32_t num_seqs,
                                int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_size, int32_t block_size,
                                int32_t max_num_blocks_per_seq, int32_t max_seq_len,
                                int64_t num_blocks, float scale, int64_t q_stride,
                                int64_t k_block_stride, int64_t k_head_stride,
                                int64_t v_block_stride, int64_t v_head_stride,
                                int32_t layout, int32_t partition_size,
                                int32_t q_dtype, int32_t cache_dtype,
                                float k_scale, float v_scale, void* stream);

/*
 * Whole-block copies between paged caches.  A block is block_bytes
 * contiguous bytes of a plane (a [num_blocks, ...] cache tensor), so every
 * layout and dtype is the same copy.  For each (src, dst) pair of
 * block_mapping and each plane i, block dst of dst_planes[i] receives block
 * src of src_planes[i].
 *   copy_blocks: pass each layer's K cache and V cache as planes that are
 *     their own source (src_planes == dst_planes).  Replaces copy_blocks
 *     (mlx_cache.cpp:302-346, copy_blocks.metal:9-39).
 *   swap_blocks: one plane pair (src, dst) on the device.  Replaces
 *     swap_blocks (mlx_cache.cpp:348-370, copy_blocks.metal:55-70); copies
 *     between host and device memory stay with the caller.
 * src_planes, dst_planes: host arrays of num_planes device pointers.
 * block_mapping: device int64 [num_pairs][2]; pairs whose ids fall outside
 *   [0, src_blocks) or [0, dst_blocks) are skipped.
 * Pairs and planes are copied concurrently: a block that is both a source
 * and a destination in one call gives an unspecified result, as in the
 * reference.  Launches on `stream`; nothing is allocated.
 */
int pkv_copy_blocks(void* const* src_planes, void* const* dst_planes,
                    int32_t num_planes, int64_t src_blocks,
                    int64_t dst_blocks, int64_t block_bytes,
                    const int64_t* block_mapping, int64_t num_pairs,
                    void* stream);

/*
 * Element-wise conversion with a scale.  Replaces convert_fp8_kernel
 * (convert_fp8.metal:13-80, all 16 pairs of PKV_F32, PKV_F16, PKV_BF16 and
 * PKV_FP8_E4M3), which the reference compiles but never binds:
 *   FP8 -> T  : decode(code) * scale, rounded to T
 *   T -> FP8  : encode(float(x) / scale)
 *   FP8 -> FP8: encode(decode(code) * scale)
 *   T -> U    : float(x) * scale, rounded to U
 * Rounding to half / bfloat16 is to nearest even (bfloat16: NaN -> 0x7FC0).
 * The encoder follows float8.metal:72-120 bit for bit, including its results
 * for 256 <= |x| < 2^14 (small codes; 256 -> +0) and for values that round
 * up to 2^-6 (+-0); from |x| >= 2^14, where the reference's shifts are
 * undefined, it gives +-inf.  dst and src may be the same buffer when the
 * element sizes are equal and must not otherwise overlap.
 */
int pkv_convert_fp8(void* dst, const void* src, int64_t num_elements,
                    float scale, int32_t src_dtype, int32_t dst_dtype,
                    void* stream);

/*
 * LDS bytes available to one workgroup on a device.
 * Replaces get_max_shared_memory_per_block_device_attribute
 * (mlx_device.cpp:16-20, bindings.cpp:130-133).
 */
int pkv_max_shared_memory_per_block(int32_t device_id, int64_t* out);

/*
 * hipDeviceGetAttribute passthrough.  Replaces get_device_attribute
 * (mlx_device.cpp:12-14, bindings.cpp:125-128), which always throws in the
 * reference; here `attribute` is a hipDeviceAttribute_t value.
 */
int pkv_get_device_attribute(int32_t attribute, int32_t device_id,
                             int64_t* out);

#ifdef __cplusplus
}
#endif

#endif /* PAGEDKV_H */
