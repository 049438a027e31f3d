// extern "C" entry points of libpagedkv_gfx950.so (declared in
// include/pagedkv.h).  They check arguments before any HIP call, size the
// decode workspace, pick the kernel instantiation and launch it on the
// caller's stream.  Nothing here allocates device memory or synchronises.
#include <stdio.h>
#include <string.h>

#include <string>

#include "../../include/pagedkv.h"
#include "pkv_launch.h"

#include <algorithm>
#include <cmath>
#include <mutex>

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

// A failed HIP call also leaves its error as the thread's pending "last
// error", which the next hipGetLastError() of any code on the thread (this
// library's launch checks, torch's) would report as its own.  The status
// returned here already carries it, so it is reset.
int hip_fail(hipError_t e, const char* where) {
  (void)hipGetLastError();
  return fail(PKV_ERR_HIP, std::string(where) + ": " + hipGetErrorString(e));
}

// Launches report failure only through hipGetLastError(), which returns the
// thread's pending error whichever call left it.  Each entry point clears it
// right before launching, so that a launch status describes that launch;
// an error left pending by other code was returned by the call that caused
// it.
void clear_pending_error() { (void)hipGetLastError(); }

int elem_bytes(int32_t dt) { return dt == PKV_F32 ? 4 : dt == PKV_FP8_E4M3 ? 1 : 2; }
// Nonzero finite scale whose reciprocal is exact: a power of two whose
// inverse is a normal float.
bool exact_reciprocal(float s) {
  int e = 0;
  const float m = std::frexp(s, &e);
  return std::isfinite(s) && (m == 0.5f || m == -0.5f) && e > -125 && e < 127;
}
bool valid_dtype(int32_t dt) { return dt == PKV_F32 || dt == PKV_F16 || dt == PKV_BF16; }
bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// Supported decode shapes (isValidConfig, mlx_paged_attention.cpp:52-59).
bool valid_head_size(int32_t d) {
  static const int hs[] = {32, 64, 80, 96, 112, 120, 128, 192, 256};
  for (int v : hs)
    if (v == d) return true;
  return false;
}
bool valid_block_size(int32_t b) { return b == 8 || b == 16 || b == 32; }

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Partition size of paged_attention_v1 on the partition path: the largest
// (at most 4096 tokens, at least 256) that still gives one workgroup per CU
// of MI355X (256).  Measured at 32K-128K contexts, fewer and longer
// partitions win once every CU has a workgroup: the per-workgroup start-up
// and merge cost is then paid fewer times.
constexpr int64_t kTargetWorkgroups = 256;
int32_t v1_partition(int32_t num_seqs, int32_t units, int32_t max_seq_len) {
  int32_t ps = pkv::kMaxPartition;
  while (ps > 256 && (int64_t)num_seqs * units * ceil_div(max_seq_len, ps) < kTargetWorkgroups) ps /= 2;
  return ps;
}

// Resolves the tokens each partition-kernel workgroup covers and the
// partition count of the workspace; returns a status.
//
// An explicit partition_size (paged_attention_v2) is the split granularity:
// the context is cut into partitions of that many tokens, and a workgroup
// takes a run of consecutive partitions -- as many as still leave the grid
// v1 would use (one workgroup per CU, at most 4096 tokens), at least one --
// whose softmax states it merges as it streams them; the merge kernel
// combines the runs with the same log-sum-exp rule.  Merging inside the
// workgroup and in the merge kernel give the same softmax, so the run only
// moves where partitions meet.  Measured at the Qwen2-7B 32K-128K contexts,
// one workgroup per 512-token partition cost up to 13% more than runs (B4
// 128K: 4096 workgroups and a 256-way merge, 195 against 172 us): each
// workgroup pays its own start-up, and the merge reads 8x the partials.
int resolve_partition(int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads, int32_t max_seq_len,
                      int32_t block_size, int32_t partition_size, int32_t* ps_out, int32_t* parts_out) {
  if (num_seqs < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return fail(PKV_ERR_INVALID, "num_heads must be divisible by num_kv_heads");
  if (max_seq_len <= 0) return fail(PKV_ERR_INVALID, "max_seq_len must be positive");
  const int32_t group = num_heads / num_kv_heads;
  const int32_t units = num_kv_heads * ((group + 15) / 16);
  int32_t ps = partition_size;
  if (ps == 0) {
    ps = v1_partition(num_seqs, units, max_seq_len);
  } else if (ps < 0 || ps % pkv::kTile != 0 || (block_size > 0 && ps % block_size != 0) ||
             ps > pkv::kMaxPartition) {
    return fail(PKV_ERR_INVALID,
                "partition_size must be a positive multiple of 16 and of block_size, at most 4096");
  } else {
    ps *= std::max<int32_t>(1, v1_partition(num_seqs, units, max_seq_len) / ps);
  }
  const int64_t parts = ceil_div(max_seq_len, ps);
  if (parts > pkv::kMaxParts)
    return fail(PKV_ERR_UNSUPPORTED, "max_seq_len / partition_size exceeds 65536 partitions");
  // One 256-thread workgroup per (partition, sequence, unit); HIP bounds a
  // launch to 2^32 work-items.
  if (parts * num_seqs * units * 256 >= ((int64_t)1 << 32))
    return fail(PKV_ERR_UNSUPPORTED, "num_seqs * num_kv_heads * partitions exceeds the launch grid limit");
  *ps_out = ps;
  *parts_out = (int32_t)parts;
  return PKV_OK;
}

}  // namespace

static_assert(PKV_COUNTER_BYTES == pkv::kCounterBytes, "the header's counter region is the kernels'");

namespace pkv {
DecodeWorkspace decode_workspace_layout(int32_t num_seqs, int32_t num_heads, int32_t head_size,
                                        int32_t max_parts) {
  DecodeWorkspace w;
  auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
  w.ml_bytes = align((size_t)num_seqs * num_heads * max_parts * 2 * sizeof(float));
  w.o_bytes = align((size_t)num_seqs * num_heads * max_parts * head_size * sizeof(float));
  w.total = (size_t)kCounterBytes + w.ml_bytes + w.o_bytes;
  return w;
}
CascadeWorkspace cascade_workspace_layout(int32_t num_seqs, int32_t num_heads, int32_t head_size,
                                          int32_t max_chunks, int32_t max_parts) {
  CascadeWorkspace w;
  auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
  w.ml_bytes = align((size_t)num_seqs * num_heads * max_chunks * 2 * sizeof(float));
  w.o_bytes = align((size_t)num_seqs * num_heads * max_chunks * head_size * sizeof(float));
  w.tail_ml_bytes = align((size_t)num_seqs * num_heads * max_parts * 2 * sizeof(float));
  w.tail_o_bytes = align((size_t)num_seqs * num_heads * max_parts * head_size * sizeof(float));
  w.total = (size_t)kCounterBytes + w.ml_bytes + w.o_bytes + w.tail_ml_bytes + w.tail_o_bytes;
  return w;
}
}  // namespace pkv

extern "C" {

const char* pkv_version(void) { return "pagedkv gfx950 (hipcc -O3, wave64, MFMA 16x16x32/16x16x16)"; }

const char* pkv_last_error(void) { return g_last_error.c_str(); }

int pkv_reshape_and_cache(const void* key, const void* value, void* key_cache, void* value_cache,
                          const int32_t* slot_mapping, int64_t num_tokens, int32_t num_kv_heads,
                          int32_t head_size, int64_t key_stride, int64_t value_stride, int32_t layout,
                          int32_t block_size, int32_t x, int64_t num_slots, int32_t kv_dtype,
                          int32_t cache_dtype, float k_scale, float v_scale, void* stream) {
  if (num_tokens < 0) return fail(PKV_ERR_INVALID, "num_tokens must be non-negative");
  if (num_kv_heads <= 0 || head_size <= 0) return fail(PKV_ERR_INVALID, "num_kv_heads and head_size must be positive");
  const bool fp8 = cache_dtype == PKV_FP8_E4M3;
  if (!valid_dtype(kv_dtype) || !(valid_dtype(cache_dtype) || fp8))
    return fail(PKV_ERR_INVALID, "Unsupported dtype");
  if (!(kv_dtype == cache_dtype || fp8 || (kv_dtype == PKV_F32 && cache_dtype != PKV_F32)))
    return fail(PKV_ERR_UNSUPPORTED, "Unsupported key/cache dtype pair");
  if (fp8 && !(std::isfinite(k_scale) && std::isfinite(v_scale) && k_scale != 0.f && v_scale != 0.f))
    return fail(PKV_ERR_INVALID, "k_scale and v_scale must be finite and nonzero for FP8 caches");
  if (layout != PKV_LAYOUT_PAGED5D && layout != PKV_LAYOUT_TOKEN_MAJOR)
    return fail(PKV_ERR_INVALID, "Unknown cache layout");
  if (num_slots <= 0 || num_slots > INT32_MAX) return fail(PKV_ERR_INVALID, "num_slots must be in [1, 2^31)");
  const int64_t row = (int64_t)num_kv_heads * head_size;
  if (key_stride < row || value_stride < row)
    return fail(PKV_ERR_INVALID, "key/value row stride is smaller than num_kv_heads * head_size");
  if (layout == PKV_LAYOUT_PAGED5D) {
    if (block_size <= 0) return fail(PKV_ERR_INVALID, "block_size must be positive");
    if (x != 16 / elem_bytes(cache_dtype))
      return fail(PKV_ERR_INVALID, "key_cache last dimension must be 16 / sizeof(cache element)");
    if (head_size % x != 0) return fail(PKV_ERR_INVALID, "head_size must be a multiple of x");
    if (num_slots % block_size != 0) return fail(PKV_ERR_INVALID, "num_slots must be a multiple of block_size");
  }
  // The FP8 token-major kernel encodes and stores 8 elements per lane step,
  // so a row must hold whole groups of 8 (and stays 8-byte aligned).
  if (fp8 && layout == PKV_LAYOUT_TOKEN_MAJOR && row % 8 != 0)
    return fail(PKV_ERR_UNSUPPORTED, "FP8 token-major caches need num_kv_heads * head_size to be a multiple of 8");
  if (num_tokens == 0) return PKV_OK;
  if (!key || !value || !key_cache || !value_cache || !slot_mapping)
    return fail(PKV_ERR_INVALID, "null buffer");
  const int kb = elem_bytes(kv_dtype);
  const bool aligned = aligned16(key) && aligned16(value) && aligned16(key_cache) && aligned16(value_cache) &&
                       (key_stride * kb) % 16 == 0 && (value_stride * kb) % 16 == 0 &&
                       (layout == PKV_LAYOUT_TOKEN_MAJOR || (head_size * kb) % 16 == 0);
  if (fp8 && !aligned)
    return fail(PKV_ERR_INVALID, "FP8 caches need 16-byte aligned key/value rows and caches");
  pkv::RacParams p;
  p.key = key;
  p.value = value;
  p.key_cache = key_cache;
  p.value_cache = value_cache;
  p.slot_mapping = slot_mapping;
  p.num_tokens = num_tokens;
  p.key_stride = key_stride;
  p.value_stride = value_stride;
  p.num_slots = num_slots;
  p.num_heads = num_kv_heads;
  p.head_size = head_size;
  p.block_size = layout == PKV_LAYOUT_PAGED5D ? block_size : 1;
  p.layout = layout;
  p.kv_dtype = kv_dtype;
  p.cache_dtype = cache_dtype;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.scales_pow2 = exact_reciprocal(k_scale) && exact_reciprocal(v_scale);
  p.k_inv = p.scales_pow2 ? 1.f / k_scale : 0.f;
  p.v_inv = p.scales_pow2 ? 1.f / v_scale : 0.f;
  clear_pending_error();
  const hipError_t e = pkv::launch_reshape_and_cache(p, aligned, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "reshape_and_cache launch");
  return PKV_OK;
}

size_t pkv_paged_attention_workspace_size(int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                          int32_t head_size, int32_t max_seq_len, int32_t partition_size) {
  int32_t ps = 0, parts = 0;
  if (head_size <= 0) return 0;
  if (resolve_partition(num_seqs, num_heads, num_kv_heads, max_seq_len, 0, partition_size, &ps, &parts) != PKV_OK)
    return 0;
  return pkv::decode_workspace_layout(num_seqs, num_heads, head_size, parts).total;
}

size_t pkv_paged_attention_cascade_workspace_size(int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                                  int32_t head_size, int32_t max_seq_len, int32_t max_chunks,
                                                  int32_t max_parts) {
  const size_t v1 = pkv_paged_attention_workspace_size(num_seqs, num_heads, num_kv_heads, head_size, max_seq_len, 0);
  if (v1 == 0 || max_chunks <= 0 || max_chunks > 65536 || max_parts <= 0 || max_parts > 65536) return 0;
  return std::max(v1, pkv::cascade_workspace_layout(num_seqs, num_heads, head_size, max_chunks, max_parts).total);
}

}  // extern "C"

namespace {

// Static scratch of pkv_paged_attention_noalloc: one copy per device, kept
// until the process ends.  Host code never names the array itself (on the
// host its name is a stand-in, not a device address); it uses the address
// hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[PKV_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch, looked up once per device
// with that device current.
int static_scratch(void** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(PKV_ERR_UNSUPPORTED, "device id beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(PKV_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return PKV_OK;
}

// pkv_paged_attention, and with use_scratch the no-allocation variant (the
// workspace is then the static scratch, fetched after every argument check).
int paged_attention_impl(void* out, const void* query, const void* key_cache, const void* value_cache,
                         const int32_t* block_tables, const int32_t* context_lens, const float* alibi_slopes,
                         int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                         int32_t block_size, int32_t max_num_blocks_per_seq, int32_t max_seq_len,
                         int64_t num_blocks, float scale, int64_t q_stride, int64_t k_block_stride,
                         int64_t k_head_stride, int64_t v_block_stride, int64_t v_head_stride, int32_t layout,
                         int32_t partition_size, void* workspace, size_t workspace_bytes, bool use_scratch,
                         int32_t q_dtype, int32_t cache_dtype, float k_scale, float v_scale, void* stream,
                         const pkv_cascade_plan* plan = nullptr) {
  if (num_seqs < 0) return fail(PKV_ERR_INVALID, "num_seqs must be non-negative");
  int32_t ps = 0, parts = 0;
  const int st = resolve_partition(num_seqs, num_heads, num_kv_heads, max_seq_len, block_size, partition_size,
                                   &ps, &parts);
  if (st != PKV_OK) return st;
  if (max_num_blocks_per_seq <= 0 || (int64_t)max_seq_len > (int64_t)max_num_blocks_per_seq * block_size)
    return fail(PKV_ERR_INVALID, "max_seq_len exceeds block table capacity");
  if (layout != PKV_LAYOUT_PAGED5D && layout != PKV_LAYOUT_TOKEN_MAJOR)
    return fail(PKV_ERR_INVALID, "Unknown cache layout");
  const bool rows = layout == PKV_LAYOUT_TOKEN_MAJOR;
  if (!valid_head_size(head_size) || !(valid_block_size(block_size) || (rows && block_size == 1)))
    return fail(PKV_ERR_UNSUPPORTED, "Unsupported head_size/block_size for paged_attention");
  const bool fp8 = cache_dtype == PKV_FP8_E4M3;
  const bool pair_ok =
      (q_dtype == PKV_BF16 && cache_dtype == PKV_BF16) || (q_dtype == PKV_F16 && cache_dtype == PKV_F16) ||
      (q_dtype == PKV_F32 && (cache_dtype == PKV_BF16 || cache_dtype == PKV_F16 || cache_dtype == PKV_F32)) ||
      (fp8 && (q_dtype == PKV_BF16 || q_dtype == PKV_F16 || q_dtype == PKV_F32));
  if (!pair_ok) return fail(PKV_ERR_UNSUPPORTED, "Unsupported query/cache dtype pair for paged_attention");
  if (cache_dtype == PKV_F32 && rows)
    return fail(PKV_ERR_UNSUPPORTED, "float32 caches are read in the paged layout");
  if (fp8 && (rows || head_size % 16 != 0))
    return fail(PKV_ERR_UNSUPPORTED, "FP8 caches are read in the paged layout with head_size a multiple of 16");
  if (fp8 && !(std::isfinite(k_scale) && std::isfinite(v_scale) && k_scale != 0.f && v_scale != 0.f))
    return fail(PKV_ERR_INVALID, "k_scale and v_scale must be finite and nonzero for FP8 caches");
  if (num_blocks <= 0) return fail(PKV_ERR_INVALID, "num_blocks must be positive");
  if (num_seqs == 0) return PKV_OK;
  if (!out || !query || !key_cache || !value_cache || !block_tables || !context_lens)
    return fail(PKV_ERR_INVALID, "null buffer");
  if (!aligned16(out)) return fail(PKV_ERR_INVALID, "out must be 16-byte aligned");
  const int qb = elem_bytes(q_dtype);
  if (!aligned16(query) || (q_stride * qb) % 16 != 0 || q_stride < (int64_t)num_heads * head_size)
    return fail(PKV_ERR_INVALID, "query rows must be 16-byte aligned with stride >= num_heads * head_size");
  if (rows && (k_block_stride % block_size != 0 || v_block_stride % block_size != 0 ||
               k_head_stride < head_size || v_head_stride < head_size ||
               k_block_stride / block_size < (int64_t)(num_kv_heads - 1) * k_head_stride + head_size ||
               v_block_stride / block_size < (int64_t)(num_kv_heads - 1) * v_head_stride + head_size))
    return fail(PKV_ERR_INVALID, "token-row caches need rows that hold num_kv_heads heads of head_size");
  if (rows && num_blocks > (int64_t)INT32_MAX / block_size)
    return fail(PKV_ERR_UNSUPPORTED, "token-row caches hold at most 2^31 - 1 rows");
  // Token rows: the row stride takes the place of the block stride below.
  const int64_t kbs = rows ? k_block_stride / block_size : k_block_stride;
  const int64_t vbs = rows ? v_block_stride / block_size : v_block_stride;
  // K: 16-byte loads; V: 8-byte loads in the paged layout, 16-byte loads of
  // token rows and of float32 caches (the same byte alignment for FP8
  // caches, whose wide tiles load 16 K codes and 8 V codes per lane).
  const int64_t cb = elem_bytes(cache_dtype);
  const int64_t k_align = 16;
  const int64_t v_align = (rows || cache_dtype == PKV_F32) ? 16 : 8;
  if (!aligned16(key_cache) || (kbs * cb) % k_align != 0 || (k_head_stride * cb) % k_align != 0 ||
      (reinterpret_cast<uintptr_t>(value_cache) % v_align) != 0 || (vbs * cb) % v_align != 0 ||
      (v_head_stride * cb) % v_align != 0)
    return fail(PKV_ERR_INVALID, "cache base or strides are not aligned for vector loads");
  if (plan != nullptr) {
    if (plan->prefix_lens == nullptr || plan->parts == nullptr)
      return fail(PKV_ERR_INVALID, "cascade plan: prefix_lens and parts are required");
    if (plan->num_tiles < 0 || plan->num_members < 0 || plan->num_parts < 0)
      return fail(PKV_ERR_INVALID, "cascade plan: num_tiles, num_members and num_parts must be non-negative");
    if (reinterpret_cast<uintptr_t>(plan->parts) % 8 != 0)
      return fail(PKV_ERR_INVALID, "cascade plan: parts must be 8-byte aligned");
    if (plan->num_tiles > 0 && (plan->members == nullptr || plan->tiles == nullptr || plan->num_members == 0))
      return fail(PKV_ERR_INVALID, "cascade plan: tiles need members");
    if (plan->tiles != nullptr && !aligned16(plan->tiles))
      return fail(PKV_ERR_INVALID, "cascade plan: tiles must be 16-byte aligned");
    if (plan->chunk_tokens <= 0 || plan->chunk_tokens % pkv::kTile != 0 || plan->chunk_tokens % block_size != 0 ||
        plan->chunk_tokens > pkv::kMaxPrefixChunk)
      return fail(PKV_ERR_INVALID, "cascade plan: chunk_tokens must be a positive multiple of 16 and of block_size, "
                                   "at most 4096");
    if (plan->part_tokens <= 0 || plan->part_tokens % pkv::kTile != 0 || plan->part_tokens % block_size != 0 ||
        plan->part_tokens > pkv::kMaxTailPart)
      return fail(PKV_ERR_INVALID, "cascade plan: part_tokens must be a positive multiple of 16 and of block_size, "
                                   "at most 1024");
    if (plan->max_chunks <= 0 || plan->max_chunks > 65536 || plan->max_parts <= 0 || plan->max_parts > 65536)
      return fail(PKV_ERR_INVALID, "cascade plan: max_chunks and max_parts must be in [1, 65536]");
    if ((int64_t)num_seqs * num_heads * (plan->max_chunks + plan->max_parts) * head_size > ((int64_t)1 << 40))
      return fail(PKV_ERR_UNSUPPORTED, "cascade plan: workspace beyond 4 TiB");
  }
  // The cascade kernels: 16-bit queries over caches of the same type or
  // FP8, head sizes 64 and 128, GQA groups of at most 16, and V rows aligned
  // for 16-byte loads.  Other shapes take the one-pass decode below, whose
  // result is the same.
  const bool cascade = plan != nullptr && !rows && (q_dtype == PKV_BF16 || q_dtype == PKV_F16) &&
                       (cache_dtype == q_dtype || (fp8 && block_size >= 16)) &&
                       (head_size == 64 || head_size == 128) &&
                       num_heads / num_kv_heads <= 16 &&
                       aligned16(value_cache) && (vbs * cb) % 16 == 0 && (v_head_stride * cb) % 16 == 0;
  const pkv::DecodeWorkspace w = pkv::decode_workspace_layout(num_seqs, num_heads, head_size, parts);
  const pkv::CascadeWorkspace cw =
      plan != nullptr ? pkv::cascade_workspace_layout(num_seqs, num_heads, head_size, plan->max_chunks, plan->max_parts)
                      : pkv::CascadeWorkspace{0, 0, 0, 0, 0};
  if (cascade && (workspace == nullptr || workspace_bytes < cw.total))
    return fail(PKV_ERR_INVALID, "workspace is smaller than pkv_paged_attention_cascade_workspace_size()");
  if (use_scratch) {
    if (w.total > (size_t)PKV_NOALLOC_SCRATCH_BYTES)
      return fail(PKV_ERR_UNSUPPORTED, "pkv_paged_attention_noalloc needs " + std::to_string(w.total) +
                                           " bytes of workspace for these sizes, more than its static scratch of " +
                                           std::to_string((size_t)PKV_NOALLOC_SCRATCH_BYTES) + " bytes");
    const int sst = static_scratch(&workspace);
    if (sst != PKV_OK) return sst;
    workspace_bytes = PKV_NOALLOC_SCRATCH_BYTES;
  }
  if (workspace == nullptr || workspace_bytes < w.total)
    return fail(PKV_ERR_INVALID, "workspace is smaller than pkv_paged_attention_workspace_size()");
  if (!aligned16(workspace)) return fail(PKV_ERR_INVALID, "workspace must be 16-byte aligned");

  pkv::DecodeParams p;
  char* ws = static_cast<char*>(workspace);
  p.out = out;
  p.q = query;
  p.k_cache = key_cache;
  p.v_cache = value_cache;
  p.block_tables = block_tables;
  p.context_lens = context_lens;
  p.alibi = alibi_slopes;
  // The workspace starts with the partition kernel's arrival counters (zero
  // between calls), then the partition states.
  p.ws_ml = reinterpret_cast<float*>(ws + pkv::kCounterBytes);
  p.ws_o = reinterpret_cast<float*>(ws + pkv::kCounterBytes + w.ml_bytes);
  p.num_blocks = num_blocks;
  p.q_stride = q_stride;
  p.k_block_stride = kbs;
  p.k_head_stride = k_head_stride;
  p.v_block_stride = vbs;
  p.v_head_stride = v_head_stride;
  p.scale_log2 = scale * 1.4426950408889634f * (fp8 ? k_scale : 1.f);
  p.v_scale = fp8 ? v_scale : 1.f;
  p.num_seqs = num_seqs;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.group = num_heads / num_kv_heads;
  p.slices = (p.group + 15) / 16;
  p.units = num_kv_heads * p.slices;
  p.max_blocks_per_seq = max_num_blocks_per_seq;
  p.max_seq_len = max_seq_len;
  p.partition = ps;
  p.max_parts = parts;
  p.persistent = partition_size == 0 &&
                 max_seq_len <= (rows ? pkv::persist_rows_max_seq(head_size) : pkv::kPersistMaxSeq);
  p.rows = rows;
  p.block_size = block_size;
  // The paged layout's partition kernel merges its own partitions when a row
  // has at most kMergeGroup of them and the batch's counters fit the counter
  // region; otherwise (and for token rows) the merge kernel runs after it.
  p.counters = (!rows && parts <= pkv::kMergeGroup && (int64_t)num_seqs * p.units * 4 <= pkv::kCounterBytes)
                   ? reinterpret_cast<int32_t*>(ws)
                   : nullptr;
  p.k_rows_bytes = p.v_rows_bytes = 0;
  if (rows) {
    const int64_t total_rows = num_blocks * block_size;
    const int64_t k_span = ((total_rows - 1) * kbs + head_size) * 2;
    const int64_t v_span = ((total_rows - 1) * vbs + head_size) * 2;
    if (k_span > (int64_t)UINT32_MAX || v_span > (int64_t)UINT32_MAX)
      p.persistent = 0;  // 64-bit addressing: the partition kernel
    else {
      p.k_rows_bytes = (uint32_t)k_span;
      p.v_rows_bytes = (uint32_t)v_span;
    }
  }

  bool ok = true;
  hipError_t e = hipErrorInvalidValue;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  clear_pending_error();
  if (cascade) {
    pkv::CascadeParams c;
    c.prefix_lens = plan->prefix_lens;
    c.members = plan->members;
    c.tiles = reinterpret_cast<const int4*>(plan->tiles);
    c.parts = reinterpret_cast<const int2*>(plan->parts);
    char* cws = ws + pkv::kCounterBytes;
    c.ws_ml = reinterpret_cast<float*>(cws);
    c.ws_o = reinterpret_cast<float*>(cws + cw.ml_bytes);
    c.ws_tail_ml = reinterpret_cast<float*>(cws + cw.ml_bytes + cw.o_bytes);
    c.ws_tail_o = reinterpret_cast<float*>(cws + cw.ml_bytes + cw.o_bytes + cw.tail_ml_bytes);
    c.num_members = plan->num_members;
    c.num_tiles = plan->num_tiles;
    c.chunk = plan->chunk_tokens;
    c.max_chunks = plan->max_chunks;
    c.num_parts = plan->num_parts;
    c.part_tokens = plan->part_tokens;
    c.max_parts = plan->max_parts;
    if (q_dtype == PKV_BF16)
      e = fp8 ? pkv::launch_cascade_typed<pkv::BF16, pkv::FP8>(p, c, head_size, block_size, s, &ok)
              : pkv::launch_cascade_typed<pkv::BF16, pkv::BF16>(p, c, head_size, block_size, s, &ok);
    else
      e = fp8 ? pkv::launch_cascade_typed<pkv::F16, pkv::FP8>(p, c, head_size, block_size, s, &ok)
              : pkv::launch_cascade_typed<pkv::F16, pkv::F16>(p, c, head_size, block_size, s, &ok);
    if (ok) {
      if (e != hipSuccess) return hip_fail(e, "paged_attention_cascade launch");
      return PKV_OK;
    }
    ok = true;  // a shape the cascade kernels do not take: the one-pass decode
  }
  if (fp8) {
    if (q_dtype == PKV_BF16)
      e = pkv::launch_decode_typed<pkv::BF16, pkv::FP8>(p, head_size, block_size, s, &ok);
    else if (q_dtype == PKV_F16)
      e = pkv::launch_decode_typed<pkv::F16, pkv::FP8>(p, head_size, block_size, s, &ok);
    else
      e = pkv::launch_decode_typed<pkv::F32, pkv::FP8>(p, head_size, block_size, s, &ok);
  } else if (cache_dtype == PKV_F32)
    e = pkv::launch_decode_typed<pkv::F32, pkv::F32>(p, head_size, block_size, s, &ok);
  else if (q_dtype == PKV_BF16)
    e = pkv::launch_decode_typed<pkv::BF16, pkv::BF16>(p, head_size, block_size, s, &ok);
  else if (q_dtype == PKV_F16)
    e = pkv::launch_decode_typed<pkv::F16, pkv::F16>(p, head_size, block_size, s, &ok);
  else if (cache_dtype == PKV_BF16)
    e = pkv::launch_decode_typed<pkv::F32, pkv::BF16>(p, head_size, block_size, s, &ok);
  else
    e = pkv::launch_decode_typed<pkv::F32, pkv::F16>(p, head_size, block_size, s, &ok);
  if (!ok) return fail(PKV_ERR_UNSUPPORTED, "Unsupported head_size/block_size for paged_attention");
  if (e != hipSuccess) return hip_fail(e, "paged_attention launch");
  return PKV_OK;
}

}  // namespace

extern "C" {

int pkv_paged_attention(void* out, const void* query, const void* key_cache, const void* value_cache,
                        const int32_t* block_tables, const int32_t* context_lens, const float* alibi_slopes,
                        int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads, int32_t head_size,
                        int32_t block_size, int32_t max_num_blocks_per_seq, int32_t max_seq_len,
                        int64_t num_blocks, float scale, int64_t q_stride, int64_t k_block_stride,
                        int64_t k_head_stride, int64_t v_block_stride, int64_t v_head_stride, int32_t layout,
                        int32_t partition_size, void* workspace, size_t workspace_bytes, int32_t q_dtype,
                        int32_t cache_dtype, float k_scale, float v_scale, void* stream) {
  return paged_attention_impl(out, query, key_cache, value_cache, block_tables, context_lens, alibi_slopes, num_seqs,
                              num_heads, num_kv_heads, head_size, block_size, max_num_blocks_per_seq, max_seq_len,
                              num_blocks, scale, q_stride, k_block_stride, k_head_stride, v_block_stride,
                              v_head_stride, layout, partition_size, workspace, workspace_bytes, false, q_dtype,
                              cache_dtype, k_scale, v_scale, stream);
}

int pkv_paged_attention_noalloc(void* out, const void* query, const void* key_cache, const void* value_cache,
                                const int32_t* block_tables, const int32_t* context_lens,
                                const float* alibi_slopes, int32_t num_seqs, int32_t num_heads,
                                int32_t num_kv_heads, int32_t head_size, int32_t block_size,
                                int32_t max_num_blocks_per_seq, int32_t max_seq_len, int64_t num_blocks,
                                float scale, int64_t q_stride, int64_t k_block_stride, int64_t k_head_stride,
                                int64_t v_block_stride, int64_t v_head_stride, int32_t layout,
                                int32_t partition_size, int32_t q_dtype, int32_t cache_dtype, float k_scale,
                                float v_scale, void* stream) {
  return paged_attention_impl(out, query, key_cache, value_cache, block_tables, context_lens, alibi_slopes, num_seqs,
                              num_heads, num_kv_heads, head_size, block_size, max_num_blocks_per_seq, max_seq_len,
                              num_blocks, scale, q_stride, k_block_stride, k_head_stride, v_block_stride,
                              v_head_stride, layout, partition_size, nullptr, 0, true, q_dtype, cache_dtype,
                              k_scale, v_scale, stream);
}

int pkv_paged_attention_cascade(void* out, const void* query, const void* key_cache, const void* value_cache,
                                const int32_t* block_tables, const int32_t* context_lens, const float* alibi_slopes,
                                const pkv_cascade_plan* plan, int32_t num_seqs, int32_t num_heads,
                                int32_t num_kv_heads, int32_t head_size, int32_t block_size,
                                int32_t max_num_blocks_per_seq, int32_t max_seq_len, int64_t num_blocks, float scale,
                                int64_t q_stride, int64_t k_block_stride, int64_t k_head_stride,
                                int64_t v_block_stride, int64_t v_head_stride, void* workspace,
                                size_t workspace_bytes, int32_t q_dtype, int32_t cache_dtype, float k_scale,
                                float v_scale, void* stream) {
  if (plan == nullptr) return fail(PKV_ERR_INVALID, "cascade plan is null");
  return paged_attention_impl(out, query, key_cache, value_cache, block_tables, context_lens, alibi_slopes, num_seqs,
                              num_heads, num_kv_heads, head_size, block_size, max_num_blocks_per_seq, max_seq_len,
                              num_blocks, scale, q_stride, k_block_stride, k_head_stride, v_block_stride,
                              v_head_stride, PKV_LAYOUT_PAGED5D, 0, workspace, workspace_bytes, false, q_dtype,
                              cache_dtype, k_scale, v_scale, stream, plan);
}

int pkv_max_shared_memory_per_block(int32_t device_id, int64_t* out) {
  if (!out) return fail(PKV_ERR_INVALID, "null output pointer");
  int v = 0;
  const hipError_t e = hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device_id);
  if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
  *out = v;
  return PKV_OK;
}

int pkv_copy_blocks(void* const* src_planes, void* const* dst_planes, int32_t num_planes, int64_t src_blocks,
                    int64_t dst_blocks, int64_t block_bytes, const int64_t* block_mapping, int64_t num_pairs,
                    void* stream) {
  if (num_planes < 0 || num_pairs < 0 || block_bytes < 0)
    return fail(PKV_ERR_INVALID, "num_planes, num_pairs and block_bytes must be non-negative");
  if (num_planes == 0 || num_pairs == 0 || block_bytes == 0) return PKV_OK;
  if (src_blocks <= 0 || dst_blocks <= 0)
    return fail(PKV_ERR_INVALID, "src and dst must have a leading block dimension");
  if (!src_planes || !dst_planes || !block_mapping) return fail(PKV_ERR_INVALID, "null buffer");
  bool aligned = block_bytes % 16 == 0;
  for (int32_t i = 0; i < num_planes; ++i) {
    if (!src_planes[i] || !dst_planes[i]) return fail(PKV_ERR_INVALID, "null buffer");
    aligned = aligned && aligned16(src_planes[i]) && aligned16(dst_planes[i]);
  }
  const int64_t max_pairs = pkv::copy_blocks_max_grid_pairs(block_bytes, aligned);
  pkv::BlockCopyParams p;
  p.src_blocks = src_blocks;
  p.dst_blocks = dst_blocks;
  p.block_bytes = block_bytes;
  clear_pending_error();
  for (int32_t plane0 = 0; plane0 < num_planes; plane0 += pkv::kMaxCopyPlanes) {
    p.num_planes = std::min<int32_t>(pkv::kMaxCopyPlanes, num_planes - plane0);
    for (int32_t i = 0; i < p.num_planes; ++i) {
      p.src[i] = static_cast<const char*>(src_planes[plane0 + i]);
      p.dst[i] = static_cast<char*>(dst_planes[plane0 + i]);
    }
    for (int64_t pair0 = 0; pair0 < num_pairs; pair0 += max_pairs) {
      p.mapping = block_mapping + 2 * pair0;
      p.num_pairs = std::min<int64_t>(max_pairs, num_pairs - pair0);
      const hipError_t e = pkv::launch_copy_blocks(p, aligned, static_cast<hipStream_t>(stream));
      if (e != hipSuccess) return hip_fail(e, "copy_blocks launch");
    }
  }
  return PKV_OK;
}

int pkv_convert_fp8(void* dst, const void* src, int64_t num_elements, float scale, int32_t src_dtype,
                    int32_t dst_dtype, void* stream) {
  if (num_elements < 0) return fail(PKV_ERR_INVALID, "num_elements must be non-negative");
  const bool types_ok = src_dtype >= PKV_F32 && src_dtype <= PKV_FP8_E4M3 && dst_dtype >= PKV_F32 &&
                        dst_dtype <= PKV_FP8_E4M3;
  if (!types_ok) return fail(PKV_ERR_UNSUPPORTED, "Unsupported dtype pair for convert_fp8");
  if (num_elements == 0) return PKV_OK;
  if (!dst || !src) return fail(PKV_ERR_INVALID, "null buffer");
  const int sb = src_dtype == PKV_FP8_E4M3 ? 1 : elem_bytes(src_dtype);
  const int db = dst_dtype == PKV_FP8_E4M3 ? 1 : elem_bytes(dst_dtype);
  if ((reinterpret_cast<uintptr_t>(src) % sb) != 0 || (reinterpret_cast<uintptr_t>(dst) % db) != 0)
    return fail(PKV_ERR_INVALID, "buffers are not aligned to their element size");
  if (sb != db || src != dst) {
    const uintptr_t s0 = reinterpret_cast<uintptr_t>(src), s1 = s0 + (uintptr_t)num_elements * sb;
    const uintptr_t d0 = reinterpret_cast<uintptr_t>(dst), d1 = d0 + (uintptr_t)num_elements * db;
    if (s0 < d1 && d0 < s1) return fail(PKV_ERR_INVALID, "dst and src overlap");
  }
  clear_pending_error();
  const hipError_t e = pkv::launch_convert_fp8(dst, src, num_elements, scale, src_dtype, dst_dtype,
                                               static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "convert_fp8 launch");
  return PKV_OK;
}

int pkv_get_device_attribute(int32_t attribute, int32_t device_id, int64_t* out) {
  if (!out) return fail(PKV_ERR_INVALID, "null output pointer");
  int v = 0;
  const hipError_t e = hipDeviceGetAttribute(&v, static_cast<hipDeviceAttribute_t>(attribute), device_id);
  if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
  *out = v;
  return PKV_OK;
}

}  // extern "C"
