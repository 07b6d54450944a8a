// gqa_abi.hip — extern "C" entry points declared in include/gqa_attn.h.
//
// Argument validation mirrors the asserts of reference
// gqa_kernels/dispatch.py:30-33 (divisible heads, head_dim in {64, 128}) plus
// the layout requirements of the vectorised kernels (unit last-dim stride,
// 16-byte aligned rows).  Nothing here allocates device memory.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "../../include/gqa_attn.h"
#include "gqa_params.hpp"

namespace {

using gqa::Dims;
using gqa::TensorRef;

// 7: gqa_paged_split_first_launch limits a chunk over pages of < 64 keys to
// GQA_PAGED_CHUNK_PAGES pages (GQA_E_SPLITS beyond); a sequence without keys
// gives zero rows on every path.  8: gqa_split_noalloc_launch.
// 9: gqa_split_launch (first pass and combine in one call).
// 10: gqa_fwd_split_counters_count adds the persistent single pass's
// scheduling counters (also for n_split = 0); gqa_fwd_split_launch with
// counters schedules the work items across the XCDs dynamically.
// 11: gqa_fwd_chunks_launch (single pass over key chunks + split combine).
// 12: gqa_paged_fwd_chunks_launch (the same over a paged cache).
// 13: gqa_paged_fwd_split_launch (the paged single pass with split blocks).
constexpr int kAbiVersion = 13;

int check_dims(int B, int Hq, int Hkv, int Sq, int Skv, int D, int dtype) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Sq < 0 || Skv < 0) return GQA_E_SHAPE;
  if (Hq % Hkv != 0) return GQA_E_SHAPE;
  if (D != 64 && D != 128) return GQA_E_HEAD_DIM;
  if (dtype != GQA_DTYPE_BF16 && dtype != GQA_DTYPE_FP16) return GQA_E_DTYPE;
  return GQA_OK;
}

// Rows must start on 16 bytes: pointer and the three outer strides (in
// 2-byte elements) multiples of 8; the last-dim stride must be 1.
int check_tensor(const void* ptr, const int64_t st[4]) {
  if (ptr == nullptr || st == nullptr) return GQA_E_NULL;
  if (st[3] != 1) return GQA_E_STRIDE;
  if ((reinterpret_cast<uintptr_t>(ptr) & 15u) != 0) return GQA_E_STRIDE;
  for (int i = 0; i < 3; ++i)
    if (st[i] % 8 != 0) return GQA_E_STRIDE;
  return GQA_OK;
}

// The single-pass kernel addresses one (batch, kv head)'s K or V rows with
// 32-bit byte offsets, up to two 64-key tiles past the last row.
bool rows_fit_32bit(int seq_kv, const int64_t st[4]) {
  return ((int64_t)seq_kv + 192) * st[2] * 2 < ((int64_t)1 << 31);
}

TensorRef ref(const void* ptr, const int64_t st[4]) { return TensorRef{ptr, st[0], st[1], st[2]}; }

// A paged cache (num_blocks, block_size, heads, D) as the kernels address it:
// sb = block stride, sh = head stride, ss = slot stride (the slot plays the
// role of the sequence position).
TensorRef cache_ref(const void* ptr, const int64_t st[4]) { return TensorRef{ptr, st[0], st[2], st[1]}; }

int to_code(hipError_t e) { return e == hipSuccess ? GQA_OK : static_cast<int>(e); }

}  // namespace

extern "C" {

int gqa_abi_version(void) { return kAbiVersion; }

const char* gqa_strerror(int code) {
  switch (code) {
    case GQA_OK: return "success";
    case GQA_E_SHAPE: return "invalid shape: sizes must be non-negative and num_heads divisible by num_kv_heads";
    case GQA_E_HEAD_DIM: return "unsupported head_dim (supported: 64, 128)";
    case GQA_E_DTYPE: return "unsupported dtype (supported: bf16, fp16)";
    case GQA_E_STRIDE:
      return "unsupported layout: last dim must be contiguous, rows 16-byte aligned, and one head's K/V rows "
             "within 2 GiB";
    case GQA_E_SPLITS:
      return "splits out of range [1, GQA_MAX_SPLITS], or a paged chunk spans more than "
             "GQA_PAGED_CHUNK_PAGES pages of under 64 keys";
    case GQA_E_GROUP: return "group size (num_heads / num_kv_heads) larger than 256";
    case GQA_E_NULL: return "null pointer argument";
    case GQA_E_BLOCK:
      return "paged cache: block_size must be a power of two in [1, GQA_MAX_BLOCK_SIZE] "
             "(gqa_paged_fwd_launch: >= 512 / head_dim) and table_stride * block_size must cover "
             "max_seq_len";
    case GQA_E_SCRATCH:
      return "gqa_split_noalloc_launch: the split partials exceed its fixed buffer "
             "(GQA_NOALLOC_SCRATCH_BYTES, 16 MiB); use fewer splits or gqa_split_first_launch with a "
             "caller workspace";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown error";
}

int gqa_device_cu_count(int device) {
  int n = 0;
  hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
  if (e != hipSuccess) return -static_cast<int>(e);
  return n;
}

size_t gqa_split_workspace_bytes(int batch, int num_heads, int seq_q, int head_dim, int splits) {
  if (batch <= 0 || num_heads <= 0 || seq_q <= 0 || head_dim <= 0 || splits <= 0) return 0;
  const size_t rows = (size_t)batch * num_heads * seq_q * splits;
  return rows * ((size_t)head_dim + 2) * sizeof(float);
}

}  // extern "C"

namespace {

int fwd_impl(const void* q, const int64_t q_stride[4], const void* k, const int64_t k_stride[4], const void* v,
             const int64_t v_stride[4], void* o, const int64_t o_stride[4], float* lse, int batch, int num_heads,
             int num_kv_heads, int seq_q, int seq_kv, int head_dim, float scale_log2, int causal, int dtype,
             void* stream, int n_split = 0, float* part_ws = nullptr, int* part_cnt = nullptr) {
  int rc = check_dims(batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, dtype);
  if (rc) return rc;
  const int G = num_heads / num_kv_heads;
  if (G > gqa::kFwdRows) return GQA_E_GROUP;
  const int block_m = gqa::kFwdRows / G;
  const int n_mblk = (seq_q + block_m - 1) / block_m;
  if (n_split < 0 || n_split > n_mblk) return GQA_E_SPLITS;
  if (batch == 0 || seq_q == 0) return GQA_OK;
  if (n_split > 0) {
    if (part_ws == nullptr || part_cnt == nullptr) return GQA_E_NULL;
    if ((reinterpret_cast<uintptr_t>(part_ws) & 15u) != 0) return GQA_E_STRIDE;
  }
  if ((reinterpret_cast<uintptr_t>(part_cnt) & 3u) != 0) return GQA_E_STRIDE;
  if ((rc = check_tensor(q, q_stride)) || (rc = check_tensor(o, o_stride))) return rc;
  if (seq_kv > 0 && ((rc = check_tensor(k, k_stride)) || (rc = check_tensor(v, v_stride)))) return rc;
  if (seq_kv > 0 && (!rows_fit_32bit(seq_kv, k_stride) || !rows_fit_32bit(seq_kv, v_stride))) return GQA_E_STRIDE;

  gqa::FwdParams p{};
  p.q = ref(q, q_stride);
  p.k = ref(k, k_stride);
  p.v = ref(v, v_stride);
  p.o = ref(o, o_stride);
  p.dm = Dims{batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, G, scale_log2, causal ? 1 : 0};
  p.block_m = block_m;
  p.n_mblk = n_mblk;
  p.lse = lse;
  p.n_split = n_split;
  p.part_ws = part_ws;
  p.part_cnt = part_cnt;
  // The scheduling counters follow the split blocks' counters.
  p.sched = part_cnt != nullptr ? part_cnt + (size_t)batch * num_kv_heads * n_split : nullptr;
  return to_code(gqa::launch_fwd(p, dtype, static_cast<hipStream_t>(stream)));
}

// Variable query lengths: q_start and q_len both NULL (uniform seq_q) or
// both 4-byte aligned device arrays.
int check_varlen(const int* q_start, const int* q_len) {
  if ((q_start == nullptr) != (q_len == nullptr)) return GQA_E_NULL;
  if (((reinterpret_cast<uintptr_t>(q_start) | reinterpret_cast<uintptr_t>(q_len)) & 3u) != 0) return GQA_E_STRIDE;
  return GQA_OK;
}

int check_lse(const float* lse) {
  if (lse == nullptr) return GQA_E_NULL;
  return (reinterpret_cast<uintptr_t>(lse) & 3u) != 0 ? GQA_E_STRIDE : GQA_OK;
}

int paged_fwd_impl(const void* q, const int64_t q_stride[4], const void* k_cache,
                   const int64_t k_cache_stride[4], const void* v_cache, const int64_t v_cache_stride[4],
                   const int* block_table, int table_stride, const int* seq_lens, const int* q_start,
                   const int* q_len, int block_size, int max_seq_len, void* o, const int64_t o_stride[4],
                   float* lse, float* workspace, int kv_splits, int batch, int num_heads, int num_kv_heads,
                   int seq_q, int head_dim, float scale_log2, int causal, int dtype, void* stream,
                   int n_split = 0, float* part_ws = nullptr, int* part_cnt = nullptr);

}  // namespace

extern "C" {

int gqa_fwd_launch(const void* q, const int64_t q_stride[4], const void* k, const int64_t k_stride[4],
                   const void* v, const int64_t v_stride[4], void* o, const int64_t o_stride[4], int batch,
                   int num_heads, int num_kv_heads, int seq_q, int seq_kv, int head_dim, float scale_log2,
                   int causal, int dtype, void* stream) {
  return fwd_impl(q, q_stride, k, k_stride, v, v_stride, o, o_stride, nullptr, batch, num_heads, num_kv_heads,
                  seq_q, seq_kv, head_dim, scale_log2, causal, dtype, stream);
}

int gqa_fwd_lse_launch(const void* q, const int64_t q_stride[4], const void* k, const int64_t k_stride[4],
                       const void* v, const int64_t v_stride[4], void* o, const int64_t o_stride[4], float* lse,
                       int batch, int num_heads, int num_kv_heads, int seq_q, int seq_kv, int head_dim,
                       float scale_log2, int causal, int dtype, void* stream) {
  const int rc = check_lse(lse);
  if (rc && batch > 0 && seq_q > 0) return rc;
  return fwd_impl(q, q_stride, k, k_stride, v, v_stride, o, o_stride, lse, batch, num_heads, num_kv_heads,
                  seq_q, seq_kv, head_dim, scale_log2, causal, dtype, stream);
}

size_t gqa_fwd_split_workspace_bytes(int batch, int num_kv_heads, int head_dim, int n_split) {
  if (batch <= 0 || num_kv_heads <= 0 || n_split <= 0 || (head_dim != 64 && head_dim != 128)) return 0;
  return (size_t)batch * num_kv_heads * n_split * 2 * gqa::kFwdPartFloats(head_dim) * sizeof(float);
}

size_t gqa_fwd_split_counters_count(int batch, int num_kv_heads, int n_split) {
  if (batch <= 0 || num_kv_heads <= 0 || n_split < 0) return 0;
  return (size_t)batch * num_kv_heads * n_split + gqa::kFwdSchedCounters;
}

int gqa_fwd_split_launch(const void* q, const int64_t q_stride[4], const void* k, const int64_t k_stride[4],
                         const void* v, const int64_t v_stride[4], void* o, const int64_t o_stride[4], float* lse,
                         float* workspace, int* counters, int n_split, int batch, int num_heads, int num_kv_heads,
                         int seq_q, int seq_kv, int head_dim, float scale_log2, int causal, int dtype,
                         void* stream) {
  if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return GQA_E_STRIDE;
  return fwd_impl(q, q_stride, k, k_stride, v, v_stride, o, o_stride, lse, batch, num_heads, num_kv_heads, seq_q,
                  seq_kv, head_dim, scale_log2, causal, dtype, stream, n_split, workspace, counters);
}

int gqa_split_first_launch(const void* q, const int64_t q_stride[4], const void* k, const int64_t k_stride[4],
                           const void* v, const int64_t v_stride[4], float* workspace, int splits, int batch,
                           int num_heads, int num_kv_heads, int seq_q, int seq_kv, int head_dim,
                           float scale_log2, int causal, int dtype, void* stream) {
  int rc = check_dims(batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, dtype);
  if (rc) return rc;
  if (splits < 1 || splits > GQA_MAX_SPLITS) return GQA_E_SPLITS;
  if (batch == 0 || seq_q == 0) return GQA_OK;
  if (workspace == nullptr) return GQA_E_NULL;
  if ((reinterpret_cast<uintptr_t>(workspace) & 15u) != 0) return GQA_E_STRIDE;
  if ((rc = check_tensor(q, q_stride))) return rc;
  if (seq_kv > 0 && ((rc = check_tensor(k, k_stride)) || (rc = check_tensor(v, v_stride)))) return rc;

  const int G = num_heads / num_kv_heads;
  gqa::SplitParams p{};
  p.q = ref(q, q_stride);
  p.k = ref(k, k_stride);
  p.v = ref(v, v_stride);
  p.dm = Dims{batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, G, scale_log2, causal ? 1 : 0};
  const size_t rows = (size_t)batch * num_heads * seq_q * splits;
  p.ws_acc = workspace;
  p.ws_m = workspace + rows * head_dim;
  p.ws_l = p.ws_m + rows;
  p.splits = splits;
  p.chunk = (seq_kv + splits - 1) / splits;
  p.n_rblk = (G * seq_q + 31) / 32;
  p.rotate = p.k.ss == head_dim && p.v.ss == head_dim;
  p.counters = nullptr;
  p.o = TensorRef{nullptr, 0, 0, 0};
  p.lse = nullptr;
  return to_code(gqa::launch_split_first(p, dtype, static_cast<hipStream_t>(stream)));
}

int gqa_paged_split_first_launch(const void* q, const int64_t q_stride[4], const void* k_cache,
                                 const int64_t k_cache_stride[4], const void* v_cache,
                                 const int64_t v_cache_stride[4], const int* block_table, int table_stride,
                                 const int* seq_lens, const int* q_start, const int* q_len, int block_size,
                                 int max_seq_len, float* workspace, int splits, int batch, int num_heads,
                                 int num_kv_heads, int seq_q, int head_dim, float scale_log2, int causal, int dtype,
                                 void* stream) {
  int rc = check_dims(batch, num_heads, num_kv_heads, seq_q, max_seq_len, head_dim, dtype);
  if (rc) return rc;
  if (block_size < 1 || block_size > GQA_MAX_BLOCK_SIZE || (block_size & (block_size - 1)) != 0)
    return GQA_E_BLOCK;
  if (table_stride < 0 || (int64_t)table_stride * block_size < (int64_t)max_seq_len) return GQA_E_BLOCK;
  if (splits < 1 || splits > GQA_MAX_SPLITS) return GQA_E_SPLITS;
  if (batch == 0 || seq_q == 0) return GQA_OK;
  if (workspace == nullptr || seq_lens == nullptr) return GQA_E_NULL;
  if ((reinterpret_cast<uintptr_t>(workspace) & 15u) != 0 || (reinterpret_cast<uintptr_t>(seq_lens) & 3u) != 0)
    return GQA_E_STRIDE;
  if ((rc = check_varlen(q_start, q_len))) return rc;
  if ((rc = check_tensor(q, q_stride))) return rc;
  if (max_seq_len > 0) {
    if (block_table == nullptr) return GQA_E_NULL;
    if ((reinterpret_cast<uintptr_t>(block_table) & 3u) != 0) return GQA_E_STRIDE;
    if ((rc = check_tensor(k_cache, k_cache_stride)) || (rc = check_tensor(v_cache, v_cache_stride))) return rc;
  }

  const int G = num_heads / num_kv_heads;
  gqa::SplitParams p{};
  p.q = ref(q, q_stride);
  p.k = cache_ref(k_cache, k_cache_stride);
  p.v = cache_ref(v_cache, v_cache_stride);
  p.dm = Dims{batch, num_heads, num_kv_heads, seq_q, max_seq_len, head_dim, G, scale_log2, causal ? 1 : 0};
  const size_t rows = (size_t)batch * num_heads * seq_q * splits;
  p.ws_acc = workspace;
  p.ws_m = workspace + rows * head_dim;
  p.ws_l = p.ws_m + rows;
  p.splits = splits;
  // Chunks start on 64-key boundaries, so with pages of 64 keys or more
  // every full 64-key sub-tile is one strided run inside one page.
  p.chunk = ((max_seq_len + splits - 1) / splits + 63) & ~63;
  p.n_rblk = (G * seq_q + 31) / 32;
  p.counters = nullptr;
  p.o = TensorRef{nullptr, 0, 0, 0};
  p.lse = nullptr;
  p.block_table = block_table;
  p.seq_lens = seq_lens;
  p.table_stride = table_stride;
  int shift = 0;
  while ((1 << shift) < block_size) ++shift;
  p.block_shift = shift;
  // Pages under 64 keys: each workgroup stages its chunk's table slice in LDS.
  static_assert(gqa::kPagedTableMax == GQA_PAGED_CHUNK_PAGES, "table slice size");
  if (shift < 6 && (p.chunk >> shift) > gqa::kPagedTableMax) return GQA_E_SPLITS;
  p.rotate = p.k.ss == head_dim && p.v.ss == head_dim;
  p.q_start = q_start;
  p.q_len = q_len;
  return to_code(gqa::launch_paged_split_first(p, dtype, static_cast<hipStream_t>(stream)));
}

int gqa_paged_fwd_launch(const void* q, const int64_t q_stride[4], const void* k_cache,
                         const int64_t k_cache_stride[4], const void* v_cache, const int64_t v_cache_stride[4],
                         const int* block_table, int table_stride, const int* seq_lens, const int* q_start,
                         const int* q_len, int block_size, int max_seq_len, void* o, const int64_t o_stride[4],
                         float* lse, int batch,
                         int num_heads, int num_kv_heads, int seq_q, int head_dim, float scale_log2, int causal,
                         int dtype, void* stream) {
  return paged_fwd_impl(q, q_stride, k_cache, k_cache_stride, v_cache, v_cache_stride, block_table, table_stride,
                        seq_lens, q_start, q_len, block_size, max_seq_len, o, o_stride, lse, nullptr, 0, batch,
                        num_heads, num_kv_heads, seq_q, head_dim, scale_log2, causal, dtype, stream);
}

int gqa_paged_fwd_chunks_launch(const void* q, const int64_t q_stride[4], const void* k_cache,
                                const int64_t k_cache_stride[4], const void* v_cache,
                                const int64_t v_cache_stride[4], const int* block_table, int table_stride,
                                const int* seq_lens, const int* q_start, const int* q_len, int block_size,
                                int max_seq_len, void* o, const int64_t o_stride[4], float* lse, float* workspace,
                                int kv_splits, int batch, int num_heads, int num_kv_heads, int seq_q, int head_dim,
                                float scale_log2, int causal, int dtype, void* stream) {
  if (kv_splits < 1 || kv_splits > GQA_MAX_SPLITS) return GQA_E_SPLITS;
  return paged_fwd_impl(q, q_stride, k_cache, k_cache_stride, v_cache, v_cache_stride, block_table, table_stride,
                        seq_lens, q_start, q_len, block_size, max_seq_len, o, o_stride, lse, workspace, kv_splits,
                        batch, num_heads, num_kv_heads, seq_q, head_dim, scale_log2, causal, dtype, stream);
}

int gqa_paged_fwd_split_launch(const void* q, const int64_t q_stride[4], const void* k_cache,
                               const int64_t k_cache_stride[4], const void* v_cache,
                               const int64_t v_cache_stride[4], const int* block_table, int table_stride,
                               const int* seq_lens, const int* q_start, const int* q_len, int block_size,
                               int max_seq_len, void* o, const int64_t o_stride[4], float* lse, float* workspace,
                               int* counters, int n_split, int batch, int num_heads, int num_kv_heads, int seq_q,
                               int head_dim, float scale_log2, int causal, int dtype, void* stream) {
  return paged_fwd_impl(q, q_stride, k_cache, k_cache_stride, v_cache, v_cache_stride, block_table, table_stride,
                        seq_lens, q_start, q_len, block_size, max_seq_len, o, o_stride, lse, nullptr, 0, batch,
                        num_heads, num_kv_heads, seq_q, head_dim, scale_log2, causal, dtype, stream, n_split,
                        workspace, counters);
}

int gqa_paged_cache_write_launch(const void* k, const int64_t k_stride[3], const void* v,
                                 const int64_t v_stride[3], void* k_cache, const int64_t k_cache_stride[4],
                                 void* v_cache, const int64_t v_cache_stride[4], const int64_t* slot_mapping,
                                 int num_tokens, int num_kv_heads, int head_dim, int block_size, int dtype,
                                 void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0) return GQA_E_SHAPE;
  if (head_dim != 64 && head_dim != 128) return GQA_E_HEAD_DIM;
  if (dtype != GQA_DTYPE_BF16 && dtype != GQA_DTYPE_FP16) return GQA_E_DTYPE;
  if (block_size < 1 || block_size > GQA_MAX_BLOCK_SIZE || (block_size & (block_size - 1)) != 0)
    return GQA_E_BLOCK;
  if (num_tokens == 0) return GQA_OK;
  if (slot_mapping == nullptr || k == nullptr || v == nullptr || k_stride == nullptr || v_stride == nullptr)
    return GQA_E_NULL;
  if ((reinterpret_cast<uintptr_t>(slot_mapping) & 7u) != 0) return GQA_E_STRIDE;
  for (const int64_t* st : {k_stride, v_stride})
    if (st[2] != 1 || st[0] % 8 != 0 || st[1] % 8 != 0) return GQA_E_STRIDE;
  if (((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15u) != 0) return GQA_E_STRIDE;
  int rc;
  if ((rc = check_tensor(k_cache, k_cache_stride)) || (rc = check_tensor(v_cache, v_cache_stride))) return rc;

  gqa::CacheWriteParams p{};
  p.k = k;
  p.v = v;
  p.k_st = k_stride[0];
  p.k_sh = k_stride[1];
  p.v_st = v_stride[0];
  p.v_sh = v_stride[1];
  p.kc = cache_ref(k_cache, k_cache_stride);
  p.vc = cache_ref(v_cache, v_cache_stride);
  p.slots = slot_mapping;
  p.n_tokens = num_tokens;
  p.Hkv = num_kv_heads;
  p.D = head_dim;
  int shift = 0;
  while ((1 << shift) < block_size) ++shift;
  p.block_shift = shift;
  p.elem_bytes = 2;
  return to_code(gqa::launch_paged_cache_write(p, static_cast<hipStream_t>(stream)));
}

size_t gqa_split_counters_count(int batch, int num_heads, int num_kv_heads, int seq_q) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || seq_q <= 0 || num_heads % num_kv_heads) return 0;
  const size_t G = (size_t)(num_heads / num_kv_heads);
  return (size_t)batch * num_kv_heads * ((G * seq_q + 31) / 32);
}

}  // extern "C"

namespace {

int fused_impl(const void* q, const int64_t q_stride[4], const void* k, const int64_t k_stride[4],
               const void* v, const int64_t v_stride[4], void* o, const int64_t o_stride[4], float* lse,
               float* workspace, int* counters, int splits, int batch, int num_heads, int num_kv_heads,
               int seq_q, int seq_kv, int head_dim, float scale_log2, int causal, int dtype, void* stream) {
  int rc = check_dims(batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, dtype);
  if (rc) return rc;
  if (splits < 1 || splits > GQA_MAX_SPLITS) return GQA_E_SPLITS;
  if (batch == 0 || seq_q == 0) return GQA_OK;
  if (workspace == nullptr || counters == nullptr) return GQA_E_NULL;
  if ((int64_t)std::min(32, (num_heads / num_kv_heads) * seq_q) * splits > gqa::kFusedMaxRowSplitsHost)
    return GQA_E_SPLITS;
  // The combine reads the partial accumulators at 32-bit byte offsets.
  if ((uint64_t)batch * num_heads * seq_q * splits * head_dim * 4u > 0xFFFFFFF0ull) return GQA_E_SPLITS;
  if ((reinterpret_cast<uintptr_t>(workspace) & 15u) != 0 || (reinterpret_cast<uintptr_t>(counters) & 3u) != 0)
    return GQA_E_STRIDE;
  if ((rc = check_tensor(q, q_stride)) || (rc = check_tensor(o, o_stride))) return rc;
  if (seq_kv > 0 && ((rc = check_tensor(k, k_stride)) || (rc = check_tensor(v, v_stride)))) return rc;

  const int G = num_heads / num_kv_heads;
  gqa::SplitParams p{};
  p.q = ref(q, q_stride);
  p.k = ref(k, k_stride);
  p.v = ref(v, v_stride);
  p.dm = Dims{batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, G, scale_log2, causal ? 1 : 0};
  const size_t rows = (size_t)batch * num_heads * seq_q * splits;
  p.ws_acc = workspace;
  p.ws_m = workspace + rows * head_dim;
  p.ws_l = p.ws_m + rows;
  p.splits = splits;
  p.chunk = (seq_kv + splits - 1) / splits;
  p.n_rblk = (G * seq_q + 31) / 32;
  p.rotate = p.k.ss == head_dim && p.v.ss == head_dim;
  p.counters = counters;
  p.o = ref(o, o_stride);
  p.lse = lse;
  return to_code(gqa::launch_split_first(p, dtype, static_cast<hipStream_t>(stream)));
}

int reduce_impl(const float* workspace, int splits, void* o, const int64_t o_stride[4], float* lse, int batch,
                int num_heads, int seq_q, int head_dim, int dtype, void* stream, const int* q_start = nullptr,
                const int* q_len = nullptr);

}  // namespace

extern "C" {

int gqa_split_fused_launch(const void* q, const int64_t q_stride[4], const void* k, const int64_t k_stride[4],
                           const void* v, const int64_t v_stride[4], void* o, const int64_t o_stride[4],
                           float* workspace, int* counters, int splits, int batch, int num_heads,
                           int num_kv_heads, int seq_q, int seq_kv, int head_dim, float scale_log2, int causal,
                           int dtype, void* stream) {
  return fused_impl(q, q_stride, k, k_stride, v, v_stride, o, o_stride, nullptr, workspace, counters, splits,
                    batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, scale_log2, causal, dtype, stream);
}

int gqa_split_fused_lse_launch(const void* q, const int64_t q_stride[4], const void* k,
                               const int64_t k_stride[4], const void* v, const int64_t v_stride[4], void* o,
                               const int64_t o_stride[4], float* lse, float* workspace, int* counters, int splits,
                               int batch, int num_heads, int num_kv_heads, int seq_q, int seq_kv, int head_dim,
                               float scale_log2, int causal, int dtype, void* stream) {
  const int rc = check_lse(lse);
  if (rc && batch > 0 && seq_q > 0) return rc;
  return fused_impl(q, q_stride, k, k_stride, v, v_stride, o, o_stride, lse, workspace, counters, splits, batch,
                    num_heads, num_kv_heads, seq_q, seq_kv, head_dim, scale_log2, causal, dtype, stream);
}

int gqa_split_launch(const void* q, const int64_t q_stride[4], const void* k, const int64_t k_stride[4],
                     const void* v, const int64_t v_stride[4], void* o, const int64_t o_stride[4], float* lse,
                     float* workspace, int splits, int batch, int num_heads, int num_kv_heads, int seq_q,
                     int seq_kv, int head_dim, float scale_log2, int causal, int dtype, void* stream) {
  int rc = check_dims(batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, dtype);
  if (rc) return rc;
  if (splits < 1 || splits > GQA_MAX_SPLITS) return GQA_E_SPLITS;
  if (batch == 0 || seq_q == 0) return GQA_OK;
  if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return GQA_E_STRIDE;
  // o is checked before the first pass is enqueued (q, k, v and the
  // workspace by the first pass).
  if ((rc = check_tensor(o, o_stride))) return rc;
  rc = gqa_split_first_launch(q, q_stride, k, k_stride, v, v_stride, workspace, splits, batch, num_heads,
                              num_kv_heads, seq_q, seq_kv, head_dim, scale_log2, causal, dtype, stream);
  if (rc) return rc;
  return reduce_impl(workspace, splits, o, o_stride, lse, batch, num_heads, seq_q, head_dim, dtype, stream);
}

int gqa_split_reduce_launch(const float* workspace, int splits, void* o, const int64_t o_stride[4], int batch,
                            int num_heads, int seq_q, int head_dim, int dtype, void* stream) {
  return reduce_impl(workspace, splits, o, o_stride, nullptr, batch, num_heads, seq_q, head_dim, dtype, stream);
}

int gqa_split_reduce_lse_launch(const float* workspace, int splits, void* o, const int64_t o_stride[4],
                                float* lse, int batch, int num_heads, int seq_q, int head_dim, int dtype,
                                void* stream) {
  const int rc = check_lse(lse);
  if (rc && batch > 0 && seq_q > 0) return rc;
  return reduce_impl(workspace, splits, o, o_stride, lse, batch, num_heads, seq_q, head_dim, dtype, stream);
}

int gqa_fwd_chunks_launch(const void* q, const int64_t q_stride[4], const void* k, const int64_t k_stride[4],
                          const void* v, const int64_t v_stride[4], void* o, const int64_t o_stride[4], float* lse,
                          float* workspace, int* counters, int kv_splits, int batch, int num_heads,
                          int num_kv_heads, int seq_q, int seq_kv, int head_dim, float scale_log2, int causal,
                          int dtype, void* stream) {
  int rc = check_dims(batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, dtype);
  if (rc) return rc;
  const int G = num_heads / num_kv_heads;
  if (G > gqa::kFwdRows) return GQA_E_GROUP;
  if (kv_splits < 1 || kv_splits > GQA_MAX_SPLITS) return GQA_E_SPLITS;
  if (batch == 0 || seq_q == 0) return GQA_OK;
  if (workspace == nullptr) return GQA_E_NULL;
  if ((reinterpret_cast<uintptr_t>(workspace) & 15u) != 0 || (reinterpret_cast<uintptr_t>(counters) & 3u) != 0)
    return GQA_E_STRIDE;
  if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return GQA_E_STRIDE;
  if ((rc = check_tensor(q, q_stride)) || (rc = check_tensor(o, o_stride))) return rc;
  if (seq_kv > 0 && ((rc = check_tensor(k, k_stride)) || (rc = check_tensor(v, v_stride)))) return rc;
  if (seq_kv > 0 && (!rows_fit_32bit(seq_kv, k_stride) || !rows_fit_32bit(seq_kv, v_stride))) return GQA_E_STRIDE;

  gqa::FwdParams p{};
  p.q = ref(q, q_stride);
  p.k = ref(k, k_stride);
  p.v = ref(v, v_stride);
  p.o = ref(o, o_stride);
  p.dm = Dims{batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, G, scale_log2, causal ? 1 : 0};
  p.block_m = gqa::kFwdRows / G;
  p.n_mblk = (seq_q + p.block_m - 1) / p.block_m;
  p.lse = nullptr;  // written by the combine
  p.sched = counters;
  const int tiles = (seq_kv + gqa::kFwdTileKeys - 1) / gqa::kFwdTileKeys;
  p.kv_splits = kv_splits;
  p.kv_chunk_tiles = std::max((tiles + kv_splits - 1) / kv_splits, 1);
  const size_t rows = (size_t)batch * num_heads * seq_q * kv_splits;
  p.ws_acc = workspace;
  p.ws_m = workspace + rows * head_dim;
  p.ws_l = p.ws_m + rows;
  rc = to_code(gqa::launch_fwd(p, dtype, static_cast<hipStream_t>(stream)));
  if (rc) return rc;
  return reduce_impl(workspace, kv_splits, o, o_stride, lse, batch, num_heads, seq_q, head_dim, dtype, stream);
}

int gqa_split_reduce_varlen_launch(const float* workspace, int splits, void* o, const int64_t o_stride[4],
                                   float* lse, const int* q_start, const int* q_len, int batch, int num_heads,
                                   int seq_q, int head_dim, int dtype, void* stream) {
  if (batch > 0 && seq_q > 0) {
    int rc = check_varlen(q_start, q_len);
    if (rc) return rc;
    if (q_start == nullptr) return GQA_E_NULL;
    if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return GQA_E_STRIDE;
  }
  return reduce_impl(workspace, splits, o, o_stride, lse, batch, num_heads, seq_q, head_dim, dtype, stream,
                     q_start, q_len);
}

}  // extern "C"

namespace {

int reduce_impl(const float* workspace, int splits, void* o, const int64_t o_stride[4], float* lse, int batch,
                int num_heads, int seq_q, int head_dim, int dtype, void* stream, const int* q_start,
                const int* q_len) {
  if (batch < 0 || num_heads <= 0 || seq_q < 0) return GQA_E_SHAPE;
  if (head_dim != 64 && head_dim != 128) return GQA_E_HEAD_DIM;
  if (dtype != GQA_DTYPE_BF16 && dtype != GQA_DTYPE_FP16) return GQA_E_DTYPE;
  if (splits < 1 || splits > GQA_MAX_SPLITS) return GQA_E_SPLITS;
  if (batch == 0 || seq_q == 0) return GQA_OK;
  if (workspace == nullptr) return GQA_E_NULL;
  if ((reinterpret_cast<uintptr_t>(workspace) & 15u) != 0) return GQA_E_STRIDE;
  int rc = check_tensor(o, o_stride);
  if (rc) return rc;
  gqa::ReduceParams p{};
  const size_t rows = (size_t)batch * num_heads * seq_q * splits;
  p.ws_acc = workspace;
  p.ws_m = workspace + rows * head_dim;
  p.ws_l = p.ws_m + rows;
  p.o = ref(o, o_stride);
  p.B = batch;
  p.Hq = num_heads;
  p.Sq = seq_q;
  p.D = head_dim;
  p.splits = splits;
  p.lse = lse;
  p.q_start = q_start;
  p.q_len = q_len;
  return to_code(gqa::launch_split_reduce(p, dtype, static_cast<hipStream_t>(stream)));
}

// The paged single pass (gqa_paged_fwd_launch) and, with kv_splits > 0, the
// same over key chunks into `workspace` followed by the split combine
// (gqa_paged_fwd_chunks_launch).
int paged_fwd_impl(const void* q, const int64_t q_stride[4], const void* k_cache,
                   const int64_t k_cache_stride[4], const void* v_cache, const int64_t v_cache_stride[4],
                   const int* block_table, int table_stride, const int* seq_lens, const int* q_start,
                   const int* q_len, int block_size, int max_seq_len, void* o, const int64_t o_stride[4],
                   float* lse, float* workspace, int kv_splits, int batch, int num_heads, int num_kv_heads,
                   int seq_q, int head_dim, float scale_log2, int causal, int dtype, void* stream,
                   int n_split, float* part_ws, int* part_cnt) {
  int rc = check_dims(batch, num_heads, num_kv_heads, seq_q, max_seq_len, head_dim, dtype);
  if (rc) return rc;
  const int G = num_heads / num_kv_heads;
  if (G > gqa::kFwdRows) return GQA_E_GROUP;
  // Each LDS-DMA instruction loads 512 / head_dim rows, which must lie in
  // one block.
  if (block_size < 512 / head_dim || block_size > GQA_MAX_BLOCK_SIZE || (block_size & (block_size - 1)) != 0)
    return GQA_E_BLOCK;
  if (table_stride < 0 || (int64_t)table_stride * block_size < (int64_t)max_seq_len) return GQA_E_BLOCK;
  const int block_m = gqa::kFwdRows / G;
  const int n_mblk = (seq_q + block_m - 1) / block_m;
  if (n_split < 0 || n_split > n_mblk || (n_split > 0 && kv_splits > 0)) return GQA_E_SPLITS;
  if (batch == 0 || seq_q == 0) return GQA_OK;
  if (seq_lens == nullptr) return GQA_E_NULL;
  if ((reinterpret_cast<uintptr_t>(seq_lens) & 3u) != 0) return GQA_E_STRIDE;
  if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return GQA_E_STRIDE;
  if (n_split > 0) {
    if (part_ws == nullptr || part_cnt == nullptr) return GQA_E_NULL;
    if ((reinterpret_cast<uintptr_t>(part_ws) & 15u) != 0 || (reinterpret_cast<uintptr_t>(part_cnt) & 3u) != 0)
      return GQA_E_STRIDE;
  }
  if (kv_splits > 0 && workspace == nullptr) return GQA_E_NULL;
  if (kv_splits > 0 && (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0) return GQA_E_STRIDE;
  if ((rc = check_varlen(q_start, q_len))) return rc;
  if ((rc = check_tensor(q, q_stride)) || (rc = check_tensor(o, o_stride))) return rc;
  if (max_seq_len > 0) {
    if (block_table == nullptr) return GQA_E_NULL;
    if ((reinterpret_cast<uintptr_t>(block_table) & 3u) != 0) return GQA_E_STRIDE;
    if ((rc = check_tensor(k_cache, k_cache_stride)) || (rc = check_tensor(v_cache, v_cache_stride))) return rc;
  }

  gqa::FwdParams p{};
  p.q = ref(q, q_stride);
  p.k = cache_ref(k_cache, k_cache_stride);
  p.v = cache_ref(v_cache, v_cache_stride);
  p.o = ref(o, o_stride);
  p.dm = Dims{batch, num_heads, num_kv_heads, seq_q, max_seq_len, head_dim, G, scale_log2, causal ? 1 : 0};
  p.block_m = block_m;
  p.n_mblk = n_mblk;
  p.lse = lse;
  // Split query blocks (two key halves merged by whichever finishes last,
  // as in gqa_fwd_split_launch; no scheduling counters: one workgroup per
  // item).
  p.n_split = n_split;
  p.part_ws = part_ws;
  p.part_cnt = part_cnt;
  p.sched = nullptr;
  p.block_table = block_table;
  p.seq_lens = seq_lens;
  p.table_stride = table_stride;
  int shift = 0;
  while ((1 << shift) < block_size) ++shift;
  p.block_shift = shift;
  p.q_start = q_start;
  p.q_len = q_len;
  if (kv_splits == 0) return to_code(gqa::launch_paged_fwd(p, dtype, static_cast<hipStream_t>(stream)));
  // Key chunks: chunk c of every query block covers key tiles [c * ct,
  // (c + 1) * ct) of the longest sequence's range; the partials go to the
  // split-KV workspace layout and the split combine writes o (and lse),
  // token-major with variable query lengths.
  p.lse = nullptr;
  const int tiles = (max_seq_len + gqa::kFwdTileKeys - 1) / gqa::kFwdTileKeys;
  p.kv_splits = kv_splits;
  p.kv_chunk_tiles = std::max((tiles + kv_splits - 1) / kv_splits, 1);
  const size_t rows = (size_t)batch * num_heads * seq_q * kv_splits;
  p.ws_acc = workspace;
  p.ws_m = workspace + rows * head_dim;
  p.ws_l = p.ws_m + rows;
  rc = to_code(gqa::launch_paged_fwd(p, dtype, static_cast<hipStream_t>(stream)));
  if (rc) return rc;
  return reduce_impl(workspace, kv_splits, o, o_stride, lse, batch, num_heads, seq_q, head_dim, dtype, stream,
                     q_start, q_len);
}

// ---------------------------------------------------------------------------
// The fixed partials buffer of gqa_split_noalloc_launch.  The runtime gives
// every device its own copy when it loads this code object; it is held until
// the process ends.  In host code `scratch` names a host-side stand-in, not
// device memory: only the address hipGetSymbolAddress returns for the
// current device may reach a kernel, memset or copy.
// ---------------------------------------------------------------------------
constexpr size_t kScratchFloats = GQA_NOALLOC_SCRATCH_BYTES / sizeof(float);
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's copy of `scratch`, looked up once
// per device with that device current.
int scratch_address(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return static_cast<int>(hipErrorInvalidDevice);
  float* a = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (a == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    a = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (a == nullptr) {
      void* sym = nullptr;
      e = hipGetSymbolAddress(&sym, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return static_cast<int>(e);
      if (sym == nullptr) return static_cast<int>(hipErrorInvalidSymbol);
      a = static_cast<float*>(sym);
      g_scratch_addr[dev].store(a, std::memory_order_release);
    }
  }
  *out = a;
  return GQA_OK;
}

}  // namespace

extern "C" {

int gqa_split_noalloc_launch(const void* q, const int64_t q_stride[4], const void* k, const int64_t k_stride[4],
                             const void* v, const int64_t v_stride[4], void* o, const int64_t o_stride[4],
                             float* lse, int splits, int batch, int num_heads, int num_kv_heads, int seq_q,
                             int seq_kv, int head_dim, float scale_log2, int causal, int dtype, void* stream) {
  int rc = check_dims(batch, num_heads, num_kv_heads, seq_q, seq_kv, head_dim, dtype);
  if (rc) return rc;
  if (splits < 1 || splits > GQA_MAX_SPLITS) return GQA_E_SPLITS;
  if (batch == 0 || seq_q == 0) return GQA_OK;
  if (gqa_split_workspace_bytes(batch, num_heads, seq_q, head_dim, splits) > GQA_NOALLOC_SCRATCH_BYTES)
    return GQA_E_SCRATCH;
  if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return GQA_E_STRIDE;
  // o is checked before the first pass is enqueued (q, k, v by the first pass).
  if ((rc = check_tensor(o, o_stride))) return rc;
  float* ws = nullptr;
  if ((rc = scratch_address(&ws))) return rc;
  rc = gqa_split_first_launch(q, q_stride, k, k_stride, v, v_stride, ws, splits, batch, num_heads, num_kv_heads,
                              seq_q, seq_kv, head_dim, scale_log2, causal, dtype, stream);
  if (rc) return rc;
  return reduce_impl(ws, splits, o, o_stride, lse, batch, num_heads, seq_q, head_dim, dtype, stream);
}

}  // extern "C"
