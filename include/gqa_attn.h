/*
 * gqa_attn.h — C ABI of the MI355X (gfx950) GQA flash-attention forward.
 *
 * Every entry point takes plain device pointers, int64 element strides and
 * int sizes, enqueues its kernels on the given HIP stream and returns at once
 * (asynchronous, like the Triton launches it replaces).  The library never
 * allocates device memory: outputs and the split-KV workspace are owned by the
 * caller.  Return value: 0 on success, a GQA_E* code below for rejected
 * arguments, or a hipError_t value (>0) reported by the launch.
 *
 * Layouts (element strides, index order b, h, s, d), as in the reference
 * gqa_kernels/dispatch.py:17-27:
 *   q : (batch, num_heads,    seq_q,  head_dim)
 *   k : (batch, num_kv_heads, seq_kv, head_dim)
 *   v : (batch, num_kv_heads, seq_kv, head_dim)
 *   o : (batch, num_heads,    seq_q,  head_dim)
 * The last dimension must be contiguous (stride 1) and each row 16-byte
 * aligned (reference README.md:112 states last-dim contiguity as an invariant).
 *
 * Semantics (reference tests/reference.py:16-34): q head h reads kv head
 * h / (num_heads / num_kv_heads); scores are scaled by head_dim^-0.5 (passed
 * here as scale_log2 = head_dim^-0.5 * log2(e), dispatch.py:48); with causal,
 * query row i attends keys [0, i + seq_kv - seq_q] (bottom-right alignment).
 */
#ifndef GQA_ATTN_H
#define GQA_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes for q, k, v and o (all four share one dtype). */
#define GQA_DTYPE_BF16 0
#define GQA_DTYPE_FP16 1

/* Error codes (negative, to stay clear of hipError_t values). */
#define GQA_OK 0
#define GQA_E_SHAPE (-1)      /* non-positive size or num_heads % num_kv_heads != 0 */
#define GQA_E_HEAD_DIM (-2)   /* head_dim not in {64, 128} (dispatch.py:32) */
#define GQA_E_DTYPE (-3)      /* dtype code not GQA_DTYPE_BF16 / GQA_DTYPE_FP16 */
#define GQA_E_STRIDE (-4)     /* last-dim stride != 1, rows not 16-byte aligned, or (single
                                 pass) (seq_kv + 192) * row stride * 2 bytes >= 2^31 */
#define GQA_E_SPLITS (-5)     /* splits outside [1, GQA_MAX_SPLITS], or chunk over
                                 GQA_PAGED_CHUNK_PAGES small pages */
#define GQA_E_GROUP (-6)      /* group size above what one packed tile holds */
#define GQA_E_NULL (-7)       /* null pointer argument */
#define GQA_E_BLOCK (-8)      /* paged cache: block_size not a power of two in
                                 [1, GQA_MAX_BLOCK_SIZE] (single pass: below
                                 512 / head_dim), or table too short */
#define GQA_E_SCRATCH (-9)    /* gqa_split_noalloc_launch: partials larger than
                                 GQA_NOALLOC_SCRATCH_BYTES */

#define GQA_MAX_SPLITS 1024
#define GQA_MAX_BLOCK_SIZE 65536
#define GQA_PAGED_CHUNK_PAGES 2048 /* pages per split chunk when block_size < 64 */

/* ABI revision; bumped when a signature or a documented limit below
 * changes.  7: a paged split chunk over pages of fewer than 64 keys may span
 * at most GQA_PAGED_CHUNK_PAGES pages (GQA_E_SPLITS beyond), and a sequence
 * without keys (seq_kv = 0, or seq_lens[b] = 0) gives zero output rows and
 * LSE -inf on every path. */
int gqa_abi_version(void);

/* Message for a return code (GQA_E* or hipError_t).  Never NULL. */
const char* gqa_strerror(int code);

/* Number of compute units of HIP device `device` (256 on MI355X), or a
 * negative value on error.  Replaces the hard-coded SM_COUNT = 28 of
 * reference gqa_kernels/dispatch.py:10. */
int gqa_device_cu_count(int device);

/* Single-pass group-packed forward: o = softmax(q k^T * scale) v.
 * Replaces the launch of gqa_fwd_kernel at reference
 * gqa_kernels/dispatch.py:49-61 (kernel gqa_kernels/gqa_fwd.py:33-109). */
int gqa_fwd_launch(const void* q, const int64_t q_stride[4],
                   const void* k, const int64_t k_stride[4],
                   const void* v, const int64_t v_stride[4],
                   void* o, const int64_t o_stride[4],
                   int batch, int num_heads, int num_kv_heads,
                   int seq_q, int seq_kv, int head_dim,
                   float scale_log2, int causal, int dtype, void* stream);

/* LSE side output.  The *_lse_launch variants below also write, for every
 * query row, lse = ln sum_k exp(scale * q.k) over the row's visible keys, as
 * fp32 into a contiguous (batch, num_heads, seq_q) array (-inf for a row
 * with no visible key).  The reference computes this quantity inside its
 * split-KV combine (gqa_kernels/gqa_split.py:134-139, m + log2 l in log2
 * units) but returns only o; it is what merging attention over separate key
 * ranges needs (context-parallel / ring attention, prefix-cache
 * composition, reference README.md:142-143).  lse must be non-NULL and
 * 4-byte aligned. */

/* gqa_fwd_launch plus the LSE side output. */
int gqa_fwd_lse_launch(const void* q, const int64_t q_stride[4],
                       const void* k, const int64_t k_stride[4],
                       const void* v, const int64_t v_stride[4],
                       void* o, const int64_t o_stride[4], float* lse,
                       int batch, int num_heads, int num_kv_heads,
                       int seq_q, int seq_kv, int head_dim,
                       float scale_log2, int causal, int dtype, void* stream);

/* Single pass with a key-range split of the heaviest query blocks and a
 * dynamic schedule of its work items (no counterpart in the reference; its
 * dispatch.py:35-45 only splits decode).
 * Under causal masking the query blocks of one (batch, kv head) carry from 1
 * to seq_kv/64 key tiles, so when there are few blocks per compute unit
 * (prefill at 2K tokens: 256 blocks for 256 CUs) the longest block sets the
 * run time.  This entry point runs the n_split heaviest blocks of every
 * (batch, kv head) as two work items each (lower and upper half of the
 * block's key tiles); the item that finishes second merges the other's
 * fp32 partial state (log-sum-exp merge) and writes o (and lse).  Results
 * equal gqa_fwd_launch's up to float rounding.  n_split in [0, number of
 * query blocks = ceil(seq_q / (256 / (num_heads / num_kv_heads)))];
 * workspace: gqa_fwd_split_workspace_bytes() bytes, 16-byte aligned (NULL
 * allowed when n_split = 0); counters: gqa_fwd_split_counters_count() int32,
 * zero on the first call and left zero by every call (one buffer serves all
 * calls on one stream; calls that overlap must not share one).  With
 * counters, the persistent single pass (head_dim 128, contiguous K/V) hands
 * out its work items dynamically when there are at least 8 per compute
 * unit: after a first static item, each workgroup takes the next from its
 * XCD's queue and then from the other XCDs' — the XCDs run at different
 * speeds under sustained MFMA load.
 * counters may be NULL when n_split = 0 (static schedule, as
 * gqa_fwd_launch).  The outputs do not depend on the schedule.  lse may be
 * NULL (no side output) or as in gqa_fwd_lse_launch. */
size_t gqa_fwd_split_workspace_bytes(int batch, int num_kv_heads, int head_dim, int n_split);
size_t gqa_fwd_split_counters_count(int batch, int num_kv_heads, int n_split);
int gqa_fwd_split_launch(const void* q, const int64_t q_stride[4],
                         const void* k, const int64_t k_stride[4],
                         const void* v, const int64_t v_stride[4],
                         void* o, const int64_t o_stride[4], float* lse,
                         float* workspace, int* counters, int n_split,
                         int batch, int num_heads, int num_kv_heads,
                         int seq_q, int seq_kv, int head_dim,
                         float scale_log2, int causal, int dtype, void* stream);

/* Single pass over key chunks, then the split-KV combine (no counterpart in
 * the reference, whose dispatch.py:47-61 runs these shapes as one program
 * per query block over all keys).  For query blocks longer than the split
 * path takes (more than 64 packed rows per kv head: chunked prefill, long
 * verify steps) against a long key cache, one work item per query block
 * leaves most compute units idle (a 128-token chunk of Llama-3.1-8B:
 * 16 items).  Here every query block of 256 packed rows runs as kv_splits
 * work items over consecutive ranges of ceil(ceil(seq_kv / 64) / kv_splits)
 * 64-key tiles, each writing the fp32 partial (m in log2 units, l,
 * unnormalised acc) of its rows into the split-KV workspace layout; the
 * split-KV combine (gqa_split_reduce_launch's kernel) then writes o and,
 * when lse is not NULL, the LSE as gqa_fwd_lse_launch.  Results equal
 * gqa_fwd_launch's up to float rounding.  kv_splits in [1, GQA_MAX_SPLITS];
 * workspace: gqa_split_workspace_bytes(batch, num_heads, seq_q, head_dim,
 * kv_splits) bytes, 16-byte aligned; counters: NULL (static schedule) or
 * gqa_fwd_split_counters_count(batch, num_kv_heads, 0) int32, zero on the
 * first call and left zero (as gqa_fwd_split_launch's). */
int gqa_fwd_chunks_launch(const void* q, const int64_t q_stride[4],
                          const void* k, const int64_t k_stride[4],
                          const void* v, const int64_t v_stride[4],
                          void* o, const int64_t o_stride[4], float* lse,
                          float* workspace, int* counters, int kv_splits,
                          int batch, int num_heads, int num_kv_heads,
                          int seq_q, int seq_kv, int head_dim,
                          float scale_log2, int causal, int dtype, void* stream);

/* Bytes of fp32 workspace the split-KV path needs for `splits` chunks:
 * acc (batch, num_heads, seq_q, splits, head_dim) followed by m and l
 * (batch, num_heads, seq_q, splits) each — the partial tensors of reference
 * gqa_kernels/gqa_split.py:160-163, packed into one buffer. */
size_t gqa_split_workspace_bytes(int batch, int num_heads, int seq_q,
                                 int head_dim, int splits);

/* Split-KV first pass: per-chunk partial (m, l, unnormalised acc) in fp32,
 * m and l in log2 units.  Replaces reference gqa_kernels/gqa_split.py:168-183
 * (kernel gqa_split.py:26-112).  Chunk s covers keys
 * [s*ceil(seq_kv/splits), (s+1)*ceil(seq_kv/splits)) ∩ [0, seq_kv). */
int gqa_split_first_launch(const void* q, const int64_t q_stride[4],
                           const void* k, const int64_t k_stride[4],
                           const void* v, const int64_t v_stride[4],
                           float* workspace, int splits,
                           int batch, int num_heads, int num_kv_heads,
                           int seq_q, int seq_kv, int head_dim,
                           float scale_log2, int causal, int dtype,
                           void* stream);

/* Split-KV second pass: log-sum-exp combine of the partials into o.
 * Replaces reference gqa_kernels/gqa_split.py:185-193
 * (kernel gqa_split.py:115-147). */
int gqa_split_reduce_launch(const float* workspace, int splits,
                            void* o, const int64_t o_stride[4],
                            int batch, int num_heads, int seq_q, int head_dim,
                            int dtype, void* stream);

/* gqa_split_reduce_launch plus the LSE side output (see gqa_fwd_lse_launch). */
int gqa_split_reduce_lse_launch(const float* workspace, int splits,
                                void* o, const int64_t o_stride[4], float* lse,
                                int batch, int num_heads, int seq_q, int head_dim,
                                int dtype, void* stream);

/* Number of int32 counters gqa_split_fused_launch needs: one per
 * (batch, kv head, block of 32 packed (position, head) rows). */
size_t gqa_split_counters_count(int batch, int num_heads, int num_kv_heads, int seq_q);

/* Split-KV first pass with the log-sum-exp combine fused in: the last
 * workgroup to finish each (batch, kv head, row block) combines the splits of
 * its rows into o (same arithmetic as gqa_split_reduce_launch).  Together the
 * two launches of reference gqa_kernels/gqa_split.py:168-193 in one kernel.
 * counters (gqa_split_counters_count ints) must be zero on entry; the kernel
 * leaves them zero, so one counter buffer can serve every call made on one
 * stream (calls that overlap in time need separate buffers).  The combine
 * stages min(32, G*seq_q) * splits values in LDS and addresses the fp32
 * partials with 32-bit offsets: above 4096 values, or with more than
 * 2^32 - 16 bytes of partial accumulators (batch * num_heads * seq_q *
 * splits * head_dim * 4), this returns GQA_E_SPLITS (use
 * gqa_split_first_launch + gqa_split_reduce_launch). */
int gqa_split_fused_launch(const void* q, const int64_t q_stride[4],
                           const void* k, const int64_t k_stride[4],
                           const void* v, const int64_t v_stride[4],
                           void* o, const int64_t o_stride[4],
                           float* workspace, int* counters, int splits,
                           int batch, int num_heads, int num_kv_heads,
                           int seq_q, int seq_kv, int head_dim,
                           float scale_log2, int causal, int dtype,
                           void* stream);

/* gqa_split_fused_launch plus the LSE side output (see gqa_fwd_lse_launch). */
int gqa_split_fused_lse_launch(const void* q, const int64_t q_stride[4],
                               const void* k, const int64_t k_stride[4],
                               const void* v, const int64_t v_stride[4],
                               void* o, const int64_t o_stride[4], float* lse,
                               float* workspace, int* counters, int splits,
                               int batch, int num_heads, int num_kv_heads,
                               int seq_q, int seq_kv, int head_dim,
                               float scale_log2, int causal, int dtype,
                               void* stream);

/* The whole split-KV forward in one call: gqa_split_first_launch into
 * `workspace`, then gqa_split_reduce_launch into o (gqa_split_reduce_lse_launch
 * when lse is not NULL), both on `stream` — what reference
 * gqa_kernels/gqa_split.py:153-194 (split_kv_forward) launches, with one
 * host-to-library transition instead of two.  Arguments and errors as those
 * two entry points; o (and lse) are checked before the first pass is
 * enqueued. */
int gqa_split_launch(const void* q, const int64_t q_stride[4],
                     const void* k, const int64_t k_stride[4],
                     const void* v, const int64_t v_stride[4],
                     void* o, const int64_t o_stride[4], float* lse,
                     float* workspace, int splits,
                     int batch, int num_heads, int num_kv_heads,
                     int seq_q, int seq_kv, int head_dim,
                     float scale_log2, int causal, int dtype, void* stream);

/* Split-KV forward that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory or hand in a
 * workspace (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  It runs gqa_split_first_launch and then
 * gqa_split_reduce_launch (gqa_split_reduce_lse_launch when lse is not
 * NULL) on `stream`, with the fp32 partials in a fixed buffer inside the
 * library instead of a caller workspace; q, k, v, o and lse are the
 * caller's, as there.
 * Limit: gqa_split_workspace_bytes(batch, num_heads, seq_q, head_dim, splits)
 * must be at most GQA_NOALLOC_SCRATCH_BYTES (16 MiB: e.g. 64 splits of a
 * decode step of 64 query heads at batch 16), else GQA_E_SCRATCH, before any
 * HIP call.  The buffer exists once per device, for the life of the
 * process, and every call on that device shares it: calls that can overlap
 * on one device (different streams, or two host threads) race on it and must
 * use gqa_split_first_launch with workspaces of their own.  The pointers and
 * the stream must belong to the current device. */
#define GQA_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int gqa_split_noalloc_launch(const void* q, const int64_t q_stride[4],
                             const void* k, const int64_t k_stride[4],
                             const void* v, const int64_t v_stride[4],
                             void* o, const int64_t o_stride[4], float* lse,
                             int splits, int batch, int num_heads, int num_kv_heads,
                             int seq_q, int seq_kv, int head_dim,
                             float scale_log2, int causal, int dtype,
                             void* stream);

/* Paged KV cache.  The reference names a persistent prefix KV cache and a
 * vLLM-shaped interface as the next step after its kernel (README.md:140-146,
 * "none of the above is in this repo"); these entry points are that step.
 * K and V of all sequences live in caches of shape
 *   k_cache, v_cache : (num_blocks, block_size, num_kv_heads, head_dim)
 * (element strides in that order, last one 1, rows 16-byte aligned), with
 * block_size a power of two.  Key j of sequence b is slot j % block_size of
 * block block_table[b * table_stride + j / block_size]; sequence b has
 * seq_lens[b] keys.  block_table and seq_lens are int32 device arrays.
 * Sequences may share blocks (a common prefix stored once).
 *
 * Variable query lengths (q_start and q_len, both NULL or both int32 device
 * arrays of batch entries): q and o are then token-major — row pos of
 * sequence b and head h is token q_start[b] + pos, at element offset
 * token * stride[2] + h * stride[1] (stride[0] is not used) — and sequence b
 * has q_len[b] <= seq_q query rows; causal alignment uses its own
 * q_len[b]: query row i attends keys [0, i + seq_lens[b] - q_len[b]].
 * Rows past q_len[b] are neither read nor written, and an LSE side output is
 * (tokens, num_heads).  With both NULL, q and o are (batch, num_heads,
 * seq_q, head_dim) as everywhere else. */

/* Split-KV first pass over a paged cache; combine with
 * gqa_split_reduce_launch / gqa_split_reduce_lse_launch (same workspace
 * layout), or gqa_split_reduce_varlen_launch with variable query lengths.  q is (batch, num_heads, seq_q, head_dim) as above; with causal,
 * query row i of sequence b attends keys [0, i + seq_lens[b] - seq_q]
 * (the bottom-right alignment of the contiguous path, per sequence).
 * max_seq_len bounds the sequences (seq_lens[b] is clamped to
 * [0, max_seq_len]; keys past it are not read) and sets the chunk size: chunk s covers keys
 * [s*C, (s+1)*C) with C = ceil(max_seq_len / splits) rounded up to a
 * multiple of 64.  Every table entry a sequence reaches must index a block
 * of the caches; table_stride * block_size >= max_seq_len.  With
 * block_size < 64 a chunk may span at most GQA_PAGED_CHUNK_PAGES pages
 * (C / block_size <= 2048), else GQA_E_SPLITS: raise splits. */
int gqa_paged_split_first_launch(const void* q, const int64_t q_stride[4],
                                 const void* k_cache, const int64_t k_cache_stride[4],
                                 const void* v_cache, const int64_t v_cache_stride[4],
                                 const int* block_table, int table_stride,
                                 const int* seq_lens, const int* q_start, const int* q_len,
                                 int block_size, int max_seq_len,
                                 float* workspace, int splits,
                                 int batch, int num_heads, int num_kv_heads,
                                 int seq_q, int head_dim,
                                 float scale_log2, int causal, int dtype,
                                 void* stream);

/* Single-pass forward over a paged cache, for query blocks too large for the
 * split-KV pass (chunked prefill against a cached prefix): the kernel of
 * gqa_fwd_launch with each K/V tile loaded from its blocks, so block_size
 * must be a power of two >= 512 / head_dim (4 for head_dim 128, 8 for 64:
 * the rows of one LDS-DMA instruction).  Caches, block_table, seq_lens,
 * max_seq_len and the causal alignment as gqa_paged_split_first_launch;
 * q and o are (batch, num_heads, seq_q, head_dim); lse may be NULL (no side
 * output) or as in gqa_fwd_lse_launch. */
int gqa_paged_fwd_launch(const void* q, const int64_t q_stride[4],
                         const void* k_cache, const int64_t k_cache_stride[4],
                         const void* v_cache, const int64_t v_cache_stride[4],
                         const int* block_table, int table_stride,
                         const int* seq_lens, const int* q_start, const int* q_len,
                         int block_size, int max_seq_len,
                         void* o, const int64_t o_stride[4], float* lse,
                         int batch, int num_heads, int num_kv_heads,
                         int seq_q, int head_dim,
                         float scale_log2, int causal, int dtype, void* stream);

/* gqa_paged_fwd_launch over key chunks, for few query blocks against long
 * sequences (a chunk of new tokens appended to a long cached prefix, with
 * few sequences in the batch): every query block runs as kv_splits work
 * items, item c over key tiles [c * ct, (c + 1) * ct) with ct =
 * ceil(ceil(max_seq_len / 64) / kv_splits), each storing its rows' fp32
 * partials in `workspace` (gqa_split_workspace_bytes(batch, num_heads,
 * seq_q, head_dim, kv_splits) bytes, 16-byte aligned), and the split combine
 * then writes o (and lse, which may be NULL), token-major with variable
 * query lengths.  Arguments otherwise as gqa_paged_fwd_launch; kv_splits in
 * [1, GQA_MAX_SPLITS].  No counterpart in the reference (whose roadmap,
 * README.md:140-146, has the paged cache); the contiguous form is
 * gqa_fwd_chunks_launch. */
int gqa_paged_fwd_chunks_launch(const void* q, const int64_t q_stride[4],
                                const void* k_cache, const int64_t k_cache_stride[4],
                                const void* v_cache, const int64_t v_cache_stride[4],
                                const int* block_table, int table_stride,
                                const int* seq_lens, const int* q_start, const int* q_len,
                                int block_size, int max_seq_len,
                                void* o, const int64_t o_stride[4], float* lse,
                                float* workspace, int kv_splits,
                                int batch, int num_heads, int num_kv_heads,
                                int seq_q, int head_dim,
                                float scale_log2, int causal, int dtype, void* stream);

/* gqa_paged_fwd_launch with the n_split heaviest query blocks of every
 * (sequence, kv head) run as two work items over the two halves of their key
 * range, merged by whichever finishes last — gqa_fwd_split_launch's split
 * over a paged cache (no counterpart in the reference, whose single pass
 * runs every query block as one program, gqa_kernels/dispatch.py:47-61).
 * Arguments as gqa_paged_fwd_launch, plus workspace:
 * gqa_fwd_split_workspace_bytes(batch, num_kv_heads, head_dim, n_split)
 * bytes, 16-byte aligned; counters: at least batch * num_kv_heads * n_split
 * int32 (gqa_fwd_split_counters_count serves), zero on the first call and
 * left zero (one buffer serves every call on one stream; calls that overlap
 * in time need separate buffers).  n_split in [0, ceil(seq_q / (256 / G))]
 * (0: gqa_paged_fwd_launch), else GQA_E_SPLITS. */
int gqa_paged_fwd_split_launch(const void* q, const int64_t q_stride[4],
                               const void* k_cache, const int64_t k_cache_stride[4],
                               const void* v_cache, const int64_t v_cache_stride[4],
                               const int* block_table, int table_stride,
                               const int* seq_lens, const int* q_start, const int* q_len,
                               int block_size, int max_seq_len,
                               void* o, const int64_t o_stride[4], float* lse,
                               float* workspace, int* counters, int n_split,
                               int batch, int num_heads, int num_kv_heads,
                               int seq_q, int head_dim,
                               float scale_log2, int causal, int dtype, void* stream);

/* gqa_split_reduce_launch for variable query lengths (q_start, q_len as
 * above, non-NULL; o token-major); lse may be NULL or receives (tokens,
 * num_heads). */
int gqa_split_reduce_varlen_launch(const float* workspace, int splits,
                                   void* o, const int64_t o_stride[4], float* lse,
                                   const int* q_start, const int* q_len,
                                   int batch, int num_heads, int seq_q, int head_dim,
                                   int dtype, void* stream);

/* Store new tokens' K and V into the paged caches:
 * k_cache[slot / block_size, slot % block_size, h, :] = k[t, h, :] (and V)
 * with slot = slot_mapping[t] (int64); tokens whose slot is negative are
 * skipped (padding).  k, v : (num_tokens, num_kv_heads, head_dim) with
 * element strides k_stride / v_stride (last one 1, rows 16-byte aligned).
 * Every non-negative slot must lie inside the caches. */
int gqa_paged_cache_write_launch(const void* k, const int64_t k_stride[3],
                                 const void* v, const int64_t v_stride[3],
                                 void* k_cache, const int64_t k_cache_stride[4],
                                 void* v_cache, const int64_t v_cache_stride[4],
                                 const int64_t* slot_mapping, int num_tokens,
                                 int num_kv_heads, int head_dim, int block_size,
                                 int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GQA_ATTN_H */
