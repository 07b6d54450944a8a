// gqa_params.hpp — kernel parameter blocks and the launchers each kernel
// translation unit exports to the C-ABI layer (gqa_abi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gqa {

// Strides are in elements; the head_dim stride is 1 (checked by the ABI).
struct TensorRef {
  const void* ptr;
  int64_t sb, sh, ss;  // batch, head, sequence strides
};

struct Dims {
  int B, Hq, Hkv, Sq, Skv, D, G;
  float c;  // head_dim^-0.5 * log2(e)
  int causal;
};

// Single-pass group-packed forward.
struct FwdParams {
  TensorRef q, k, v, o;
  Dims dm;
  int block_m;  // query positions per workgroup (G * block_m <= kFwdRows packed rows)
  int n_mblk;   // ceil(Sq / block_m)
  float* lse;   // optional (nullptr): natural-log LSE per row, contiguous (B, Hq, Sq)
  // Key-range split of the n_split heaviest query blocks of every (b, kv
  // head) into two work items (lower and upper half of the block's key
  // tiles); the second item to finish merges the two partial states.
  // part_ws: kFwdPartFloats<D> floats per part, two parts per split block;
  // part_cnt: one zero-initialised counter per split block (left zero).
  int n_split;
  float* part_ws;
  int* part_cnt;
  // Paged K/V (gqa_paged_fwd_launch only): k/v as in SplitParams (block,
  // head and slot strides), block_size >= 64 so a 64-key tile lies in one
  // block; sequence b has min(seq_lens[b], Skv) keys.
  const int* block_table;
  const int* seq_lens;
  int table_stride;
  int block_shift;
  // Variable query lengths (nullptr: every sequence has Sq rows in the
  // (B, H, S, D) q and o).  Otherwise q and o are token-major: row `pos` of
  // sequence b, head h is token q_start[b] + pos at ptr + token * ss + h * sh,
  // and sequence b has q_len[b] <= Sq query rows.
  const int* q_start;
  const int* q_len;
  // Persistent single pass (contiguous K/V, head_dim 128): workgroups
  // launched, each working through a list of items (set by launch_fwd).
  int n_wg;
  // Persistent single pass: nullptr (static schedule) or kFwdSchedCounters
  // zero-initialised ints (dynamic schedule across XCDs), left zero.
  int* sched;
  // Key chunks (contiguous K/V, fixed query lengths; n_split = 0): when
  // kv_splits > 0 every query block runs as kv_splits work items over
  // consecutive ranges of kv_chunk_tiles key tiles, each writing the fp32
  // partial (m in log2 units, l, unnormalised acc) of its valid rows into
  // the split-KV workspace layout (SplitParams::ws_*; the split combine
  // then writes o and lse) instead of o.
  int kv_splits;
  int kv_chunk_tiles;
  float* ws_acc;  // (B, Hq, Sq, kv_splits, D)
  float* ws_m;    // (B, Hq, Sq, kv_splits)
  float* ws_l;    // (B, Hq, Sq, kv_splits)
};

// Split-KV first pass: one workgroup per (b, kv head, row block, split).
struct SplitParams {
  TensorRef q, k, v;
  Dims dm;
  float* ws_acc;  // (B, Hq, Sq, splits, D)
  float* ws_m;    // (B, Hq, Sq, splits), log2 units
  float* ws_l;    // (B, Hq, Sq, splits)
  int splits;
  int chunk;   // ceil(Skv / splits)
  int n_rblk;  // ceil(G * Sq / 32)
  // Fused combine (optional): when counters != nullptr, the last workgroup of
  // each (b, kv head, row block) to finish combines the splits into o.
  // counters: B * Hkv * n_rblk ints, zero on entry, left zero on exit.
  int* counters;
  TensorRef o;
  float* lse;  // optional, fused combine only: as FwdParams::lse
  // Paged K/V cache (gqa_paged_split_first_launch only): k/v point at a
  // (num_blocks, block_size, Hkv, D) cache with sb = block stride, ss = slot
  // stride, sh = head stride (not the dimension order); key j of sequence b
  // is slot j % block_size of block block_table[b * table_stride + j /
  // block_size]; sequence b has seq_lens[b] keys (dm.Skv is the longest).
  const int* block_table;
  const int* seq_lens;
  int table_stride;
  int block_shift;  // log2(block_size)
  // Variable query lengths (nullptr: every sequence has Sq rows in the
  // (B, H, S, D) q and o).  Otherwise q and o are token-major: row `pos` of
  // sequence b, head h is token q_start[b] + pos at ptr + token * ss + h * sh,
  // and sequence b has q_len[b] <= Sq query rows.
  const int* q_start;
  const int* q_len;
  // Stagger the tile order of the splits (set when each head's K and V rows
  // are consecutive: key stride == head_dim).
  int rotate;
};

// Split-KV combine: one workgroup per (b, q head, query row).
struct ReduceParams {
  const float* ws_acc;
  const float* ws_m;
  const float* ws_l;
  TensorRef o;
  int B, Hq, Sq, D, splits;
  float* lse;  // optional: as FwdParams::lse
  const int* q_start;  // optional: as FwdParams::q_start / q_len
  const int* q_len;
};

// Packed query rows per single-pass workgroup (8 waves x 32 rows).
constexpr int kFwdRows = 256;
constexpr int kFwdThreads = 512;
// One partial state of a split query block: per lane of the 8 waves, D/2
// accumulators, the reference max and the lane's partial row sum.
constexpr int kFwdPartFloats(int D) { return kFwdThreads * (D / 2 + 2); }
// Scheduling counters of the persistent single pass (8 XCD queues, 8 + 1
// counts of finished workgroups, padding), and the items per workgroup from
// which it schedules dynamically.
constexpr int kFwdSchedCounters = 32;
constexpr int kFwdDynMinItemsPerWg = 8;
// ln(2): converts a log2-domain log-sum-exp to the natural-log LSE.
constexpr float kLn2 = 0.693147180559945309f;
// Keys per single-pass LDS tile, and per split-KV LDS tile.
constexpr int kFwdTileKeys = 64;
constexpr int kSplitTileKeys = 128;
// The fused combine stages (valid rows of a 32-row block) x splits values in
// LDS; above this the separate combine kernel is used.
constexpr int kFusedMaxRowSplitsHost = 4096;
// Block-table entries a split-KV workgroup over pages of fewer than 64 keys
// copies to LDS (8 KiB): its chunk may span at most this many pages.
constexpr int kPagedTableMax = 2048;

// Paged cache write: new tokens (num_tokens, Hkv, D) into
// (num_blocks, block_size, Hkv, D) caches at slot_mapping[t].
struct CacheWriteParams {
  const void* k;
  const void* v;
  int64_t k_st, k_sh, v_st, v_sh;  // token and head strides of k / v (elements)
  TensorRef kc, vc;                // caches: sb = block, ss = slot, sh = head strides
  const int64_t* slots;
  int n_tokens, Hkv, D, block_shift;
  int elem_bytes;
};

// Compute units of the current device (0 if unknown), cached per device.
inline int device_cu_count() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev < 64) cached[dev] = n;
  return n;
}

hipError_t launch_fwd(const FwdParams& p, int dtype, hipStream_t stream);
hipError_t launch_paged_fwd(const FwdParams& p, int dtype, hipStream_t stream);
hipError_t launch_split_first(const SplitParams& p, int dtype, hipStream_t stream);  // fused if p.counters
hipError_t launch_paged_split_first(const SplitParams& p, int dtype, hipStream_t stream);
hipError_t launch_paged_cache_write(const CacheWriteParams& p, hipStream_t stream);
hipError_t launch_split_reduce(const ReduceParams& p, int dtype, hipStream_t stream);
// Decode-shaped first pass (gqa_decode.hip): head_dim 128, contiguous K/V,
// fixed query lengths, 32-bit chunk and workspace offsets.
bool decode_kernel_fits(const SplitParams& p);
hipError_t launch_decode_first(const SplitParams& p, int dtype, hipStream_t stream);  // fused if p.counters

}  // namespace gqa
