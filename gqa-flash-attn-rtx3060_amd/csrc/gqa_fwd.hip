// gqa_fwd.hip — single-pass group-packed GQA forward for gfx950.
//
// Replaces the Triton kernel gqa_fwd_kernel (reference
// gqa_kernels/gqa_fwd.py:33-109).  One workgroup = 8 waves = 256 packed query
// rows of ONE (batch, kv head): G query heads x block_m positions (row r ->
// head r / block_m, position r % block_m, as gqa_fwd.py:58-63), so each K/V
// tile staged in LDS feeds the whole query group.  Per 64-key tile and wave
// (32 rows):
//   S^T = K Q^T        (bf16/f16 MFMA 32x32x16, fp32 accumulate)
//   online softmax     (exp2 domain, scale applied in fp32, gqa_fwd.py:98-101)
//   O^T += V^T P^T     (P rounded to the input type, gqa_fwd.py:103)
// Causal: the key loop stops at the workgroup's last visible key
// (gqa_fwd.py:70-73) and masks only the tiles that cross the diagonal or the
// end of the keys.
//
// Schedule ("ping-pong").  The waves form two groups of four, A = waves 0-3
// and B = waves 4-7; wave w and wave w+4 share a SIMD.  Work alternates
// between MFMA phases (the P*V product of the previous tile and S^T of the
// current one: 32 MFMAs per wave) and softmax phases (VALU only), and the two
// groups run one phase apart, separated by workgroup barriers: while one
// group's MFMAs occupy the matrix core of a SIMD, the other group's softmax
// runs on the same SIMD's vector ALU.
//
//   phase:   0       1       2       3       4     ...
//   A:     S(0)    sm(0)   PV(0)   sm(1)   PV(1)
//                          +S(1)           +S(2)
//   B:     (idle)  S(0)    sm(0)   PV(0)   sm(1)
//                                  +S(1)
//
// K and V tiles are both loaded straight into LDS (buffer loads in their
// LDS-DMA form) through a ring of three stages; stage t holds K(t) and
// V(t-1), the operands of MFMA phase t.  Each softmax phase issues the loads
// two tiles ahead (group A: K, group B: V) and waits for the ones issued one
// softmax phase earlier, so a load has two phases to land and the ring never
// overwrites a stage that is still read.
#include <algorithm>
#include <type_traits>

#include "gqa_common.hpp"
#include "gqa_lds.hpp"
#include "gqa_params.hpp"

namespace gqa {

// ---------------------------------------------------------------------------
// Online softmax of one 64-key S^T tile held as two 32-key blocks (16 values
// per lane and block; the two lane halves hold the other 16 keys of the
// same row), exp2 domain.
//
// Lazy rescaling: the reference point m_ref of a row is kept as long as the
// probabilities computed against it stay at most 2^kRescaleLog2, which
// bf16/fp16 P and fp32 l/acc hold as exactly as probabilities <= 1.  A tile's
// exponentials are first computed against the current m_ref, with no row
// max; a lane's partial row sum bounds each of its probabilities, so only
// when some lane's sum exceeds 2^kRescaleLog2 (or is NaN / inf), or some row
// has no reference yet, does the wave take the tile's exact row max, raise
// m_ref to it, rescale l and the accumulators, and recompute the tile's
// exponentials.  The decision is wave-uniform, so in steady state neither a
// max tree nor the O accumulators cost VALU work.  The result o = acc / l is
// unchanged (both are relative to the same m_ref).  A row whose m_ref is
// still -inf after the exact pass (every key masked so far) uses 0 as the
// reference, so a fully masked tile contributes p = 0, never NaN.
// ---------------------------------------------------------------------------
constexpr float kRescaleSum = 256.0f;  // 2^8

// Exact pass: the tile's row max (a max3 tree), m_ref raised to it, l and the
// accumulators rescaled.  Returns -m_ref * c, the offset of the exponent.
template <int NACC>
__device__ inline float softmax_rebase(const f32x16 (&s)[2], float& m_ref, float& l_run, f32x16 (&acc)[NACC],
                                       float c) {
  float m1[11];
#pragma unroll
  for (int k = 0; k < 10; ++k) {
    const int i0 = 3 * k, i1 = 3 * k + 1, i2 = 3 * k + 2;
    m1[k] = vmax3(s[i0 >> 4][i0 & 15], s[i1 >> 4][i1 & 15], s[i2 >> 4][i2 & 15]);
  }
  m1[10] = vmax3(s[1][14], s[1][15], s[1][15]);
  const float n0 = vmax3(m1[0], m1[1], m1[2]), n1 = vmax3(m1[3], m1[4], m1[5]);
  const float n2 = vmax3(m1[6], m1[7], m1[8]), n3 = vmax3(m1[9], m1[10], m1[10]);
  const float mx = xhalf_max(vmax3(vmax3(n0, n1, n2), n3, n3));
  const float m_new = fmaxf(m_ref, mx);
  const float m_new_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
  const float alpha = fast_exp2((m_ref - m_new_use) * c);
  l_run *= alpha;
#pragma unroll
  for (int db = 0; db < NACC; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[db][v] *= alpha;
  m_ref = m_new;
  return -m_new_use * c;
}

// One 32-key block: p = 2^(s*c - m_ref*c) in fp32, rounded to the input type
// and packed as the P^T operand; returns the fp32 row sum (a tree).
template <int DT>
__device__ inline float softmax_exp(const f32x16& s, float nmc, float c, u32x4 (&pk)[2]) {
  using E = Elem<DT>;
  float pv[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) pv[v] = fast_exp2(__builtin_fmaf(s[v], c, nmc));
  float s8[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) s8[j] = pv[2 * j] + pv[2 * j + 1];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int e = 0; e < 4; ++e) pk[kk][e] = E::pack2(pv[8 * kk + 2 * e], pv[8 * kk + 2 * e + 1]);
  return ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
}

// ---------------------------------------------------------------------------
// Instruction schedule of an MFMA phase: slot j is one MFMA; the LDS reads of
// slot j + P are issued right after MFMA j (P slots ahead, to cover the LDS
// latency).  Slots [0, NRD2) are P*V MFMAs with two transposing reads each,
// the rest S^T MFMAs with one 16-byte read each.
// ---------------------------------------------------------------------------
template <int NRD2, int NSLOT, int P, int J>
__device__ __forceinline__ void mphase_prefetch() {
  if constexpr (J < P && J < NSLOT) {
    __builtin_amdgcn_sched_group_barrier(0x100, (J < NRD2) ? 2 : 1, 0);  // LDS reads
    mphase_prefetch<NRD2, NSLOT, P, J + 1>();
  }
}
template <int NRD2, int NSLOT, int P, int J>
__device__ __forceinline__ void mphase_pipe() {
  if constexpr (J < NSLOT) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    if constexpr (J + P < NSLOT) __builtin_amdgcn_sched_group_barrier(0x100, (J + P < NRD2) ? 2 : 1, 0);
    mphase_pipe<NRD2, NSLOT, P, J + 1>();
  }
}

// PG: 0 contiguous K/V; 1 a paged cache through the block table with pages
// of >= 64 keys (one buffer descriptor per 64-key tile, ending at the
// sequence's last key); 2 pages of RPI..8 keys (RPI = 512 / D rows per
// LDS-DMA instruction: each instruction's rows lie in one page, and every
// instruction gets its own descriptor); 3 pages of 16 or 32 keys (each wave
// loads 16 consecutive rows of a tile, which lie in one page: one table
// read and one descriptor per wave and tile).
// D = 64 keeps to 128 VGPRs (four waves per SIMD): two workgroups share a
// compute unit, which outweighs the shorter LDS-read lookahead it needs.
//
// Contiguous K/V at D = 128 (one workgroup per compute unit) runs
// persistent: p.n_wg workgroups each work through a list of items (below),
// and an item's start overlaps the previous item's end: as soon as the
// finished item's output has left the LDS stages, the workgroup issues the
// next item's first K/V tiles and Q, and the output stores drain while
// those loads are in flight.  The workgroup launch between items leaves the
// critical path.
// KC: key chunks (FwdParams::kv_splits > 0), a separate instance so the
// others keep their registers.
template <int DT, int D, int PG, bool KC = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(D == 64 ? 4 : 2))) void gqa_fwd_kernel(
    FwdParams p) {
  using E = Elem<DT>;
  using T = typename E::T;
  using ST = FwdStage<D>;
  constexpr int CPR = ST::CPR;
  constexpr bool PAGED = PG != 0;
  constexpr bool SMALL = PG == 2;
  constexpr bool MEDIUM = PG == 3;
  constexpr bool PERSIST = PG == 0 && D == 128;
  // Block ids a wave needs per tile: one, or (small pages) one per LDS-DMA
  // instruction it issues.
  struct TileBlocks { int id[SMALL ? ST::NI : 1]; };
  constexpr int NDB = D / 32;  // 32-wide d blocks of O^T
  constexpr int NKS = D / 16;  // k-steps of S^T
  constexpr int PF = (D == 64) ? 3 : 6;  // MFMA slots of LDS-read lookahead
  // Six separate arrays (not one): the compiler can then tell the LDS-DMA
  // targets of later tiles from the buffers being read, and does not wait for
  // those loads before the reads.
  // The V stages take the low 48 KiB: an MFMA phase reads V with twice as
  // many LDS instructions as K, and below 64 KiB a stage's address fits the
  // 16-bit offset field of ds_read, so those reads need no VALU address
  // arithmetic (which would compete with the other wave's softmax on the
  // SIMD).  The compiler lays kernel LDS variables out in name order.
  __shared__ __attribute__((aligned(1024))) char lds0_v0[ST::kTileBytes];
  __shared__ __attribute__((aligned(1024))) char lds0_v1[ST::kTileBytes];
  __shared__ __attribute__((aligned(1024))) char lds0_v2[ST::kTileBytes];
  __shared__ __attribute__((aligned(1024))) char lds1_k0[ST::kTileBytes];
  __shared__ __attribute__((aligned(1024))) char lds1_k1[ST::kTileBytes];
  __shared__ __attribute__((aligned(1024))) char lds1_k2[ST::kTileBytes];
  __shared__ int s_last;

  const Dims& dm = p.dm;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6) & 7;  // wave-uniform (SGPR)
  const int grp = wave >> 2;                                     // 0: group A, 1: group B
  const int gw = wave & 3;                                       // wave index in its group
  const int i = lane & 31, hh = lane >> 5;
  const bool varlen = p.q_len != nullptr;

  // Work items: heavy (late) query blocks first under causal, and every XCD
  // gets a contiguous range of items (same kv head -> same L2).  With a key
  // split, the n_split heaviest blocks of each (b, kv head) come as two
  // items: first the upper halves of their key ranges, then (in the usual
  // order) the lower halves and the unsplit blocks.
  // Key chunks: kv_splits items per query block, the blocks of one chunk
  // consecutive (they read the same keys).
  constexpr bool chunked = KC;
  const int n_items = chunked ? p.n_mblk * p.kv_splits : p.n_mblk + p.n_split;
  const int total = n_items * dm.Hkv * dm.B;
  // The k-th item of this workgroup (-1: none).  One item per workgroup
  // (xcd_remap), or persistent: the workgroups of XCD x (hardware ids x,
  // x + 8, ...) take the XCD's item range round by round in snake order
  // (round j: slot c takes item j*S + c, or j*S + S-1-c in odd rounds), so
  // the heavy-first order hands every slot a mix of heavy and light items.
  const int n_wg = PERSIST ? p.n_wg : total;
  // Item range of XCD x: [lo, lo + n), served by its S workgroups.
  auto xrange = [&](int x, int& lo, int& n, int& S) {
    S = (n_wg - x + 7) >> 3;
    const int q = total >> 3, r = total & 7;
    lo = x * q + min(x, r);
    n = q + (x < r ? 1 : 0);
  };
  auto item_at = [&](int k) -> int {
    if (!PERSIST) return k == 0 ? xcd_remap(blockIdx.x, total) : -1;
    const int x = blockIdx.x & 7, slot = blockIdx.x >> 3;
    int lo, n, S;
    xrange(x, lo, n, S);
    const int j = k;
    const int e = j * S + ((j & 1) ? S - 1 - slot : slot);
    return e < n ? lo + e : -1;
  };
  // Dynamic schedule (persistent kernel, p.sched set): the XCDs run at
  // different speeds under sustained MFMA load (their workgroups end up to
  // 6 % apart on a static schedule), so after its first item (slot c of XCD
  // x takes item c of x's range, as above) a workgroup claims the next one
  // from its own XCD's queue — items S, S + 1, ... of the range, heavy
  // first — and, once that is empty, from the other XCDs' queues.  One
  // thread claims with an agent-scope atomic issued as the epilogue begins
  // and resolves it after the output stores, so its latency is hidden.
  // Items are independent (a split block's halves merge in a fixed order),
  // so the outputs do not depend on who computes what.  p.sched: 8 queue
  // counters, 8 + 1 counts of workgroups done, zero on entry; the last
  // workgroup to finish leaves them zero.  The counters' address waits in
  // LDS (kept in registers, it would add to those held across the tile
  // loop).
  __shared__ int s_next;
  __shared__ int* s_sched;
  if (PERSIST && t == 0) s_sched = p.sched;

  // One work item's parameters.
  struct Item {
    int b, kvh, bh, pid_m, part;  // part: -1 whole key range, 0 lower half, 1 upper half
    int skv, sq, tb, ntiles, qpos_lo;
    int64_t tok0;
    int pos, head, qpos;  // this lane's query row
    bool valid;
    const char* kbh;
    const char* vbh;
    __amdgpu_buffer_rsrc_t rk, rv;
    const int* table_row;
  };
  const uint32_t kssb = (uint32_t)(2 * p.k.ss), vssb = (uint32_t)(2 * p.v.ss);
  auto decode = [&](int w, int i, int block_m) __attribute__((always_inline)) -> Item {
    Item x;
    x.bh = w / n_items;
    int idx = w - x.bh * n_items;
    int chunk = 0;
    if constexpr (chunked) {
      chunk = idx / p.n_mblk;
      idx -= chunk * p.n_mblk;
    }
    if (idx < p.n_split) {
      x.pid_m = p.n_mblk - 1 - idx;
      x.part = 1;
    } else {
      const int mrank = idx - p.n_split;
      x.pid_m = dm.causal ? (p.n_mblk - 1 - mrank) : mrank;
      x.part = (x.pid_m >= p.n_mblk - p.n_split) ? 0 : -1;
    }
    x.b = x.bh / dm.Hkv;
    x.kvh = x.bh - x.b * dm.Hkv;
    // Keys of this sequence (paged: its own length, clamped to [0, Skv]),
    // and its query rows (variable lengths: q_len[b], tokens from q_start[b]).
    x.skv = PAGED ? min(max(load_uniform(p.seq_lens + x.b), 0), dm.Skv) : dm.Skv;
    x.sq = varlen ? min(max(load_uniform(p.q_len + x.b), 0), dm.Sq) : dm.Sq;
    x.tok0 = varlen ? (int64_t)load_uniform(p.q_start + x.b) : 0;
    // This lane's query row.
    const int r = wave * 32 + i;
    const int g = r / block_m, ml = r - g * block_m;
    x.pos = x.pid_m * block_m + ml;
    x.valid = (g < dm.G) && (x.pos < x.sq);
    x.head = x.kvh * dm.G + (g < dm.G ? g : 0);
    x.qpos = x.pos + (x.skv - x.sq);
    // Key range of this item: tiles [tb, tb + ntiles).
    const int pos_lo = x.pid_m * block_m;
    const int pos_hi = min(pos_lo + block_m, x.sq) - 1;
    int kv_end = x.skv;
    if (dm.causal) kv_end = min(x.skv, pos_hi + (x.skv - x.sq) + 1);
    kv_end = max(kv_end, 0);
    const int ntiles_all = (kv_end + ST::kKeys - 1) / ST::kKeys;
    const int tsplit = ntiles_all >> 1;
    x.tb = (x.part == 1) ? tsplit : 0;
    x.ntiles = (x.part == 0) ? tsplit : ntiles_all - x.tb;
    if constexpr (chunked) {
      // Tiles [chunk * ct, (chunk + 1) * ct) of the block's range (none
      // for a chunk past it: an empty partial).
      x.tb = chunk * p.kv_chunk_tiles;
      x.ntiles = max(min(ntiles_all - x.tb, p.kv_chunk_tiles), 0);
    }
    x.qpos_lo = pos_lo + (x.skv - x.sq);
    // Global side: buffer descriptors over this (b, kv head)'s K and V rows,
    // each ending at the last byte of row seq_kv - 1.  The host guarantees
    // (seq_kv + 192) * row stride * 2 < 2^31, so every offset (up to two
    // tiles past the end) fits 32 bits.  (An empty key range gets an empty
    // descriptor: every load reads zero.)
    x.kbh = static_cast<const char*>(p.k.ptr) + 2 * ((PAGED ? 0 : (int64_t)x.b * p.k.sb) + (int64_t)x.kvh * p.k.sh);
    x.vbh = static_cast<const char*>(p.v.ptr) + 2 * ((PAGED ? 0 : (int64_t)x.b * p.v.sb) + (int64_t)x.kvh * p.v.sh);
    const bool flat = !PAGED && dm.Skv > 0;
    x.rk = make_rsrc(x.kbh, flat ? (uint32_t)(dm.Skv - 1) * kssb + 2 * D : 0u);
    x.rv = make_rsrc(x.vbh, flat ? (uint32_t)(dm.Skv - 1) * vssb + 2 * D : 0u);
    x.table_row = PAGED ? p.block_table + (int64_t)x.b * p.table_stride : nullptr;
    return x;
  };

  int k_item = 0;
  Item it = decode(item_at(0), i, p.block_m);
  if (!PERSIST && it.pid_m * p.block_m >= it.sq) return;  // a block past this sequence's queries (variable lengths)
  // Element offset of (query row pos, head h) in q / o.
  auto row_off = [&](const Item& x, const TensorRef& tr, int pos_, int h) -> int64_t {
    return varlen ? (x.tok0 + pos_) * tr.ss + (int64_t)h * tr.sh
                  : (int64_t)x.b * tr.sb + (int64_t)h * tr.sh + (int64_t)pos_ * tr.ss;
  };

  const int lrow = lane / CPR;
  const uint32_t koff =
      (uint32_t)(lrow * kssb) + 16u * (uint32_t)((lane % CPR) ^ ST::gk((gw * ST::RPI + lrow) & 15));
  const uint32_t voff = (uint32_t)(lrow * vssb) + 16u * (uint32_t)((lane % CPR) ^ ST::sv(lrow));

  // Issue this wave's share of K or V tile `tile` (absolute index) into LDS.
  // Paged, blocks of >= 64 keys: the tile's 64 rows are one run inside one
  // block; its descriptor starts at the tile's first row and ends at the
  // sequence's last key, so rows past the sequence (and whole tiles past it,
  // which read no table entry) load as zeros.  Smaller blocks: the same per
  // LDS-DMA instruction (RPI rows, one run inside one block).
  // Paged: the block(s) holding a tile, or this wave's instructions of it
  // (read only for rows that start inside the sequence).  The softmax phases
  // use block ids read one phase ahead (blk_next), so the table reads'
  // latency is off the issue path.
  auto tile_block = [&](const Item& x, int tile) -> TileBlocks {
    TileBlocks tbk;
    const int key0 = tile * ST::kKeys;
    if constexpr (SMALL) {
#pragma unroll
      for (int j = 0; j < ST::NI; ++j) {
        const int key = key0 + (j * 4 + gw) * ST::RPI;  // first row of instruction j
        tbk.id[j] = key < x.skv ? load_uniform(x.table_row + (key >> p.block_shift)) : 0;
      }
    } else if constexpr (MEDIUM) {
      const int key = key0 + 16 * gw;  // first of this wave's 16 rows
      tbk.id[0] = key < x.skv ? load_uniform(x.table_row + (key >> p.block_shift)) : 0;
    } else {
      tbk.id[0] = (PAGED && key0 < x.skv) ? load_uniform(x.table_row + (key0 >> p.block_shift)) : 0;
    }
    return tbk;
  };
  auto issue_tile = [&](const Item& x, char* lds, const char* head, __amdgpu_buffer_rsrc_t rsrc, uint32_t rowb,
                        uint32_t off, int64_t blk_stride, int tile, const TileBlocks& blk, bool is_k) {
    const int key0 = tile * ST::kKeys;
    if constexpr (MEDIUM) {
      // This wave's rows [key, key + 16) of the tile, one run in one page:
      // instruction j loads rows key + j * RPI + 0..RPI-1 (scalar offset) into
      // LDS rows 16 gw + j * RPI + ...  Both swizzles are linear in the row
      // bits: V's depends on the lane's row lrow alone (off as given); K's
      // chunk is (lane % CPR) ^ gk(lrow) ^ gk(j * RPI).
      (void)rsrc;
      typedef __attribute__((address_space(3))) void lds_void;
      const int key = key0 + 16 * gw;
      const int rows = x.skv - key;
      __amdgpu_buffer_rsrc_t rt = make_rsrc(head, 0u);
      if (rows > 0) {
        const char* base = head + 2 * ((int64_t)blk.id[0] * blk_stride +
                                       (int64_t)(key & ((1 << p.block_shift) - 1)) * (rowb >> 1));
        rt = make_rsrc(base, (uint32_t)(min(rows, 16) - 1) * rowb + 2 * D);
      }
      if constexpr (D == 64) {
        // Derived from `off` (the lane's offset for LDS rows gw * RPI + lr),
        // so no offsets of their own stay live across the loop: sv depends
        // on lr alone, so V's is `off` for both instructions; gk(gw * RPI +
        // lr) = gk(lr) ^ gk(8 (gw & 1)) with gk(8) = 2, so K's is `off` for
        // instruction j = gw & 1 and `off` with chunk bit 1 flipped (byte
        // offset ^ 32, as lr * rowb is a multiple of 64: the host takes
        // this path only for such row strides) for the other.
        // The empty asm keeps the XOR here: hoisted out of the tile loop, its
        // result would hold a register across the loop.
        (void)lane;
        uint32_t flip = off;
        if (is_k) {
          asm volatile("" : "+v"(flip));
          flip ^= 32u;
        }
        const uint32_t other = flip;
#pragma unroll
        for (int j = 0; j < ST::NI; ++j) {
          const uint32_t o = (j == (gw & 1)) ? off : other;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (lds_void*)(lds + (gw * ST::NI + j) * 1024), 16, o,
                                                   (uint32_t)(j * ST::RPI) * rowb, 0, 0);
        }
      } else {
        (void)off;
        const int lr = lane / CPR, lc = lane % CPR;
#pragma unroll
        for (int j = 0; j < ST::NI; ++j) {
          const int sw = is_k ? (ST::gk(lr) ^ ST::gk(j * ST::RPI)) : ST::sv(lr);
          const uint32_t o = (uint32_t)(lr * rowb) + 16u * (uint32_t)(lc ^ sw);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (lds_void*)(lds + (gw * ST::NI + j) * 1024), 16, o,
                                                   (uint32_t)(j * ST::RPI) * rowb, 0, 0);
        }
      }
    } else if constexpr (SMALL) {
      // Instruction j loads rows [key, key + RPI) of the tile, one run in
      // one page (key is a multiple of RPI and pages hold >= RPI keys); its
      // descriptor ends at the sequence's last key.
      typedef __attribute__((address_space(3))) void lds_void;
#pragma unroll
      for (int j = 0; j < ST::NI; ++j) {
        const int step = j * 4 + gw;
        const int key = key0 + step * ST::RPI;
        const int rows = x.skv - key;
        __amdgpu_buffer_rsrc_t rt = make_rsrc(head, 0u);
        if (rows > 0) {
          const char* base = head + 2 * ((int64_t)blk.id[j] * blk_stride +
                                         (int64_t)(key & ((1 << p.block_shift) - 1)) * (rowb >> 1));
          rt = make_rsrc(base, (uint32_t)(min(rows, ST::RPI) - 1) * rowb + 2 * D);
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (lds_void*)(lds + step * 1024), 16, off, 0, 0, 0);
      }
    } else if constexpr (PAGED) {
      const int rows = x.skv - key0;
      __amdgpu_buffer_rsrc_t rt = make_rsrc(head, 0u);
      if (rows > 0) {
        const char* base =
            head + 2 * ((int64_t)blk.id[0] * blk_stride + (int64_t)(key0 & ((1 << p.block_shift) - 1)) * (rowb >> 1));
        rt = make_rsrc(base, (uint32_t)(min(rows, ST::kKeys) - 1) * rowb + 2 * D);
      }
      issue_tile_dma<D>(lds, rt, 0u, rowb, off, gw);
    } else {
      (void)blk;
      (void)head;
      issue_tile_dma<D>(lds, rsrc, (uint32_t)key0 * rowb, rowb, off, gw);
    }
  };
  auto issue_k = [&](const Item& x, char* lds, int tile, const TileBlocks& blk) {
    issue_tile(x, lds, x.kbh, x.rk, kssb, koff, p.k.sb, tile, blk, true);
  };
  auto issue_v = [&](const Item& x, char* lds, int tile, const TileBlocks& blk) {
    issue_tile(x, lds, x.vbh, x.rv, vssb, voff, p.v.sb, tile, blk, false);
  };

  // LDS side: per-lane read offsets (the 32-key block, chunk and row offsets
  // of each read are immediates on top of these).  The masks are no-ops on
  // the values; they give the compiler known bounds.
  constexpr uint32_t kKMask = (ST::kTileBytes / 2 - 1) & ~15u;
  constexpr uint32_t kVMask = (ST::kTileBytes - 1) & ~7u;
  uint32_t ka[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks)
    ka[ks] = (uint32_t)(pi_key(i) * (2 * D) + 16 * ((2 * ks + hh) ^ ST::gk(pi_key(i)))) & kKMask;
  // At D = 128, K stages 1 and 2 lie above 64 KiB, out of reach of
  // ds_read's 16-bit offset field.  Their reads address from kah = ka + the
  // LDS address of stage 1, kept in registers (refreshed as opaque values in
  // every MFMA phase, so the compiler neither folds them back into ka nor
  // recomputes them): the stage and block offsets stay immediates, and the
  // reads need no VALU address arithmetic beside the other wave's softmax.
  // (At D = 64 every stage lies below 64 KiB.)
  constexpr bool kHighK = 6 * ST::kTileBytes > 65536;
  const uint32_t k1base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds1_k1;
  uint32_t kah[kHighK ? NKS : 1];
#pragma unroll
  for (int ks = 0; ks < (kHighK ? NKS : 1); ++ks) kah[ks] = ka[ks] + k1base;
  uint32_t vb[NDB];
  {
    const int q = lane >> 4, ii = lane & 15;                  // 16-lane group, lane in group
    const int rowl = 8 * (q >> 1) + (ii >> 2);                // key row addressed by this lane
    const int f = (CPR == 16) ? (ii >> 2) : ((ii >> 3) & 1);  // sv(rowl) / 4
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      vb[db] = (uint32_t)(rowl * (2 * D) + 16 * (4 * (db ^ f) + 2 * (q & 1) + ((ii & 3) >> 1)) + 8 * (ii & 1)) &
               kVMask;
  }

  f32x16 acc[NDB];
  float m_run, l_run;
  const float c = dm.c;
  f32x16 sc[2];    // S^T of the current tile (MFMA phase -> softmax phase)
  u32x4 pk[2][2];  // P^T operands (softmax phase -> next MFMA phase)
  u32x4 qreg[NKS];

  auto kstage = [&](auto s3) -> char* {
    constexpr int S3 = decltype(s3)::value;
    return S3 == 0 ? lds1_k0 : (S3 == 1 ? lds1_k1 : lds1_k2);
  };
  auto vstage = [&](auto s3) -> char* {
    constexpr int S3 = decltype(s3)::value;
    return S3 == 0 ? lds0_v0 : (S3 == 1 ? lds0_v1 : lds0_v2);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using BT = std::true_type;
  using BF = std::false_type;

  // Prologue loads of item x: stage 0 = K(0), stage 1 = K(1) + V(0), and V(1)
  // of stage 2 (tile indices relative to tb), then Q.  The tile loads go
  // first: the Q loads behind them touch 32 rows per instruction and, issued
  // first, held the tile loads back by ~2 us.  An invalid row loads row 0 of
  // its sequence (always present here) and is zeroed.  Paged: returns the
  // block(s) of the tile the first softmax phase issues.
  auto prologue_q = [&](const Item& x) __attribute__((always_inline)) {
    const T* qrow = static_cast<const T*>(p.q.ptr) + row_off(x, p.q, x.valid ? x.pos : 0, x.head);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(qrow + 16 * ks + 8 * hh);
      qreg[ks] = x.valid ? v : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto prologue_kv = [&](const Item& x) __attribute__((always_inline)) -> TileBlocks {
    TileBlocks bn = tile_block(x, x.tb);
    if (grp == 0) {
      issue_k(x, lds1_k0, x.tb, bn);
    } else {
      issue_v(x, lds0_v1, x.tb, bn);
    }
    bn = tile_block(x, x.tb + 1);
    if (grp == 0) {
      issue_k(x, lds1_k1, x.tb + 1, bn);
    } else {
      issue_v(x, lds0_v2, x.tb + 1, bn);
    }
    bn = tile_block(x, x.tb + 2);
    return bn;
  };
  TileBlocks blk_next = prologue_kv(it);
  prologue_q(it);

  // MFMA phase of tile tt: P*V of tile tt-1 and S^T of tile tt, from ring
  // slot s3 = tt % 3.
  auto mphase = [&](auto s3, auto pvc, auto sc_) {
    constexpr bool DO_PV = decltype(pvc)::value;
    constexpr bool DO_S = decltype(sc_)::value;
    constexpr int NPV = DO_PV ? 4 * NDB : 0;
    constexpr int NS = DO_S ? 2 * NKS : 0;
    const char* ck = kstage(s3);
    const char* cv = vstage(s3);
    // Issue priority: the MFMA-phase wave of a SIMD first (its MFMA stream is
    // the matrix core's only work), the softmax wave in the gaps (~+2 %).
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(3);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 opv[NPV > 0 ? NPV : 1];
    u32x4 opk[NS > 0 ? NS : 1];
    if constexpr (DO_PV) {
#pragma unroll
      for (int j = 0; j < NPV; ++j) {
        const int mb = j / (2 * NDB), kk = (j / NDB) & 1, db = j % NDB;
        const int ro = (32 * mb + 16 * kk) * (2 * D);
        const u32x2 lo = ld_tr(cv + vb[db] + ro);
        const u32x2 hi = ld_tr(cv + vb[db] + ro + 4 * (2 * D));
        opv[j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
    }
    if constexpr (DO_S) {
      if constexpr (decltype(s3)::value == 0 || !kHighK) {
#pragma unroll
        for (int j = 0; j < NS; ++j) opk[j] = *reinterpret_cast<const u32x4*>(ck + (j & 1) * 32 * (2 * D) + ka[j >> 1]);
      } else {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) asm volatile("" : "+v"(kah[ks]));
#pragma unroll
        for (int j = 0; j < NS; ++j)
          opk[j] = *reinterpret_cast<const u32x4*>(ck + (j & 1) * 32 * (2 * D) + (kah[j >> 1] - k1base));
      }
    }
    if constexpr (DO_PV) {
#pragma unroll
      for (int j = 0; j < NPV; ++j) {
        const int mb = j / (2 * NDB), kk = (j / NDB) & 1, db = j % NDB;
        acc[db] = E::mfma(opv[j], pk[mb][kk], acc[db]);
      }
    }
    if constexpr (DO_S) {
      sc[0] = f32x16{};
      sc[1] = f32x16{};
#pragma unroll
      for (int j = 0; j < NS; ++j) sc[j & 1] = E::mfma(opk[j], qreg[j >> 1], sc[j & 1]);
    }
    mphase_prefetch<NPV, NPV + NS, PF, 0>();
    mphase_pipe<NPV, NPV + NS, PF, 0>();
    if constexpr (DO_S) {
      pin(sc[0]);
      pin(sc[1]);
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) pin(acc[db]);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    phase_barrier();
  };

  // Softmax phase of tile tt (ring slot tt % 3; tt counts from tb).  First
  // issues this wave's share of the loads two tiles ahead (group A: K(tt+2)
  // into stage tt+2; group B: V(tt+2) into stage tt+3), last waits for the
  // loads it issued one softmax phase earlier.
  auto vphase = [&](auto s3, int tt) {
    constexpr int S3 = decltype(s3)::value;
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
    __builtin_amdgcn_sched_barrier(0);
    const int ta = it.tb + tt;  // absolute tile index
    if (grp == 0) {
      issue_k(it, kstage(std::integral_constant<int, (S3 + 2) % 3>{}), ta + 2, blk_next);
    } else {
      issue_v(it, vstage(s3), ta + 2, blk_next);
    }
    blk_next = tile_block(it, ta + 3);
    const int key0 = ta * ST::kKeys;
    const bool need_mask = (key0 + ST::kKeys > it.skv) || (dm.causal && key0 + ST::kKeys - 1 > it.qpos_lo);
    if (need_mask) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = key0 + 32 * mb + key_of(v, hh);
          const bool off = key >= it.skv || (dm.causal && key > it.qpos);
          sc[mb][v] = off ? -__builtin_inff() : sc[mb][v];
        }
    }
    // Exponentials against the current reference; the exact pass when a
    // row has none yet or a lane's partial sum leaves the bound (not
    // `> kRescaleSum`: NaN and inf sums take the exact pass too).
    float rs0 = 0.f, rs1 = 0.f;
    bool keep = __builtin_amdgcn_ballot_w64(m_run == -__builtin_inff()) == 0;
    if (keep) {
      const float nmc = -m_run * c;
      rs0 = softmax_exp<DT>(sc[0], nmc, c, pk[0]);
      rs1 = softmax_exp<DT>(sc[1], nmc, c, pk[1]);
      keep = __builtin_amdgcn_ballot_w64(!(rs0 + rs1 <= kRescaleSum)) == 0;
    }
    if (!keep) {
      const float nmc = softmax_rebase<NDB>(sc, m_run, l_run, acc, c);
      rs0 = softmax_exp<DT>(sc[0], nmc, c, pk[0]);
      rs1 = softmax_exp<DT>(sc[1], nmc, c, pk[1]);
    }
    l_run += rs0 + rs1;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) pin(pk[mb][kk]);
#pragma unroll
    for (int db = 0; db < NDB; ++db) pin(acc[db]);
    pin(l_run);
    pin(m_run);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(ST::NI));  // all but this phase's loads
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    phase_barrier();
  };

  for (;;) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
    m_run = -__builtin_inff();
    l_run = 0.f;
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // the prologue loads
    phase_barrier();
    if (grp == 1) phase_barrier();  // group B runs one phase behind

    const int ntiles = it.ntiles;
    if (ntiles > 0) {
      mphase(I0{}, BF{}, BT{});
      vphase(I0{}, 0);
      int tt = 1;
      for (; tt + 3 <= ntiles; tt += 3) {
        mphase(I1{}, BT{}, BT{});
        vphase(I1{}, tt);
        mphase(I2{}, BT{}, BT{});
        vphase(I2{}, tt + 1);
        mphase(I0{}, BT{}, BT{});
        vphase(I0{}, tt + 2);
      }
      if (tt < ntiles) {
        mphase(I1{}, BT{}, BT{});
        vphase(I1{}, tt);
        ++tt;
        if (tt < ntiles) {
          mphase(I2{}, BT{}, BT{});
          vphase(I2{}, tt);
          ++tt;
        }
      }
      const int s3 = tt % 3;
      if (s3 == 0) mphase(I0{}, BT{}, BF{});
      else if (s3 == 1) mphase(I1{}, BT{}, BF{});
      else mphase(I2{}, BT{}, BF{});
    } else {
      phase_barrier();
    }
    if (grp == 0) phase_barrier();  // both groups pass the same number of barriers
    // No LDS-DMA load (of a tile past the end) may still be writing when the
    // stages are reused (by the next item, or for the output below), nor
    // when the workgroup exits.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();

    int* sched = nullptr;
    if constexpr (PERSIST) sched = s_sched;
    const bool dyn = sched != nullptr;
    int w_next = PERSIST && !dyn ? item_at(k_item + 1) : -1;
    // Dynamic schedule: thread 0 claims a ticket of this XCD's queue as the
    // epilogue begins; it is resolved after the output stores, which hide
    // the atomic's round trip.
    const int xq = (int)(__builtin_amdgcn_s_getreg((31 << 11) | 20) & 7);  // HW_REG_XCC_ID
    int ticket = 0;
    if (dyn && t == 0) ticket = __hip_atomic_fetch_add(&sched[xq], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // One workgroup per item: this item's parameters and the lane ids again,
    // from the item index, block_m and a zero laundered through SGPRs (the
    // lane id through v_mbcnt): kept from the start, the values read only
    // here would stay live across the whole tile loop (at D = 64, in
    // scratch).  The persistent kernel keeps them (and measured 35-60 %
    // slower on short key-split prefills when re-deriving them).
    int w_cur = item_at(k_item), zero = 0, bm = p.block_m;
    if constexpr (!PERSIST) asm volatile("" : "+s"(w_cur), "+s"(zero), "+s"(bm));
    const int lane_e =
        PERSIST ? lane : (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, (unsigned)zero));
    const int t_e = wave * 64 + lane_e, i_e = lane_e & 31, hh_e = lane_e >> 5;
    const Item ie = PERSIST ? it : decode(w_cur, i_e, bm);

    // Split query block: publish this half's state (reference max, lane
    // partial row sum, accumulators, lane-major so each lane of the other
    // item reads back exactly its own row); the item that completes the
    // block's counter merges the other half into its registers and writes o.
    // The counter is read first: when the other half has already published
    // (counter 1), this item is the last one and skips publishing its own.
    // Otherwise it publishes, then counts itself in; whichever item's
    // increment finds 1 merges.  Every increment follows its item's completed
    // stores, so a counter of 1 means the other state is readable.
    bool write_out = true;
    if (!chunked && ie.part >= 0) {
      constexpr int PF_ = kFwdPartFloats(D);
      constexpr int NA = NDB * 16;  // accumulators per lane
      const int slot = ie.bh * p.n_split + (p.n_mblk - 1 - ie.pid_m);
      float* mine = p.part_ws + ((int64_t)slot * 2 + ie.part) * PF_;
      const float* other = p.part_ws + ((int64_t)slot * 2 + (1 - ie.part)) * PF_;
      if (t_e == 0) s_last = __hip_atomic_load(&p.part_cnt[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1;
      __syncthreads();
      bool last = s_last;
      if (!last) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int v = 0; v < 16; ++v) store_coherent(mine + (db * 16 + v) * kFwdThreads + t_e, acc[db][v]);
        store_coherent(mine + NA * kFwdThreads + t_e, m_run);
        store_coherent(mine + (NA + 1) * kFwdThreads + t_e, l_run);
        __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are done
        __syncthreads();
        if (t_e == 0) s_last = __hip_atomic_fetch_add(&p.part_cnt[slot], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1;
        __syncthreads();
        last = s_last;
      }
      __syncthreads();  // every wave has read s_last before the next item's writes it
      if (last) {
        // Both halves have arrived: leave the counter zero for the next call.
        if (t_e == 0) __hip_atomic_store(&p.part_cnt[slot], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // The merge is written in terms of the lower (0) and upper (1) half,
        // not of this item and the other one, so the rounding (fma
        // contraction included) does not depend on which half finished
        // last: repeated calls give identical outputs.
        const bool lo = ie.part == 0;
        const float m_o = load_coherent(other + NA * kFwdThreads + t_e);
        const float l_o = load_coherent(other + (NA + 1) * kFwdThreads + t_e);
        const float m0 = lo ? m_run : m_o, m1 = lo ? m_o : m_run;
        const float mm = fmaxf(m0, m1);
        const float mu = (mm == -__builtin_inff()) ? 0.f : mm;
        const float a0 = fast_exp2((m0 - mu) * c), a1 = fast_exp2((m1 - mu) * c);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const float x_o = load_coherent(other + (db * 16 + v) * kFwdThreads + t_e);
            const float x0 = lo ? acc[db][v] : x_o, x1 = lo ? x_o : acc[db][v];
            acc[db][v] = __builtin_fmaf(x0, a0, x1 * a1);
          }
        const float l0 = lo ? l_run : l_o, l1 = lo ? l_o : l_run;
        l_run = __builtin_fmaf(l0, a0, l1 * a1);
        m_run = mm;
      }
      write_out = last;
    }

    if constexpr (chunked) {
      // Key chunk: the partial state of this lane's row, as the split-KV
      // first pass stores it (m = m_ref * c in log2 units, relative to which
      // l and acc are kept; -inf with l = 0 for a row that saw no key in
      // this chunk; 0 for a sequence without keys, which the combine turns
      // into a zero row).  Lane (i, hh) holds dims 32 db + 8 j + 4 hh + 0..3
      // of its row in acc[db][4 j .. 4 j + 3].
      const float l_tot = xhalf_sum(l_run);
      if (ie.valid) {
        const int chunk = ie.tb / p.kv_chunk_tiles;
        const int64_t row = (((int64_t)ie.b * dm.Hq + ie.head) * dm.Sq + ie.pos) * p.kv_splits + chunk;
        float* wa = p.ws_acc + row * D + 4 * hh_e;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            *reinterpret_cast<f32x4*>(wa + 32 * db + 8 * j) =
                f32x4{acc[db][4 * j], acc[db][4 * j + 1], acc[db][4 * j + 2], acc[db][4 * j + 3]};
        if (hh_e == 0) {
          p.ws_m[row] = ie.skv == 0 ? 0.f : m_run * c;
          p.ws_l[row] = l_tot;
        }
      }
    } else if (write_out) {
      // Epilogue: o = acc / l (0/0 = NaN for a row whose keys are all
      // masked, as the reference's acc / l_i at gqa_fwd.py:106).  A sequence
      // with no keys at all gives zero rows instead: tests/reference.py:33-34
      // takes the softmax over an empty key axis and multiplies it with an
      // empty V.  Optional LSE side output: ln sum_k exp(s_k * D^-0.5) =
      // (m_ref * c + log2 l) * ln 2 (l is relative to the reference point
      // m_ref); -inf for a row with no visible key.
      const float l_tot = xhalf_sum(l_run);
      const float inv = ie.skv == 0 ? 0.f : 1.0f / l_tot;
      if (p.lse != nullptr && ie.valid && hh_e == 0) {
        // (B, Hq, Sq), or (tokens, Hq) with variable lengths.
        const int64_t li = varlen ? (ie.tok0 + ie.pos) * dm.Hq + ie.head
                                  : ((int64_t)ie.b * dm.Hq + ie.head) * dm.Sq + ie.pos;
        p.lse[li] = (m_run * c + __log2f(l_tot)) * kLn2;
      }
      {
        // The wave's 32 x D output tile goes through LDS (row-major, 16-byte
        // chunks XOR-swizzled by row; two waves per former K/V stage), so that
        // it leaves as whole rows: each store instruction writes 64 lanes x 16
        // bytes covering RPI complete rows, where storing straight from the
        // O^T accumulators would write 16 bytes into each of 32 rows per
        // instruction.
        constexpr int CPR16 = 2 * D / 16;  // 16-byte chunks per row
        constexpr int RPI = 64 / CPR16;    // rows per store instruction
        const int sw = wave >> 1;
        char* ot = (sw == 0 ? lds1_k0 : sw == 1 ? lds1_k1 : sw == 2 ? lds1_k2 : lds0_v0) + (wave & 1) * (32 * 2 * D);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            u32x2 x;
            x[0] = E::pack2(acc[db][4 * j] * inv, acc[db][4 * j + 1] * inv);
            x[1] = E::pack2(acc[db][4 * j + 2] * inv, acc[db][4 * j + 3] * inv);
            const int ch = (4 * db + j) ^ (i_e & (CPR16 - 1));
            *reinterpret_cast<u32x2*>(ot + i_e * (2 * D) + ch * 16 + 8 * hh_e) = x;
          }
        __builtin_amdgcn_s_waitcnt(kLgkm0);  // this wave's LDS writes before its reads
        const int cc = lane_e % CPR16;
#pragma unroll
        for (int ri = 0; ri < 32 / RPI; ++ri) {
          const int rr = RPI * ri + lane_e / CPR16;  // row of the tile
          const u32x4 x = *reinterpret_cast<const u32x4*>(ot + rr * (2 * D) + ((cc ^ (rr & (CPR16 - 1))) * 16));
          const int r2 = wave * 32 + rr;
          const int g2 = r2 / bm, pos2 = ie.pid_m * bm + (r2 - g2 * bm);
          if (g2 < dm.G && pos2 < ie.sq) {
            T* orow = static_cast<T*>(const_cast<void*>(p.o.ptr)) + row_off(ie, p.o, pos2, ie.kvh * dm.G + g2);
            *reinterpret_cast<u32x4*>(orow + 8 * cc) = x;
          }
        }
      }
    }
    if (dyn) {
      if (wave == 0) {
        int lo, n, S;
        xrange(xq, lo, n, S);
        int w = __builtin_amdgcn_readfirstlane(S + ticket < n ? lo + S + ticket : -1);
        // This XCD's queue is empty: lanes 1-7 read the other queues'
        // counters at once; the first one with items left is claimed (a
        // failed claim means that queue has just run out: counters only
        // grow, so at most 7 rounds).
        for (int round = 0; round < 8 && w < 0; ++round) {
          const int y = (xq + lane) & 7;
          int ly, ny, Sy;
          xrange(y, ly, ny, Sy);
          int left = 0;
          if (lane >= 1 && lane < 8 && Sy < ny)
            left = ny - Sy - __hip_atomic_load(&sched[y], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const uint64_t has = __builtin_amdgcn_ballot_w64(left > 0);
          if (has == 0) break;  // every queue is empty
          const int d = __builtin_ffsll((long long)has) - 1;
          const int yc = (xq + d) & 7;
          int lc, nc, Sc;
          xrange(yc, lc, nc, Sc);
          int tk = 0;
          if (lane == 0) tk = __hip_atomic_fetch_add(&sched[yc], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          tk = __builtin_amdgcn_readfirstlane(tk);
          if (Sc + tk < nc) w = lc + Sc + tk;
        }
        if (w < 0 && lane == 0) {
          // No work left: count out, in two levels so that the workgroups
          // ending together do not all queue on one counter: the S
          // workgroups of group g = blockIdx % 8, then the groups.  The
          // last workgroup out has seen every other workgroup's claims
          // complete: it clears the counters.
          const int g = blockIdx.x & 7;
          int lg, ng, Sg;
          xrange(g, lg, ng, Sg);
          const int dg = __hip_atomic_fetch_add(&sched[8 + g], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (dg == Sg - 1) {
            const int groups = min(n_wg, 8);
            const int dt = __hip_atomic_fetch_add(&sched[16], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (dt == groups - 1)
              for (int z = 0; z < 17; ++z) __hip_atomic_store(&sched[z], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
        if (lane == 0) s_next = w;
      }
      __syncthreads();
      w_next = s_next;
    }
    if (!PERSIST || w_next < 0) break;
    // Persistent: the next item's first tiles (once every wave's output has
    // left the stages) and Q, loaded while the output stores drain.
    __syncthreads();
    it = decode(w_next, i, p.block_m);
    blk_next = prologue_kv(it);
    prologue_q(it);
    ++k_item;
  }
}

template <int DT, int D, int PG>
static hipError_t launch_fwd_t(FwdParams p, hipStream_t stream) {
  const int per_bh = p.kv_splits > 0 ? p.n_mblk * p.kv_splits : p.n_mblk + p.n_split;
  const int total = per_bh * p.dm.Hkv * p.dm.B;
  if (total <= 0) return hipSuccess;
  int grid = total;
  if (PG == 0 && D == 128) {
    const int cus = device_cu_count();
    grid = cus > 0 ? std::min(total, cus) : total;
    p.n_wg = grid;
    // The dynamic schedule pays for its claims (atomic round trips of ~2 us,
    // and a tail of them as the last workgroups finish) only with many
    // items per workgroup: measured -0.5 to -1.1 % at 8 (16K-token
    // prefill), +1 to +3 % at 2-4 and +25 % at 1-2 (key-split short
    // prefill); below 8 the static snake schedule runs.
    if (total < kFwdDynMinItemsPerWg * grid) p.sched = nullptr;
  } else {
    p.sched = nullptr;
  }
  if (p.kv_splits > 0)
    hipLaunchKernelGGL((gqa_fwd_kernel<DT, D, PG, true>), dim3(grid), dim3(kFwdThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((gqa_fwd_kernel<DT, D, PG>), dim3(grid), dim3(kFwdThreads), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_fwd(const FwdParams& p, int dtype, hipStream_t stream) {
  if (dtype == 0)
    return p.dm.D == 128 ? launch_fwd_t<0, 128, 0>(p, stream) : launch_fwd_t<0, 64, 0>(p, stream);
  return p.dm.D == 128 ? launch_fwd_t<1, 128, 0>(p, stream) : launch_fwd_t<1, 64, 0>(p, stream);
}

template <int PG>
static hipError_t launch_paged_fwd_t(const FwdParams& p, int dtype, hipStream_t stream) {
  if (dtype == 0)
    return p.dm.D == 128 ? launch_fwd_t<0, 128, PG>(p, stream) : launch_fwd_t<0, 64, PG>(p, stream);
  return p.dm.D == 128 ? launch_fwd_t<1, 128, PG>(p, stream) : launch_fwd_t<1, 64, PG>(p, stream);
}

// Requires block_size >= 512 / D, the rows of one LDS-DMA instruction
// (pages of >= 64 keys hold whole tiles, of 16-32 keys whole 16-row wave
// shares of a tile, smaller ones whole instructions).  The 16-32-key form at
// D = 64 derives its K offsets by an XOR of bit 5 and so takes row strides
// of a multiple of 64 bytes; other strides take the per-instruction form,
// which serves any page of >= 8 keys there.
hipError_t launch_paged_fwd(const FwdParams& p, int dtype, hipStream_t stream) {
  if ((1 << p.block_shift) < 512 / p.dm.D) return hipErrorInvalidValue;
  if (p.block_shift >= 6) return launch_paged_fwd_t<1>(p, dtype, stream);
  const bool medium = p.block_shift >= 4 && (p.dm.D != 64 || (2 * p.k.ss) % 64 == 0);
  return medium ? launch_paged_fwd_t<3>(p, dtype, stream) : launch_paged_fwd_t<2>(p, dtype, stream);
}

}  // namespace gqa
