// gqa_decode.hip — split-KV first pass for short query blocks (decode) at
// head_dim 128 over contiguous K/V, with an optional fused combine.
//
// Replaces, for these shapes, the Triton gqa_split_first_kernel (reference
// gqa_kernels/gqa_split.py:26-112) and, when fused, gqa_split_reduce_kernel
// (gqa_split.py:115-147).  The work decomposition, the packed rows and the
// partials are those of gqa_split.hip: one workgroup per (batch, kv head,
// row block of 32 or 64 rows, split), rows packed position-major (row r -> position r / G,
// head r % G), partials (m in log2 units, l, unnormalised acc) per (row,
// split) in the same workspace layout.
//
// Streaming: the chunk's keys arrive in 64-key K and V tiles written
// straight into LDS by buffer loads in their LDS-DMA form (no staging
// registers, no VALU transposes), through a ring of two stages; a stage is
// refilled with the tile two ahead as soon as every wave has read it, so one
// to two tiles stay in flight per workgroup (two workgroups per CU).  V is
// read transposed by ds_read_b64_tr_b16 (the single-pass kernel's layout,
// gqa_lds.hpp).
//
// The 4 waves of a workgroup split the keys and the head dimension.  RW = 1
// (one 32-row block): waves 2k + h take keys [32k, 32k + 32) of every
// 64-key tile (key group k) and dims [64h, 64h + 64), each running its own
// exact online softmax over its keys; RW = 2 (33-64 packed rows per kv
// head, e.g. verify steps of 9-16 tokens at G = 4): waves 2r + k take rows
// [32r, 32r + 32) of the block, key group k, all 128 dims; RW = 4 (65-128
// rows): wave r takes rows [32r, 32r + 32), all keys and dims.  At the end
// of the chunk key group 1 hands its state to key group 0 through LDS,
// which merges the two as the combine merges two splits and stores the
// valid rows' partials of its dims.  (Splitting only the dims made every
// wave of a row block compute the same scores and probabilities: 2 % more
// time on the 70B decode shape.)  With a decode group of 4 query rows most
// of each S^T MFMA is padding; it runs hidden under the HBM stream.
//
// Wide row blocks (RW = 2 or 4) stream the chunk's K/V once instead of once
// per 32-row block.  Partials and the fused combine stay per 32-row block.
//
// Fused combine (SplitParams::counters set): the last workgroup of each
// (b, kv head, row block) to count its partial in combines all splits
// (gqa_split.py:134-147) with one round of global loads — m and l of every
// (row, split) and this thread's accumulators are requested together.
#include <type_traits>

#include "gqa_common.hpp"
#include "gqa_lds.hpp"
#include "gqa_params.hpp"

namespace gqa {

namespace {

constexpr int kDecD = 128;
constexpr int kDecTileBytes = FwdStage<kDecD>::kTileBytes;  // one 64-key K or V tile: 16 KiB
// Splits one combining thread requests per round (16-byte loads in flight).
constexpr int kDecBatch = 32;
// (row, split) pairs of m and l one combining thread loads (R * S <= 4096).
constexpr int kDecMlPerThread = kFusedMaxRowSplitsHost / 256;
static_assert(kFusedMaxRowSplitsHost * 4 <= kDecTileBytes, "m (or l) of the fused combine fits one LDS stage");
static_assert(256 * 16 <= kDecTileBytes && 32 * (kDecD / 4) * 16 <= kDecTileBytes,
              "the fused combine's split-group sums fit one LDS stage");

// 16-byte device-coherent store (sc1: written through to the point where
// all XCDs are coherent), through a buffer descriptor over the workspace.
__device__ inline void store_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), r, off, 0, 16);
}

// Fused log-sum-exp combine of the R valid rows of one (b, kv head, 32-row
// block) over all S splits (gqa_split.py:134-147), by one workgroup:
//   1. m and l of every (row, split), and the accumulators of this thread's
//      first kDecBatch splits, are requested in one round; m and l go to
//      LDS; per row (one wave, lanes over the splits) m* = max m, a = exp2(m
//      - m*), l* = sum a * l;
//   2. thread (split group sg, row, 4 columns) sums a * acc over splits sg,
//      sg + nsg, ... (further rounds only beyond kDecBatch splits), the
//      split groups are added in order in LDS, o = sum / l*.
// Rows whose chunks are all empty give NaN (m* = -inf), as the reference's
// combine; a sequence without keys (every split stores m = 0, l = 0) gives
// zeros.  LDS: ma and la hold R * S floats each, rowst 64 floats, red
// nsg * R * D / 4 f32x4 (at most 16 KiB: nsg * R * D / 4 <= max(256, R * D / 4)).
template <int DT>
__device__ void decode_combine(const SplitParams& p, int b, int kvh, int rb, int t, float* ma, float* la,
                               float* rowst, f32x4* red) {
  using E = Elem<DT>;
  using T = typename E::T;
  constexpr int D = kDecD, NDP = D / 4;
  const Dims& dm = p.dm;
  const int S = p.splits;
  const int r0 = 32 * rb;
  const int R = min(32, dm.G * dm.Sq - r0);
  const int lane = t & 63, wave = t >> 6;
  // ma [R][S]: m, then the scale factors a; la [R][S]: l.
  float* mst = rowst;       // [32]: m* per row
  float* lst = rowst + 32;  // [32]: l* per row

  auto row_index = [&](int rl) -> int64_t {  // workspace row of split 0
    const int r = r0 + rl;
    const int pos = r / dm.G, g = r - pos * dm.G;
    return (((int64_t)b * dm.Hq + kvh * dm.G + g) * dm.Sq + pos) * S;
  };
  const int items = R * NDP;
  const int nsg = items >= 256 ? 1 : max(1, min(S, 256 / items));
  const int n_work = items * nsg;
  // 16-byte loads through a descriptor over the whole acc workspace (the
  // host bounds its size to 32-bit offsets).
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.ws_acc, 0xFFFFFFF0u);

  // Step 1: m and l into registers, then this thread's first batch of
  // accumulators, all in flight together.
  float mreg[kDecMlPerThread], lreg[kDecMlPerThread];
#pragma unroll
  for (int k = 0; k < kDecMlPerThread; ++k) {
    const int f = t + 256 * k;
    if (f < R * S) {
      const int rl = f / S, sp = f - rl * S;
      const int64_t ix = row_index(rl) + sp;
      mreg[k] = load_coherent(p.ws_m + ix);
      lreg[k] = load_coherent(p.ws_l + ix);
    }
  }
  f32x4 buf[kDecBatch];
  int it = t;
  int item = it % items, sg = it / items;
  int rl = item / NDP, d4 = item - rl * NDP;
  uint32_t base = (uint32_t)((row_index(rl) * D + 4 * d4) * 4);
  if (it < n_work) {
#pragma unroll
    for (int k = 0; k < kDecBatch; ++k) {
      const int sp = sg + k * nsg;
      if (sp < S) buf[k] = load_coherent4(ra, base + (uint32_t)sp * (D * 4));
    }
  }
#pragma unroll
  for (int k = 0; k < kDecMlPerThread; ++k) {
    const int f = t + 256 * k;
    if (f < R * S) {
      ma[f] = mreg[k];
      la[f] = lreg[k];
    }
  }
  __syncthreads();
  for (int rr = wave; rr < R; rr += 4) {
    float m = -__builtin_inff();
    for (int sp = lane; sp < S; sp += 64) m = fmaxf(m, ma[rr * S + sp]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    // exp2(-inf - -inf) = NaN when every chunk of a row is empty, as the
    // reference's combine (gqa_split.py:138) gives.
    float l = 0.f;
    for (int sp = lane; sp < S; sp += 64) {
      const float a = fast_exp2(ma[rr * S + sp] - m);
      ma[rr * S + sp] = a;
      l += a * la[rr * S + sp];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off, 64);
    if (lane == 0) {
      mst[rr] = m;
      lst[rr] = l;
      // LSE of a row with no visible key is -inf (its o stays NaN).
      if (p.lse != nullptr)
        p.lse[row_index(rr) / S] = m == -__builtin_inff() ? -__builtin_inff() : (m + __log2f(l)) * kLn2;
    }
  }
  __syncthreads();

  // Step 2 (more load batches only past kDecBatch splits per thread): a * acc.
  for (bool first = true; it < n_work; it += 256, first = false) {
    if (!first) {
      item = it % items;
      sg = it / items;
      rl = item / NDP;
      d4 = item - rl * NDP;
      base = (uint32_t)((row_index(rl) * D + 4 * d4) * 4);
    }
    const float* a = ma + rl * S;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = sg; s0 < S; s0 += kDecBatch * nsg) {
      if (!(first && s0 == sg)) {
#pragma unroll
        for (int k = 0; k < kDecBatch; ++k) {
          const int sp = s0 + k * nsg;
          if (sp < S) buf[k] = load_coherent4(ra, base + (uint32_t)sp * (D * 4));
        }
      }
#pragma unroll
      for (int k = 0; k < kDecBatch; ++k) {
        const int sp = s0 + k * nsg;
        if (sp < S) o += a[sp] * buf[k];
      }
    }
    red[it] = o;  // [sg][item]: it = sg * items + item
  }
  __syncthreads();
  for (int f = t; f < items; f += 256) {
    const int rl2 = f / NDP, d42 = f - (f / NDP) * NDP;
    f32x4 o = red[f];
    for (int g2 = 1; g2 < nsg; ++g2) o += red[g2 * items + f];
    // A sequence without keys (finite m*, l* = 0, o = 0): 0 / inf = 0.
    const float l = (lst[rl2] == 0.f && mst[rl2] > -__builtin_inff()) ? __builtin_inff() : lst[rl2];
    const int r = r0 + rl2;
    const int pos = r / dm.G, g = r - pos * dm.G;
    T* orow = static_cast<T*>(const_cast<void*>(p.o.ptr)) + (int64_t)b * p.o.sb +
              (int64_t)(kvh * dm.G + g) * p.o.sh + (int64_t)pos * p.o.ss + 4 * d42;
    u32x2 x;
    x[0] = E::pack2(o[0] / l, o[1] / l);
    x[1] = E::pack2(o[2] / l, o[3] / l);
    *reinterpret_cast<u32x2*>(orow) = x;
  }
}

}  // namespace

// KV: 0 contiguous K/V; 1 a paged cache with pages of >= 64 keys (one
// buffer descriptor per 64-key tile, from the block table); 3 pages of
// 16-32 keys (one descriptor per wave and tile: each wave loads 16
// consecutive rows); 2 pages of 4-8 keys (one descriptor per LDS-DMA
// instruction, whose 4 rows lie in one page).  Paged caches are
// (num_blocks, block_size, Hkv, D) in any strides
// (SplitParams::k/v: sb = block, ss = slot, sh = head stride); sequence b has
// min(seq_lens[b], Skv) keys.  With q_start / q_len set, q is token-major and
// sequence b has q_len[b] query rows from token q_start[b].
// RW: 32-row blocks per workgroup (1, 2 or 4).
template <int DT, int KV, int RW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gqa_decode_kernel(SplitParams p) {
  constexpr int D = kDecD;
  constexpr bool PAGED = KV != 0;
  using E = Elem<DT>;
  using ST = FwdStage<D>;
  constexpr int CPR = ST::CPR;
  constexpr int NKS = D / 16;  // k-steps of S^T
  constexpr int NI = ST::NI;   // LDS-DMA instructions per wave per K (or V) tile
  // Four separate arrays (K and V of two stages), not one: the compiler can
  // then tell the LDS-DMA target of the tile in flight from the stage being
  // read and does not wait for those loads before the reads.  The fused
  // combine reuses them, each region inside one array (m and l of up to
  // kFusedMaxRowSplitsHost (row, split) pairs take one 16 KiB array each).
  __shared__ __attribute__((aligned(1024))) char lds_a_k0[kDecTileBytes];
  __shared__ __attribute__((aligned(1024))) char lds_b_v0[kDecTileBytes];
  __shared__ __attribute__((aligned(1024))) char lds_c_k1[kDecTileBytes];
  __shared__ __attribute__((aligned(1024))) char lds_d_v1[kDecTileBytes];
  __shared__ int s_last;

  const Dims& dm = p.dm;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6) & 3;
  const int i = lane & 31, hh = lane >> 5;
  // This wave's 32-row block within the workgroup's (rh), its key group kh
  // and its NDB 32-dim blocks of O^T from db0.  The WPR waves of a row block
  // are KS key groups (each takes 64 / KS keys of every tile with its own
  // online softmax state; the groups' states are merged in LDS after the
  // chunk) times DS dim groups: RW = 1, two key groups x two dim groups of
  // 64 dims; RW = 2, two key groups of all 128 dims; RW = 4, one wave with
  // all 128 dims.  Splitting the keys instead of only the dims spares the
  // waves of a row block computing the same scores and probabilities twice.
  constexpr int WPR = 4 / RW;  // waves per 32-row block
  constexpr int KS = WPR >= 2 ? 2 : 1;
  constexpr int DS = WPR / KS;
  constexpr int NDB = 4 / DS;
  constexpr int NMB = 2 / KS;  // 32-key blocks of a tile per wave
  const int rh = wave / WPR;
  const int kh = (wave % WPR) % KS;
  const int db0 = ((wave % WPR) / KS) * NDB;

  const int n_wblk = (p.n_rblk + RW - 1) / RW;
  const int total = dm.B * dm.Hkv * n_wblk * p.splits;
  const int w = xcd_remap(blockIdx.x, total);
  const int s = w % p.splits;
  int rest = w / p.splits;
  const int rbw = rest % n_wblk;
  rest /= n_wblk;
  const int kvh = rest % dm.Hkv;
  const int b = rest / dm.Hkv;
  const int rb = RW * rbw + rh;  // this wave's 32-row block
  // Keys of this sequence (paged: its own length, clamped to [0, Skv], so no
  // key past the block table's covered range is addressed) and its query
  // rows (variable lengths: q_len[b] rows from token q_start[b]).
  const int skv = PAGED ? min(max(load_uniform(p.seq_lens + b), 0), dm.Skv) : dm.Skv;
  const bool varlen = p.q_len != nullptr;
  const int sq = varlen ? min(max(load_uniform(p.q_len + b), 0), dm.Sq) : dm.Sq;
  const int64_t tok0 = varlen ? (int64_t)load_uniform(p.q_start + b) : 0;
  const int wr0 = 32 * RW * rbw;        // the workgroup's first packed row
  if (wr0 / dm.G >= sq) return;          // a row block past this sequence's queries

  // This lane's query row (position-major packing).
  const int r = 32 * rb + i;
  const int pos = r / dm.G, g = r - pos * dm.G;
  const bool valid = pos < sq;
  const int head = kvh * dm.G + g;
  const int qpos = pos + (skv - sq);

  // Keys of this chunk (gqa_split.py:55-60), clamped to the block's last
  // visible key under causal.
  const int c0 = s * p.chunk;
  int c1 = min(c0 + p.chunk, skv);
  const int pos_lo = wr0 / dm.G;
  const int pos_hi = min(sq - 1, (wr0 + 32 * RW - 1) / dm.G);
  if (dm.causal) c1 = min(c1, pos_hi + (skv - sq) + 1);
  const int nk = max(c1 - c0, 0);
  const int ntiles = (nk + 63) >> 6;
  const int qpos_lo = pos_lo + (skv - sq);

  // Contiguous K/V: buffer descriptors over the chunk's K and V rows, each
  // ending at the chunk's last key: rows of a partial last tile past it read
  // as zero (and are masked).  The host bounds (chunk + 64) * row stride to
  // 31 bits.  Paged: descriptors per tile or per instruction (issue).
  const uint32_t kssb = (uint32_t)(2 * p.k.ss), vssb = (uint32_t)(2 * p.v.ss);
  const char* kbase = static_cast<const char*>(p.k.ptr) +
                      2 * ((PAGED ? 0 : (int64_t)b * p.k.sb + (int64_t)c0 * p.k.ss) + (int64_t)kvh * p.k.sh);
  const char* vbase = static_cast<const char*>(p.v.ptr) +
                      2 * ((PAGED ? 0 : (int64_t)b * p.v.sb + (int64_t)c0 * p.v.ss) + (int64_t)kvh * p.v.sh);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, !PAGED && nk > 0 ? (uint32_t)(nk - 1) * kssb + 2 * D : 0u);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase, !PAGED && nk > 0 ? (uint32_t)(nk - 1) * vssb + 2 * D : 0u);
  const int* table_row = PAGED ? p.block_table + (int64_t)b * p.table_stride : nullptr;

  // Tile order.  With one head's keys in consecutive rows, every workgroup
  // would otherwise stream its chunk from the same relative offset in lock
  // step with the others, concentrating the concurrent reads on a subset of
  // the HBM channels; splits s = 0..3 (mod 4) start a quarter of the chunk
  // apart.  The online softmax does not depend on the order.
  // Tiles past the chunk (the prologue's tiles of a chunk shorter than two,
  // the padding of an odd count) are not rotated: they lie beyond the
  // descriptors, read as zero and are fully masked.
  const int rot = (p.rotate && ntiles >= 4) ? (s & 3) * (ntiles >> 2) : 0;
  auto tile_rel = [&](int it) {
    const int j = it + rot;
    return it >= ntiles ? it : (j >= ntiles ? j - ntiles : j);
  };

  // LDS-DMA source offsets of this lane (its row within an instruction's 4
  // rows, its swizzled chunk), as the single pass.
  const int lrow = lane / CPR;
  const uint32_t koff =
      (uint32_t)(lrow * kssb) + 16u * (uint32_t)((lane % CPR) ^ ST::gk((wave * ST::RPI + lrow) & 15));
  const uint32_t voff = (uint32_t)(lrow * vssb) + 16u * (uint32_t)((lane % CPR) ^ ST::sv(lrow));
  // The prologue issues tiles 0 and 1 unconditionally (a tile past the
  // chunk reads zeros); the loop issues a tile only if it exists.
  auto issue = [&](int it, char* kst, char* vst) {
    const int j = tile_rel(it) * 64;
    if constexpr (KV == 0) {
      issue_tile_dma<D, kDmaStream>(kst, rk, (uint32_t)j * kssb, kssb, koff, wave);
      issue_tile_dma<D, kDmaStream>(vst, rv, (uint32_t)j * vssb, vssb, voff, wave);
    } else if constexpr (KV == 1) {
      // The tile's 64 rows are one strided run inside one page; its
      // descriptors start at the tile's first row and end at the chunk's
      // last key (a tile past the chunk reads no table entry: zeros).
      const int key0 = c0 + j, rows = c1 - key0;
      __amdgpu_buffer_rsrc_t tk = make_rsrc(kbase, 0u), tv = make_rsrc(vbase, 0u);
      if (rows > 0) {
        const int64_t pg = load_uniform(table_row + (key0 >> p.block_shift));
        const int64_t slot = key0 & ((1 << p.block_shift) - 1);
        const uint32_t n = (uint32_t)(min(rows, 64) - 1);
        tk = make_rsrc(kbase + 2 * (pg * p.k.sb + slot * p.k.ss), n * kssb + 2 * D);
        tv = make_rsrc(vbase + 2 * (pg * p.v.sb + slot * p.v.ss), n * vssb + 2 * D);
      }
      issue_tile_dma<D, kDmaStream>(kst, tk, 0u, kssb, koff, wave);
      issue_tile_dma<D, kDmaStream>(vst, tv, 0u, vssb, voff, wave);
    } else if constexpr (KV == 3) {
      // Pages of 16-32 keys: this wave loads rows [key, key + 16) of the
      // tile, one run in one page (one table read, one descriptor each for K
      // and V); instruction jj takes rows key + 4 jj + 0..3 (scalar offset)
      // into LDS rows 16 wave + 4 jj + ...  K's swizzle is linear in the row
      // bits: chunk (lane % CPR) ^ gk(lrow) ^ gk(4 jj); V's depends on lrow.
      typedef __attribute__((address_space(3))) void lds_void;
      const int key = c0 + j + 16 * wave, rows = c1 - key;
      __amdgpu_buffer_rsrc_t tk = make_rsrc(kbase, 0u), tv = make_rsrc(vbase, 0u);
      if (rows > 0) {
        const int64_t pg = load_uniform(table_row + (key >> p.block_shift));
        const int64_t slot = key & ((1 << p.block_shift) - 1);
        const uint32_t n = (uint32_t)(min(rows, 16) - 1);
        tk = make_rsrc(kbase + 2 * (pg * p.k.sb + slot * p.k.ss), n * kssb + 2 * D);
        tv = make_rsrc(vbase + 2 * (pg * p.v.sb + slot * p.v.ss), n * vssb + 2 * D);
      }
#pragma unroll
      for (int jj = 0; jj < NI; ++jj) {
        const uint32_t ko = (uint32_t)(lrow * kssb) +
                            16u * (uint32_t)((lane % CPR) ^ ST::gk(lrow) ^ ST::gk(jj * ST::RPI));
        __builtin_amdgcn_raw_ptr_buffer_load_lds(tk, (lds_void*)(kst + (wave * NI + jj) * 1024), 16, ko,
                                                 (uint32_t)(jj * ST::RPI) * kssb, 0, kDmaStream);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(tv, (lds_void*)(vst + (wave * NI + jj) * 1024), 16, voff,
                                                 (uint32_t)(jj * ST::RPI) * vssb, 0, kDmaStream);
      }
    } else {
      // Pages of 4-8 keys: instruction `step` loads rows [key, key + 4) of
      // the tile, one run in one page; each gets its own descriptors.
      typedef __attribute__((address_space(3))) void lds_void;
#pragma unroll
      for (int jj = 0; jj < NI; ++jj) {
        const int step = jj * 4 + wave;
        const int key = c0 + j + step * ST::RPI, rows = c1 - key;
        __amdgpu_buffer_rsrc_t tk = make_rsrc(kbase, 0u), tv = make_rsrc(vbase, 0u);
        if (rows > 0) {
          const int64_t pg = load_uniform(table_row + (key >> p.block_shift));
          const int64_t slot = key & ((1 << p.block_shift) - 1);
          const uint32_t n = (uint32_t)(min(rows, ST::RPI) - 1);
          tk = make_rsrc(kbase + 2 * (pg * p.k.sb + slot * p.k.ss), n * kssb + 2 * D);
          tv = make_rsrc(vbase + 2 * (pg * p.v.sb + slot * p.v.ss), n * vssb + 2 * D);
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(tk, (lds_void*)(kst + step * 1024), 16, koff, 0, 0, kDmaStream);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(tv, (lds_void*)(vst + step * 1024), 16, voff, 0, 0, kDmaStream);
      }
    }
  };

  // Loads in issue order: tile 0, Q, tile 1 (the wait for tile 0 and Q then
  // leaves tile 1 in flight).  Only lanes of valid rows load Q (a decode
  // step has 4 of 32): the others would re-request the same rows from L2 in
  // every wave of every workgroup, beside the K/V stream.
  // (Through a descriptor over this kv head's query group: an invalid
  // lane's offset lies past its end and reads zero without a memory access,
  // and no branch splits the wave.)
  issue(0, lds_a_k0, lds_b_v0);
  u32x4 qreg[NKS];
  {
    const char* qg = static_cast<const char*>(p.q.ptr) +
                     2 * ((varlen ? tok0 * p.q.ss : (int64_t)b * p.q.sb) + (int64_t)kvh * dm.G * p.q.sh);
    const uint32_t qext = (uint32_t)(2 * ((int64_t)(dm.G - 1) * p.q.sh + (int64_t)(sq - 1) * p.q.ss + D));
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(qg, qext);
    const uint32_t qo = valid ? (uint32_t)(2 * ((int64_t)g * p.q.sh + (int64_t)pos * p.q.ss) + 16 * hh) : 0x80000000u;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
      qreg[ks] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, qo + 32u * ks, 0, 0));
  }
  issue(1, lds_c_k1, lds_d_v1);
  // Tile 0 and Q have landed (tile 1 may still be in flight).  Waiting here,
  // explicitly, also settles Q for the compiler: otherwise it waits for
  // every load in flight before entering the tile loop.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * NI));

  // LDS read offsets: S^T A operand (K rows pi(i)), V^T A operand of this
  // wave's dims (transposing reads), as the single pass.
  constexpr uint32_t kKMask = (kDecTileBytes / 2 - 1) & ~15u;
  constexpr uint32_t kVMask = (kDecTileBytes - 1) & ~7u;
  uint32_t ka[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks)
    ka[ks] = (uint32_t)(pi_key(i) * (2 * D) + 16 * ((2 * ks + hh) ^ ST::gk(pi_key(i)))) & kKMask;
  uint32_t vb[NDB];
  {
    const int q = lane >> 4, ii = lane & 15;
    const int rowl = 8 * (q >> 1) + (ii >> 2);
    const int f = ii >> 2;  // sv(rowl) / 4
#pragma unroll
    for (int d = 0; d < NDB; ++d)
      vb[d] = (uint32_t)(rowl * (2 * D) + 16 * (4 * ((db0 + d) ^ f) + 2 * (q & 1) + ((ii & 3) >> 1)) + 8 * (ii & 1)) &
              kVMask;
  }

  f32x16 acc[NDB] = {};
  float m_run = -__builtin_inff(), l_run = 0.f;
  const float c = dm.c;

  // Issue priority falls with progress (3 for the first quarter of the
  // chunk, then 2, 1, 0): two workgroups share a compute unit, and ranking
  // by progress keeps them within a quarter of each other instead of the
  // older one streaming ahead and the younger one finishing alone.
  auto set_prio = [&](int it) {
    const int lvl = (4 * it) / ntiles;
    if (lvl == 0) __builtin_amdgcn_s_setprio(3);
    else if (lvl == 1) __builtin_amdgcn_s_setprio(2);
    else if (lvl == 2) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
  };

  // One 64-key tile from stage S3 (tile it of this chunk's order); with
  // ISSUE, the stage is then refilled with tile it + 2; LAST: no tile is in
  // flight behind this one.  Both are compile-time decisions: a run-time
  // condition around the issue makes the compiler's own wait tracking merge
  // the two paths and wait for every load in flight before the next LDS
  // reads.
  auto step = [&](auto s3, auto issue_c, auto last_c, int it) {
    constexpr int S3 = decltype(s3)::value;
    constexpr bool ISSUE = decltype(issue_c)::value;
    constexpr bool LAST = decltype(last_c)::value;
    char* kst = S3 == 0 ? lds_a_k0 : lds_c_k1;
    char* vst = S3 == 0 ? lds_b_v0 : lds_d_v1;
    const char* ck = kst;
    const char* cv = vst;
    if ((it & 3) == 0) set_prio(it);
    // This wave's loads of tile it have landed (those of tile it + 1 may
    // still be in flight); after the barrier, every wave's have.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(LAST ? 0 : 2 * NI));
    phase_barrier();

    // S^T for this wave's keys of the tile: NMB 32-key blocks (blocks
    // kh * NMB + mb of the tile), NKS k-steps each.
    f32x16 sc[NMB] = {};
    {
      u32x4 opk[NMB * NKS];
#pragma unroll
      for (int j = 0; j < NMB * NKS; ++j)
        opk[j] = *reinterpret_cast<const u32x4*>(ck + (kh * NMB + j % NMB) * 32 * (2 * D) + ka[j / NMB]);
#pragma unroll
      for (int j = 0; j < NMB * NKS; ++j) sc[j % NMB] = E::mfma(opk[j], qreg[j / NMB], sc[j % NMB]);
    }
    const int key0 = c0 + tile_rel(it) * 64;
    const bool need_mask = (key0 + 64 > c1) || (dm.causal && key0 + 63 > qpos_lo);
    if (need_mask) {
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = key0 + 32 * (kh * NMB + mb) + key_of(v, hh);
          const bool off = key >= c1 || (dm.causal && key > qpos);
          sc[mb][v] = off ? -__builtin_inff() : sc[mb][v];
        }
    }
    // Exact online softmax (gqa_split.py:92-101) in exp2 units; a row with
    // no visible key so far keeps m = -inf and uses 0 as reference, so its
    // probabilities are 0, never NaN.
    float mx;
    if constexpr (NMB == 2) {
      float m1[11];
#pragma unroll
      for (int k = 0; k < 10; ++k) {
        const int i0 = 3 * k, i1 = 3 * k + 1, i2 = 3 * k + 2;
        m1[k] = vmax3(sc[i0 >> 4][i0 & 15], sc[i1 >> 4][i1 & 15], sc[i2 >> 4][i2 & 15]);
      }
      m1[10] = vmax3(sc[NMB - 1][14], sc[NMB - 1][15], sc[NMB - 1][15]);
      const float n0 = vmax3(m1[0], m1[1], m1[2]), n1 = vmax3(m1[3], m1[4], m1[5]);
      const float n2 = vmax3(m1[6], m1[7], m1[8]), n3 = vmax3(m1[9], m1[10], m1[10]);
      mx = xhalf_max(vmax3(vmax3(n0, n1, n2), n3, n3));
    } else {
      float m1[5];
#pragma unroll
      for (int k = 0; k < 5; ++k) m1[k] = vmax3(sc[0][3 * k], sc[0][3 * k + 1], sc[0][3 * k + 2]);
      mx = xhalf_max(vmax3(vmax3(m1[0], m1[1], m1[2]), vmax3(m1[3], m1[4], sc[0][15]), sc[0][15]));
    }
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
    const float alpha = fast_exp2((m_run - m_use) * c);
    const float nmc = -m_use * c;
    u32x4 pk[NMB][2];
    float rs = 0.f;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      float pv[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) pv[v] = fast_exp2(__builtin_fmaf(sc[mb][v], c, nmc));
      float s8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) s8[j] = pv[2 * j] + pv[2 * j + 1];
      rs += ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int e = 0; e < 4; ++e) pk[mb][kk][e] = E::pack2(pv[8 * kk + 2 * e], pv[8 * kk + 2 * e + 1]);
    }
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int d = 0; d < NDB; ++d)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[d][v] *= alpha;

    // O^T (this wave's dims) += V^T P^T over this wave's keys.
#pragma unroll
    for (int d = 0; d < NDB; ++d)
#pragma unroll
      for (int j = 0; j < 2 * NMB; ++j) {
        const int mb = j >> 1, kk = j & 1;
        const int ro = (32 * (kh * NMB + mb) + 16 * kk) * (2 * D);
        const u32x2 lo = ld_tr(cv + vb[d] + ro);
        const u32x2 hi = ld_tr(cv + vb[d] + ro + 4 * (2 * D));
        acc[d] = E::mfma(u32x4{lo[0], lo[1], hi[0], hi[1]}, pk[mb][kk], acc[d]);
      }
    // Every wave is done with this stage: refill it with the tile two ahead.
    phase_barrier();
    if constexpr (ISSUE) issue(it + 2, kst, vst);
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using BT = std::true_type;
  using BF = std::false_type;
  // Tiles in pairs (stage 0, stage 1); an odd count is padded with one tile
  // past the chunk (zeros, every key masked: it adds nothing).
  const int ne = (ntiles + 1) & ~1;
  int it = 0;
  for (; it + 4 <= ne; it += 2) {
    step(I0{}, BT{}, BF{}, it);
    step(I1{}, BT{}, BF{}, it + 1);
  }
  if (it < ne) {
    step(I0{}, BF{}, BF{}, it);
    step(I1{}, BF{}, BT{}, it + 1);
  }
  __builtin_amdgcn_s_setprio(0);
  // Nothing is left in flight (an empty chunk still issued the prologue's
  // two tiles of zeros) before the workgroup exits or the combine reuses the
  // stages.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  if constexpr (KS == 2) {
    // Key group 1 hands its state (the same lanes' rows and dims) to key
    // group 0 through LDS, lane-major; group 0 merges it as the combine
    // merges two splits (gqa_split.py:137-144), a group with no visible key
    // (m = -inf, l = 0, acc = 0) adding nothing.  Pair (row block, dim
    // group) g uses stage arrays 2 g (accumulators, NDB * 4 KiB) and 2 g + 1
    // (m, l).
    const int pair = wave / KS;
    float* xa = reinterpret_cast<float*>(pair == 0 ? lds_a_k0 : lds_c_k1);
    float* xm = reinterpret_cast<float*>(pair == 0 ? lds_b_v0 : lds_d_v1);
    __syncthreads();  // every wave is done with the stages
    if (kh == 1) {
#pragma unroll
      for (int d = 0; d < NDB; ++d)
#pragma unroll
        for (int v = 0; v < 16; ++v) xa[(d * 16 + v) * 64 + lane] = acc[d][v];
      xm[lane] = m_run;
      xm[64 + lane] = l_run;
    }
    __syncthreads();
    if (kh == 0) {
      const float m1 = xm[lane], l1 = xm[64 + lane];
      const float mm = fmaxf(m_run, m1);
      const float mu = (mm == -__builtin_inff()) ? 0.f : mm;
      const float a0 = fast_exp2((m_run - mu) * c), a1 = fast_exp2((m1 - mu) * c);
#pragma unroll
      for (int d = 0; d < NDB; ++d)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[d][v] = __builtin_fmaf(acc[d][v], a0, xa[(d * 16 + v) * 64 + lane] * a1);
      l_run = __builtin_fmaf(l_run, a0, l1 * a1);
      m_run = mm;
    }
    __syncthreads();  // the stages are free again (the fused combine reuses them)
  }

  // This wave's dims of the valid rows' partials: lane (i, hh) holds dims
  // 32 * (db0 + d) + 8 * j + 4 * hh + 0..3 in acc[d][4j .. 4j + 3].  With
  // two key groups, group 0 holds the merged state.
  const float l_tot = xhalf_sum(l_run);
  if (valid && kh == 0) {
    const int64_t row = (((int64_t)b * dm.Hq + head) * dm.Sq + pos) * p.splits + s;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.ws_acc, 0xFFFFFFF0u);
#pragma unroll
    for (int d = 0; d < NDB; ++d) {
      const uint32_t ob = (uint32_t)((row * D + 32 * (db0 + d) + 4 * hh) * 4);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        store_coherent4(rw, ob + 32u * j,
                        f32x4{acc[d][4 * j], acc[d][4 * j + 1], acc[d][4 * j + 2], acc[d][4 * j + 3]});
    }
    // A sequence without keys stores m = 0, l = 0 (never produced otherwise:
    // the chunk's largest score contributes exp2(0) = 1 to l), which the
    // combine turns into a zero row.  One wave per row half stores them.
    if (db0 == 0 && hh == 0) {
      store_coherent(p.ws_m + row, skv == 0 ? 0.f : m_run * c);
      store_coherent(p.ws_l + row, l_tot);
    }
  }

  if (PAGED || p.counters == nullptr) return;
  // Fused combine: count this partial once its stores have completed; the
  // workgroup completing the count for this (b, kv head, row block) combines
  // (a wide block counts on its first 32-row block's counter and combines
  // both).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    const int idx = (b * dm.Hkv + kvh) * p.n_rblk + RW * rbw;
    const int prev = __hip_atomic_fetch_add(&p.counters[idx], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == p.splits - 1);
    // Every increment of this call has landed: leave the counter zero.
    if (s_last) __hip_atomic_store(&p.counters[idx], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  // One call site in a loop (a second inlined copy of the combine would
  // put its register arrays on the stack).
#pragma unroll 1
  for (int rbc = RW * rbw; rbc < RW * rbw + RW && rbc < p.n_rblk && (32 * rbc) / dm.G < sq; ++rbc) {
    if (rbc > RW * rbw) __syncthreads();  // the previous combine's LDS reads are done
    decode_combine<DT>(p, b, kvh, rbc, t, reinterpret_cast<float*>(lds_a_k0), reinterpret_cast<float*>(lds_b_v0),
                       reinterpret_cast<float*>(lds_d_v1), reinterpret_cast<f32x4*>(lds_c_k1));
  }
}

// ---------------------------------------------------------------------------
// 16-row first pass: a (b, kv head) with at most 16 packed rows (a decode
// step of one token up to G = 16, or of 16 / G tokens).  Same stream, tile
// order, partials and combine as gqa_decode_kernel, with the tile computed
// by v_mfma_f32_16x16x32: half the matrix cycles, and half the scores per
// lane (16 instead of 32, with 28 of every 32 rows of the 32-row form being
// padding at a Llama-3.1-8B decode step), so a chunk's tiles take about
// half the compute between their arrival and the next refill.  At these
// shapes the time between a tile's arrival and the issue of its stage's
// next tile is what bounds each workgroup's stream (decode at 2K-32K keys
// runs as fast from the Infinity Cache as from HBM).
//
// Lane l = (row i16 = l % 16, lane group lg = l / 16).  S^T for the 64 keys
// of a tile is four 16-key blocks: register v of block kb holds key
// 16 kb + 4 lg + v of row i16 (C layout of the 16x16 MFMA), so a row's 64
// scores are spread over the 4 lane groups (row max / sum across them by
// v_permlane16_swap and v_permlane32_swap).  The P^T operand of the 32-key
// block j takes lane l's own 8 probabilities — keys 32 j + 4 lg + 0..3 and
// 32 j + 16 + 4 lg + 0..3 — as k-slots 8 lg + 0..7, so the V^T operand reads
// the same two 4-key runs (two ds_read_b64_tr_b16).  V tiles are swizzled
// by sv16(r) = 2 (r & 7): the 8 rows one half-wave's transposing read
// touches (two lane groups x 4 keys) then cover all 64 banks once.  Wave w
// accumulates O^T for dims [32 w, 32 w + 32) as two 16-dim blocks.
// Head_dim 64 (128-byte rows, 8 rows per LDS-DMA instruction): wave w takes
// dims [16 w, 16 w + 16), one block, and V is swizzled by sv16(r) = r & 6
// (a half-wave's 8 rows x 32 bytes: rows of one parity share a bank half,
// and r & 6 gives their four 32-byte pieces four distinct bank groups); the
// fused combine is not built for it (its callers take the two-launch form).
// ---------------------------------------------------------------------------
template <int DT, int KV, int D = kDecD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gqa_decode16_kernel(SplitParams p) {
  static_assert(D == 128 || D == 64, "head_dim 64 or 128");
  constexpr bool PAGED = KV != 0;
  using E = Elem<DT>;
  using ST = FwdStage<D>;
  constexpr int CPR = ST::CPR;
  constexpr int NI = ST::NI;    // LDS-DMA instructions per wave per K (or V) tile
  constexpr int NKS = D / 32;   // k-steps of S^T
  constexpr int NDB = D / 64;   // 16-dim blocks of O^T per wave
  // Keys per step: 64 at head_dim 128; 128 at head_dim 64 (two 64-row
  // sub-tiles per stage), so that a step moves the same 32 KiB of K and V.
  constexpr int TK = D == 64 ? 128 : 64;
  constexpr int NKB = TK / 16;  // 16-key blocks of S^T per step
  constexpr int NSUB = TK / 64;
  // The V swizzle (chunk XOR) of tile row r: a function of r & 7.
  auto sv16 = [](int r) { return D == 128 ? 2 * (r & 7) : (r & 6); };
  // LDS as gqa_decode_kernel: two stages (64 KiB at head_dim 128, two
  // workgroups per CU; a third stage for grids of one workgroup per CU
  // measured slower at 8K-32K keys), reused by the fused combine.
  __shared__ __attribute__((aligned(1024))) char lds_a_k0[NSUB * ST::kTileBytes];
  __shared__ __attribute__((aligned(1024))) char lds_b_v0[NSUB * ST::kTileBytes];
  __shared__ __attribute__((aligned(1024))) char lds_c_k1[NSUB * ST::kTileBytes];
  __shared__ __attribute__((aligned(1024))) char lds_d_v1[NSUB * ST::kTileBytes];
  __shared__ int s_last;

  const Dims& dm = p.dm;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6) & 3;
  const int i16 = lane & 15, lg = lane >> 4;

  const int total = dm.B * dm.Hkv * p.splits;  // one row block per (b, kv head)
  const int w = xcd_remap(blockIdx.x, total);
  const int s = w % p.splits;
  const int rest = w / p.splits;
  const int kvh = rest % dm.Hkv;
  const int b = rest / dm.Hkv;
  const int skv = PAGED ? min(max(load_uniform(p.seq_lens + b), 0), dm.Skv) : dm.Skv;
  const bool varlen = p.q_len != nullptr;
  const int sq = varlen ? min(max(load_uniform(p.q_len + b), 0), dm.Sq) : dm.Sq;
  const int64_t tok0 = varlen ? (int64_t)load_uniform(p.q_start + b) : 0;
  if (sq <= 0) return;  // a sequence without query rows (variable lengths)

  // This lane's query row (position-major packing).
  const int pos = i16 / dm.G, g = i16 - pos * dm.G;
  const bool valid = pos < sq;
  const int head = kvh * dm.G + g;
  const int qpos = pos + (skv - sq);

  // Keys of this chunk (gqa_split.py:55-60), clamped to the block's last
  // visible key under causal.
  const int c0 = s * p.chunk;
  int c1 = min(c0 + p.chunk, skv);
  const int pos_hi = min(sq - 1, 15 / dm.G);
  if (dm.causal) c1 = min(c1, pos_hi + (skv - sq) + 1);
  const int nk = max(c1 - c0, 0);
  const int ntiles = (nk + TK - 1) / TK;
  const int qpos_lo = skv - sq;

  const uint32_t kssb = (uint32_t)(2 * p.k.ss), vssb = (uint32_t)(2 * p.v.ss);
  const char* kbase = static_cast<const char*>(p.k.ptr) +
                      2 * ((PAGED ? 0 : (int64_t)b * p.k.sb + (int64_t)c0 * p.k.ss) + (int64_t)kvh * p.k.sh);
  const char* vbase = static_cast<const char*>(p.v.ptr) +
                      2 * ((PAGED ? 0 : (int64_t)b * p.v.sb + (int64_t)c0 * p.v.ss) + (int64_t)kvh * p.v.sh);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase, !PAGED && nk > 0 ? (uint32_t)(nk - 1) * kssb + 2 * D : 0u);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase, !PAGED && nk > 0 ? (uint32_t)(nk - 1) * vssb + 2 * D : 0u);
  const int* table_row = PAGED ? p.block_table + (int64_t)b * p.table_stride : nullptr;

  // Tile order: splits start a quarter of the chunk apart (as gqa_decode_kernel).
  const int rot = (p.rotate && ntiles >= 4) ? (s & 3) * (ntiles >> 2) : 0;
  auto tile_rel = [&](int it) {
    const int j = it + rot;
    return it >= ntiles ? it : (j >= ntiles ? j - ntiles : j);
  };

  // LDS-DMA source offsets of this lane: its row within an instruction's
  // RPI rows, its chunk swizzled by gk (K) or sv16 (V) of the tile row, whose
  // low bits are those of RPI w + lrow for every instruction this wave issues
  // (instruction j of wave w loads rows RPI (4 j + w) + 0..RPI-1).
  const int lrow = lane / CPR;
  const uint32_t koff =
      (uint32_t)(lrow * kssb) + 16u * (uint32_t)((lane % CPR) ^ ST::gk((wave * ST::RPI + lrow) & 15));
  const uint32_t voff = (uint32_t)(lrow * vssb) + 16u * (uint32_t)((lane % CPR) ^ sv16(wave * ST::RPI + lrow));
  // Loads of the 64 rows from key j of the chunk into kst / vst.
  auto issue64 = [&](int j, char* kst, char* vst) {
    if constexpr (KV == 0) {
      issue_tile_dma<D, kDmaStream>(kst, rk, (uint32_t)j * kssb, kssb, koff, wave);
      issue_tile_dma<D, kDmaStream>(vst, rv, (uint32_t)j * vssb, vssb, voff, wave);
    } else if constexpr (KV == 1) {
      const int key0 = c0 + j, rows = c1 - key0;
      __amdgpu_buffer_rsrc_t tk = make_rsrc(kbase, 0u), tv = make_rsrc(vbase, 0u);
      if (rows > 0) {
        const int64_t pg = load_uniform(table_row + (key0 >> p.block_shift));
        const int64_t slot = key0 & ((1 << p.block_shift) - 1);
        const uint32_t n = (uint32_t)(min(rows, 64) - 1);
        tk = make_rsrc(kbase + 2 * (pg * p.k.sb + slot * p.k.ss), n * kssb + 2 * D);
        tv = make_rsrc(vbase + 2 * (pg * p.v.sb + slot * p.v.ss), n * vssb + 2 * D);
      }
      issue_tile_dma<D, kDmaStream>(kst, tk, 0u, kssb, koff, wave);
      issue_tile_dma<D, kDmaStream>(vst, tv, 0u, vssb, voff, wave);
    } else if constexpr (KV == 3) {
      // Pages of 16-32 keys: this wave loads rows [key, key + 16) of the
      // tile (one page; as gqa_decode_kernel).  Instruction jj loads rows
      // 16 wave + RPI jj + lrow, whose V swizzle is sv16(RPI jj + lrow).
      typedef __attribute__((address_space(3))) void lds_void;
      const int key = c0 + j + 16 * wave, rows = c1 - key;
      __amdgpu_buffer_rsrc_t tk = make_rsrc(kbase, 0u), tv = make_rsrc(vbase, 0u);
      if (rows > 0) {
        const int64_t pg = load_uniform(table_row + (key >> p.block_shift));
        const int64_t slot = key & ((1 << p.block_shift) - 1);
        const uint32_t n = (uint32_t)(min(rows, 16) - 1);
        tk = make_rsrc(kbase + 2 * (pg * p.k.sb + slot * p.k.ss), n * kssb + 2 * D);
        tv = make_rsrc(vbase + 2 * (pg * p.v.sb + slot * p.v.ss), n * vssb + 2 * D);
      }
#pragma unroll
      for (int jj = 0; jj < NI; ++jj) {
        const uint32_t ko = (uint32_t)(lrow * kssb) +
                            16u * (uint32_t)((lane % CPR) ^ ST::gk(lrow) ^ ST::gk(jj * ST::RPI));
        const uint32_t vo = (uint32_t)(lrow * vssb) + 16u * (uint32_t)((lane % CPR) ^ sv16(jj * ST::RPI + lrow));
        __builtin_amdgcn_raw_ptr_buffer_load_lds(tk, (lds_void*)(kst + (wave * NI + jj) * 1024), 16, ko,
                                                 (uint32_t)(jj * ST::RPI) * kssb, 0, kDmaStream);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(tv, (lds_void*)(vst + (wave * NI + jj) * 1024), 16, vo,
                                                 (uint32_t)(jj * ST::RPI) * vssb, 0, kDmaStream);
      }
    } else {
      typedef __attribute__((address_space(3))) void lds_void;
#pragma unroll
      for (int jj = 0; jj < NI; ++jj) {
        const int step = jj * 4 + wave;
        const int key = c0 + j + step * ST::RPI, rows = c1 - key;
        __amdgpu_buffer_rsrc_t tk = make_rsrc(kbase, 0u), tv = make_rsrc(vbase, 0u);
        if (rows > 0) {
          const int64_t pg = load_uniform(table_row + (key >> p.block_shift));
          const int64_t slot = key & ((1 << p.block_shift) - 1);
          const uint32_t n = (uint32_t)(min(rows, ST::RPI) - 1);
          tk = make_rsrc(kbase + 2 * (pg * p.k.sb + slot * p.k.ss), n * kssb + 2 * D);
          tv = make_rsrc(vbase + 2 * (pg * p.v.sb + slot * p.v.ss), n * vssb + 2 * D);
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(tk, (lds_void*)(kst + step * 1024), 16, koff, 0, 0, kDmaStream);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(tv, (lds_void*)(vst + step * 1024), 16, voff, 0, 0, kDmaStream);
      }
    }
  };
  // Step `it` (TK keys from tile_rel(it) * TK): NSUB sub-tiles of 64 rows.
  auto issue = [&](int it, char* kst, char* vst) {
    const int j = tile_rel(it) * TK;
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) issue64(j + 64 * sub, kst + sub * ST::kTileBytes, vst + sub * ST::kTileBytes);
  };

  // Loads in issue order: tile 0, Q (only lanes of valid rows touch memory:
  // an invalid lane's offset lies past the query group's descriptor and
  // reads zero), tile 1.
  issue(0, lds_a_k0, lds_b_v0);
  u32x4 qreg[NKS];
  {
    const char* qg = static_cast<const char*>(p.q.ptr) +
                     2 * ((varlen ? tok0 * p.q.ss : (int64_t)b * p.q.sb) + (int64_t)kvh * dm.G * p.q.sh);
    const uint32_t qext = (uint32_t)(2 * ((int64_t)(dm.G - 1) * p.q.sh + (int64_t)(sq - 1) * p.q.ss + D));
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(qg, qext);
    const uint32_t qo = valid ? (uint32_t)(2 * ((int64_t)g * p.q.sh + (int64_t)pos * p.q.ss) + 16 * lg) : 0x80000000u;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
      qreg[ks] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, qo + 64u * ks, 0, 0));
  }
  issue(1, lds_c_k1, lds_d_v1);
  // Tile 0 and Q have landed (tile 1 may still be in flight).
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * NI * NSUB));

  // LDS read offsets.  K: row 16 kb + i16, chunk 4 ks + lg (16 lanes of a
  // lane group read 16 rows at distinct swizzled chunks: conflict-free).
  // V: the first run's row 4 lg + jj / 4 (jj = lane within its 16-lane
  // group), dims (D / 4) wave + 16 db + 4 (jj % 4).
  uint32_t ka[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks)
    ka[ks] = (uint32_t)(i16 * (2 * D) + 16 * ((4 * ks + lg) ^ ST::gk(i16))) & (uint32_t)((32 * D - 1) & ~15);
  uint32_t vb[NDB];
  {
    const int jj = lane & 15;
    const int rr = 4 * lg + (jj >> 2);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      vb[db] = (uint32_t)(rr * (2 * D) + 16 * (((D / 32) * wave + 2 * db + ((jj & 3) >> 1)) ^ sv16(rr)) + 8 * (jj & 1)) &
               (uint32_t)((32 * D - 1) & ~7);
  }

  f32x4 acc[NDB] = {};
  float m_run = -__builtin_inff(), l_run = 0.f;
  const float c = dm.c;

  auto set_prio = [&](int it) {
    const int lvl = (4 * it) / ntiles;
    if (lvl == 0) __builtin_amdgcn_s_setprio(3);
    else if (lvl == 1) __builtin_amdgcn_s_setprio(2);
    else if (lvl == 2) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
  };

  auto step = [&](auto s3, auto issue_c, auto last_c, int it) {
    constexpr int S3 = decltype(s3)::value;
    constexpr bool ISSUE = decltype(issue_c)::value;
    constexpr bool LAST = decltype(last_c)::value;
    char* kst = S3 == 0 ? lds_a_k0 : lds_c_k1;
    char* vst = S3 == 0 ? lds_b_v0 : lds_d_v1;
    const char* ck = kst;
    const char* cv = vst;
    if ((it & 3) == 0) set_prio(it);
    // This wave's loads of tile it have landed (those of tile it + 1 may
    // still be in flight); after the barrier, every wave's have.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(LAST ? 0 : 2 * NI * NSUB));
    phase_barrier();

    // S^T for the TK keys: NKB 16-key blocks, NKS k-steps each.
    f32x4 sc[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) sc[kb] = f32x4{};
    {
      u32x4 opk[NKB * NKS];
#pragma unroll
      for (int j = 0; j < NKB * NKS; ++j)
        opk[j] = *reinterpret_cast<const u32x4*>(ck + (j / NKS) * 16 * (2 * D) + ka[j % NKS]);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) sc[kb] = E::mfma16(opk[kb * NKS + ks], qreg[ks], sc[kb]);
    }
    const int key0 = c0 + tile_rel(it) * TK;
    const bool need_mask = (key0 + TK > c1) || (dm.causal && key0 + TK - 1 > qpos_lo);
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int key = key0 + 16 * kb + 4 * lg + v;
          const bool off = key >= c1 || (dm.causal && key > qpos);
          sc[kb][v] = off ? -__builtin_inff() : sc[kb][v];
        }
    }
    // Exact online softmax (gqa_split.py:92-101) in exp2 units; a row with
    // no visible key so far keeps m = -inf and uses 0 as reference.
    float mx;
    if constexpr (NKB == 4) {
      const float t0 = vmax3(sc[0][0], sc[0][1], sc[0][2]), t1 = vmax3(sc[0][3], sc[1][0], sc[1][1]);
      const float t2 = vmax3(sc[1][2], sc[1][3], sc[2][0]), t3 = vmax3(sc[2][1], sc[2][2], sc[2][3]);
      const float t4 = vmax3(sc[3][0], sc[3][1], sc[3][2]);
      mx = xhalf_max(xquad_max(fmaxf(vmax3(t0, t1, t2), vmax3(t3, t4, sc[3][3]))));
    } else {
      float tb[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) tb[kb] = fmaxf(vmax3(sc[kb][0], sc[kb][1], sc[kb][2]), sc[kb][3]);
#pragma unroll
      for (int w = NKB / 2; w >= 1; w /= 2)
#pragma unroll
        for (int kb = 0; kb < w; ++kb) tb[kb] = fmaxf(tb[kb], tb[kb + w]);
      mx = xhalf_max(xquad_max(tb[0]));
    }
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
    const float alpha = fast_exp2((m_run - m_use) * c);
    const float nmc = -m_use * c;
    float pv[NKB][4];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int v = 0; v < 4; ++v) pv[kb][v] = fast_exp2(__builtin_fmaf(sc[kb][v], c, nmc));
    float rs;
    if constexpr (NKB == 4) {
      rs = ((pv[0][0] + pv[0][1]) + (pv[0][2] + pv[0][3])) + ((pv[1][0] + pv[1][1]) + (pv[1][2] + pv[1][3])) +
           (((pv[2][0] + pv[2][1]) + (pv[2][2] + pv[2][3])) + ((pv[3][0] + pv[3][1]) + (pv[3][2] + pv[3][3])));
    } else {
      float tb[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) tb[kb] = (pv[kb][0] + pv[kb][1]) + (pv[kb][2] + pv[kb][3]);
#pragma unroll
      for (int w = NKB / 2; w >= 1; w /= 2)
#pragma unroll
        for (int kb = 0; kb < w; ++kb) tb[kb] = tb[kb] + tb[kb + w];
      rs = tb[0];
    }
    u32x4 pk[NKB / 2];
#pragma unroll
    for (int j = 0; j < NKB / 2; ++j)
      pk[j] = u32x4{E::pack2(pv[2 * j][0], pv[2 * j][1]), E::pack2(pv[2 * j][2], pv[2 * j][3]),
                    E::pack2(pv[2 * j + 1][0], pv[2 * j + 1][1]), E::pack2(pv[2 * j + 1][2], pv[2 * j + 1][3])};
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc[db] *= alpha;

    // O^T (this wave's dims) += V^T P^T over the TK keys.
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int j = 0; j < NKB / 2; ++j) {
        const u32x2 lo = ld_tr(cv + vb[db] + (32 * j) * (2 * D));
        const u32x2 hi = ld_tr(cv + vb[db] + (32 * j + 16) * (2 * D));
        acc[db] = E::mfma16(u32x4{lo[0], lo[1], hi[0], hi[1]}, pk[j], acc[db]);
      }
    phase_barrier();
    if constexpr (ISSUE) issue(it + 2, kst, vst);
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using BT = std::true_type;
  using BF = std::false_type;
  // Tiles in pairs; an odd count is padded with one tile past the chunk
  // (zeros, every key masked); the last pair refills nothing.
  const int ne = (ntiles + 1) & ~1;
  int it = 0;
  for (; it + 4 <= ne; it += 2) {
    step(I0{}, BT{}, BF{}, it);
    step(I1{}, BT{}, BF{}, it + 1);
  }
  if (it < ne) {
    step(I0{}, BF{}, BF{}, it);
    step(I1{}, BF{}, BT{}, it + 1);
  }
  __builtin_amdgcn_s_setprio(0);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  // This wave's dims of the valid rows' partials: lane (i16, lg) holds dims
  // (D / 4) wave + 16 db + 4 lg + 0..3 in acc[db]; l is summed over the 4 lane
  // groups (each holds the sum over its own keys).
  const float l_tot = xhalf_sum(xquad_sum(l_run));
  if (valid) {
    const int64_t row = (((int64_t)b * dm.Hq + head) * dm.Sq + pos) * p.splits + s;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.ws_acc, 0xFFFFFFF0u);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      store_coherent4(rw, (uint32_t)((row * D + (D / 4) * wave + 16 * db + 4 * lg) * 4), acc[db]);
    if (wave == 0 && lg == 0) {
      store_coherent(p.ws_m + row, skv == 0 ? 0.f : m_run * c);
      store_coherent(p.ws_l + row, l_tot);
    }
  }

  if (PAGED || D != kDecD || p.counters == nullptr) return;
  // Fused combine, as gqa_decode_kernel.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    const int idx = (b * dm.Hkv + kvh) * p.n_rblk;
    const int prev = __hip_atomic_fetch_add(&p.counters[idx], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == p.splits - 1);
    if (s_last) __hip_atomic_store(&p.counters[idx], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  decode_combine<DT>(p, b, kvh, 0, t, reinterpret_cast<float*>(lds_a_k0), reinterpret_cast<float*>(lds_b_v0),
                     reinterpret_cast<float*>(lds_d_v1), reinterpret_cast<f32x4*>(lds_c_k1));
}

bool decode_kernel_fits(const SplitParams& p) {
  const int D = p.dm.D;
  // Head_dim 64: the 16-row first pass only (at most 16 packed rows per kv
  // head), in the two-launch form (no fused combine at that width).
  if (D == 64) {
    if (p.dm.G * p.dm.Sq > 16 || p.counters != nullptr) return false;
  } else if (D != kDecD) {
    return false;
  }
  const bool paged = p.block_table != nullptr;
  // Paged: whole LDS-DMA instructions (512 / D rows) in a page, and
  // 64-key-aligned chunks (so a tile lies in a page of >= 64 keys).
  if (paged && ((1 << p.block_shift) < 512 / D || (p.chunk & 63) != 0)) return false;
  // 32-bit descriptor offsets: (contiguous) a chunk plus the padding step
  // past it (two steps of 64 keys at head_dim 128, of 128 at 64), (paged) a
  // 64-row sub-tile; the whole accumulator workspace.
  const int64_t span = paged ? 64 : (int64_t)p.chunk + (D == 64 ? 256 : 128);
  if (span * p.k.ss * 2 >= ((int64_t)1 << 31) || span * p.v.ss * 2 >= ((int64_t)1 << 31)) return false;
  const int64_t acc_bytes = (int64_t)p.dm.B * p.dm.Hq * p.dm.Sq * p.splits * D * 4;
  // ... and a kv head's query group (its G heads x Sq rows).
  const int64_t q_bytes = 2 * ((int64_t)(p.dm.G - 1) * p.q.sh + (int64_t)(p.dm.Sq - 1) * p.q.ss + D);
  return acc_bytes <= 0xFFFFFFF0ll && q_bytes < ((int64_t)1 << 31);
}

// Every 32-row block of a kv head in one workgroup up to four (each K/V
// chunk is then streamed once per 64 or 128 rows, not per 32).
template <int DT, int KV>
static hipError_t launch_decode_t(const SplitParams& p, hipStream_t stream) {
  const int rw = p.n_rblk >= 3 ? 4 : p.n_rblk == 2 ? 2 : 1;
  const int64_t total = (int64_t)p.dm.B * p.dm.Hkv * ((p.n_rblk + rw - 1) / rw) * p.splits;
  if (total <= 0) return hipSuccess;
  if (p.dm.D == 64)  // decode_kernel_fits: at most 16 packed rows
    hipLaunchKernelGGL((gqa_decode16_kernel<DT, KV, 64>), dim3((unsigned)total), dim3(256), 0, stream, p);
  else if (p.dm.G * p.dm.Sq <= 16)
    hipLaunchKernelGGL((gqa_decode16_kernel<DT, KV>), dim3((unsigned)total), dim3(256), 0, stream, p);
  else if (rw == 4)
    hipLaunchKernelGGL((gqa_decode_kernel<DT, KV, 4>), dim3((unsigned)total), dim3(256), 0, stream, p);
  else if (rw == 2)
    hipLaunchKernelGGL((gqa_decode_kernel<DT, KV, 2>), dim3((unsigned)total), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((gqa_decode_kernel<DT, KV, 1>), dim3((unsigned)total), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <int KV>
static hipError_t launch_decode_kv(const SplitParams& p, int dtype, hipStream_t stream) {
  return dtype == 0 ? launch_decode_t<0, KV>(p, stream) : launch_decode_t<1, KV>(p, stream);
}

hipError_t launch_decode_first(const SplitParams& p, int dtype, hipStream_t stream) {
  if (p.block_table == nullptr) return launch_decode_kv<0>(p, dtype, stream);
  if (p.block_shift >= 6) return launch_decode_kv<1>(p, dtype, stream);
  return p.block_shift >= 4 ? launch_decode_kv<3>(p, dtype, stream) : launch_decode_kv<2>(p, dtype, stream);
}

}  // namespace gqa
