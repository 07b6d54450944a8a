// gqa_split.hip — split-KV decode path for gfx950: first pass + LSE combine.
//
// Replaces the Triton kernels gqa_split_first_kernel and
// gqa_split_reduce_kernel (reference gqa_kernels/gqa_split.py:26-147).
//
// First pass: one workgroup per (batch, kv head, 32-row block, split).  The
// packed rows are the G*Sq (head, position) pairs of one kv head, position
// major (row r -> position r / G, head r % G), so a decode step (Sq = 1) packs
// its whole query group into one MFMA N block and the K/V of the chunk is read
// from HBM exactly once.  The chunk is streamed in 128-key tiles through LDS
// (the next tile's loads are in flight during compute); each of the 4 waves
// runs its own online softmax over 32 keys of every tile, and the 4 partial
// states are merged in LDS before one fp32 partial (m, l, unnormalised acc)
// per row is written (gqa_split.py:102-112).  Chunk bounds follow
// gqa_split.py:55-60, including the causal clamp to the block's last visible
// key; a chunk with no visible key stores m = -inf, l = 0, acc = 0.
//
// Combine: one workgroup per (batch, q head, row):
//   m* = max m_s, a_s = exp2(m_s - m*), l* = sum a_s l_s,
//   o = sum a_s acc_s / l*                         (gqa_split.py:134-147)
// Rows whose keys are all masked give NaN (m* = -inf), as the reference's
// combine; rows of a sequence with no keys at all (first pass stores m = 0,
// l = 0: a finite m* with l* = 0) give zeros, as tests/reference.py:33-34.
//
// Paged variants (KV = 1, 2; no counterpart in the reference): the same
// first pass over a (num_blocks, block_size, Hkv, D) cache, with each
// sequence's key count read from seq_lens[b] and each key row located
// through the block table (PagedRows).  With pages of >= 64 keys (KV = 1) a
// 64-key sub-tile is one strided run inside one page and loads like a
// contiguous tile after one table lookup; smaller pages (KV = 2) resolve the
// page of every row, from a copy of the chunk's table slice in LDS.
#include <type_traits>

#include "gqa_common.hpp"
#include "gqa_params.hpp"

namespace gqa {

// Largest (valid rows x splits) the in-kernel combine stages in LDS; the host
// uses the separate combine kernel beyond it.
constexpr int kFusedMaxRowSplits = 4096;

// Log-sum-exp combine of all splits for the R valid rows of one (b, kv head,
// 32-row block), by one workgroup (gqa_split.py:134-147), spread over all 256
// threads so the tail it adds stays short (every phase is one round of
// loads in flight together, then LDS and wave reductions):
//   1. m and l of every (row, split) into LDS; per row (one wave, lanes over
//      the splits): m* (wave max), a = exp2(m - m*), l* = sum a * l (wave
//      sum);
//   2. work items (split group, row, 4 columns), one per thread where R * D
//      / 4 <= 256: each sums a * acc over its splits with 16-byte
//      device-coherent loads, 16 splits in flight; the split groups are then
//      added up in LDS and o = sum / l*.
// scratch: >= 2*R*S + 2*32 floats plus 1024 f32x4 (reuses the tile buffer).
template <int DT, int D>
__device__ inline void combine_rows(const SplitParams& p, int b, int kvh, int rb, int t, float* scratch) {
  using E = Elem<DT>;
  using T = typename E::T;
  constexpr int NDP = D / 4;
  const Dims& dm = p.dm;
  const int S = p.splits;
  const int r0 = 32 * rb;
  const int R = min(32, dm.G * dm.Sq - r0);  // valid rows: position-major packing
  const int lane = t & 63, wave = t >> 6;
  float* ma = scratch;              // [R][S]: m, then the scale factors a
  float* la = ma + R * S;           // [R][S]: l
  float* mst = la + R * S;          // [32]: m* per row
  float* lst = mst + 32;            // [32]: l* per row
  f32x4* red = reinterpret_cast<f32x4*>(scratch + ((2 * R * S + 64 + 3) & ~3));  // [NSG][R][NDP]

  auto row_index = [&](int rl) {    // (b, head, pos) -> index of split 0 in the workspace
    const int r = r0 + rl;
    const int pos = r / dm.G, g = r - pos * dm.G;
    return ((((int64_t)b * dm.Hq + kvh * dm.G + g) * dm.Sq + pos) * S);
  };

  for (int f = t; f < R * S; f += 256) {
    const int rl = f / S, sp = f - rl * S;
    const int64_t ix = row_index(rl) + sp;
    ma[f] = load_coherent(p.ws_m + ix);
    la[f] = load_coherent(p.ws_l + ix);
  }
  __syncthreads();
  for (int rl = wave; rl < R; rl += 4) {
    float m = -__builtin_inff();
    for (int sp = lane; sp < S; sp += 64) m = fmaxf(m, ma[rl * S + sp]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    // exp2(-inf - -inf) = NaN when every chunk of a row is empty, as the
    // reference's combine (gqa_split.py:138) gives.
    float l = 0.f;
    for (int sp = lane; sp < S; sp += 64) {
      const float a = fast_exp2(ma[rl * S + sp] - m);
      ma[rl * S + sp] = a;
      l += a * la[rl * S + sp];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off, 64);
    if (lane == 0) {
      mst[rl] = m;
      lst[rl] = l;
      // LSE of a row with no visible key is -inf (its o stays NaN).
      if (p.lse != nullptr)
        p.lse[row_index(rl) / S] = m == -__builtin_inff() ? -__builtin_inff() : (m + __log2f(l)) * kLn2;
    }
  }
  __syncthreads();

  // Split groups: one work item per thread (or as many as R * D / 4 needs),
  // each with a long run of independent loads.
  int nsg = 256 / (R * NDP);
  nsg = max(1, min(nsg, S));
  const int items = nsg * R * NDP;
  // 16-byte loads through a buffer descriptor over the whole acc workspace
  // (its size fits the 32-bit offsets: the launcher bounds it).
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.ws_acc, 0xFFFFFFF0u);
  for (int it = t; it < items; it += 256) {
    const int d4 = it % NDP;
    const int rl = (it / NDP) % R;
    const int sg = it / (NDP * R);
    const uint32_t base = (uint32_t)(row_index(rl) * D + 4 * d4) * 4u;
    const float* a = ma + rl * S;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 16
    for (int sp = sg; sp < S; sp += nsg) o += a[sp] * load_coherent4(ra, base + (uint32_t)sp * (D * 4));
    red[it] = o;
  }
  __syncthreads();
  for (int f = t; f < R * NDP; f += 256) {
    const int d4 = f % NDP, rl = f / NDP;
    f32x4 o = red[f];
    for (int sg = 1; sg < nsg; ++sg) o += red[sg * R * NDP + f];
    // A sequence without keys (finite m*, l* = 0, o = 0): 0 / inf = 0.
    const float l = (lst[rl] == 0.f && mst[rl] > -__builtin_inff()) ? __builtin_inff() : lst[rl];
    const int r = r0 + rl;
    const int pos = r / dm.G, g = r - pos * dm.G;
    T* orow = static_cast<T*>(const_cast<void*>(p.o.ptr)) + (int64_t)b * p.o.sb +
              (int64_t)(kvh * dm.G + g) * p.o.sh + (int64_t)pos * p.o.ss + 4 * d4;
    u32x2 x;
    x[0] = E::pack2(o[0] / l, o[1] / l);
    x[1] = E::pack2(o[2] / l, o[3] / l);
    *reinterpret_cast<u32x2*>(orow) = x;
  }
}

// KV: 0 contiguous K/V, 1 paged cache with pages of >= 64 keys, 2 paged
// cache with smaller pages.
template <int DT, int D, int KV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gqa_split_first_kernel(SplitParams p) {
  using E = Elem<DT>;
  using T = typename E::T;
  using ST = SubTile<D>;
  // One 128-key tile = two 64-key sub-tiles; reused for the wave merge and
  // the fused combine.
  constexpr int kCombineBytes = 2 * kFusedMaxRowSplits * 4 + 64 * 4 + 16 + 1024 * 16;
  constexpr int kSmemBytes = 2 * ST::kBytes > kCombineBytes ? 2 * ST::kBytes : kCombineBytes;
  __shared__ __attribute__((aligned(16))) char smem[kSmemBytes];
  __shared__ float m_s[128], l_s[128];
  __shared__ int s_tab[KV == 2 ? kPagedTableMax : 1];

  const Dims& dm = p.dm;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int i = lane & 31, hh = lane >> 5;

  const int total = dm.B * dm.Hkv * p.n_rblk * p.splits;
  const int w = xcd_remap(blockIdx.x, total);
  const int s = w % p.splits;
  int rest = w / p.splits;
  const int rb = rest % p.n_rblk;
  rest /= p.n_rblk;
  const int kvh = rest % dm.Hkv;
  const int b = rest / dm.Hkv;

  // Keys of this sequence: all of them, or (paged) its own length, clamped
  // to [0, max_seq_len] so that no key past the block table's covered range
  // is ever addressed.
  constexpr bool PAGED = KV != 0;
  const int skv = PAGED ? min(max(load_uniform(p.seq_lens + b), 0), dm.Skv) : dm.Skv;
  // Query rows of this sequence (variable lengths: q_len[b] rows, tokens
  // from q_start[b]; q token-major).
  const bool varlen = p.q_len != nullptr;
  const int sq = varlen ? min(max(load_uniform(p.q_len + b), 0), dm.Sq) : dm.Sq;
  const int64_t tok0 = varlen ? (int64_t)load_uniform(p.q_start + b) : 0;
  if ((32 * rb) / dm.G >= sq) return;  // a row block past this sequence's queries

  // This lane's query row (position-major packing).
  const int r = 32 * rb + i;
  const int pos = r / dm.G, g = r - pos * dm.G;
  const bool valid = pos < sq;
  const int head = kvh * dm.G + g;
  const int qpos = pos + (skv - sq);

  u32x4 qreg[D / 16];
  {
    const int qp = valid ? pos : 0;
    const T* qrow = static_cast<const T*>(p.q.ptr) +
                    (varlen ? (tok0 + qp) * p.q.ss + (int64_t)head * p.q.sh
                            : (int64_t)b * p.q.sb + (int64_t)head * p.q.sh + (int64_t)qp * p.q.ss);
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      u32x4 x = {0u, 0u, 0u, 0u};
      if (valid) x = *reinterpret_cast<const u32x4*>(qrow + 16 * ks + 8 * hh);
      qreg[ks] = x;
    }
  }

  // Keys of this chunk, clamped to the block's last visible key.
  const int c0 = s * p.chunk;
  int c1 = min(c0 + p.chunk, skv);
  const int pos_lo = (32 * rb) / dm.G;
  const int pos_hi = min(sq - 1, (32 * rb + 31) / dm.G);
  if (dm.causal) c1 = min(c1, pos_hi + (skv - sq) + 1);
  const int ntiles = c1 > c0 ? (c1 - c0 + kSplitTileKeys - 1) / kSplitTileKeys : 0;
  const int qpos_lo = pos_lo + (skv - sq);

  using Rows = typename std::conditional<PAGED, PagedRows<T, KV == 1>, ContigRows<T>>::type;
  Rows kr, vr;
  if constexpr (PAGED) {
    const int* table = p.block_table + (int64_t)b * p.table_stride;
    int tab0 = 0;
    if constexpr (KV == 2) {
      // Pages under 64 keys: every key row resolves its own page, so the
      // chunk's slice of the block table is copied to LDS once and the
      // per-row lookups read it there (LDS reads) instead of re-reading
      // global memory on the load path.  The launch rejects chunks of more
      // than kPagedTableMax pages; the bound on the copy keeps LDS safe
      // regardless.
      const int p0 = c0 >> p.block_shift;
      const int np = c1 > c0 ? ((c1 - 1) >> p.block_shift) - p0 + 1 : 0;
      for (int e = t; e < np && e < kPagedTableMax; e += 256) s_tab[e] = table[p0 + e];
      __syncthreads();
      table = s_tab;  // entry e = page p0 + e
      tab0 = p0;
    }
    kr = Rows{static_cast<const T*>(p.k.ptr) + (int64_t)kvh * p.k.sh, table, p.k.sb, p.k.ss, p.block_shift, tab0};
    vr = Rows{static_cast<const T*>(p.v.ptr) + (int64_t)kvh * p.v.sh, table, p.v.sb, p.v.ss, p.block_shift, tab0};
  } else {
    kr = Rows{static_cast<const T*>(p.k.ptr) + (int64_t)b * p.k.sb + (int64_t)kvh * p.k.sh, p.k.ss};
    vr = Rows{static_cast<const T*>(p.v.ptr) + (int64_t)b * p.v.sb + (int64_t)kvh * p.v.sh, p.v.ss};
  }

  f32x16 acc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) acc[db] = f32x16{};
  float m_run = -__builtin_inff();
  float l_run = 0.f;
  const float c = dm.c;

  // Tile order.  With one head's keys in consecutive rows, every workgroup
  // would otherwise stream its chunk from the same relative offset in lock
  // step with the others (chunks are equally long and equally aligned),
  // which concentrates the concurrent reads on a subset of the HBM channels;
  // starting splits s = 0..3 (mod 4) a quarter of the chunk apart spreads
  // them (~11% faster decode at 131072 keys).  The online softmax does not
  // depend on the order.
  const int rot = (p.rotate && ntiles >= 4) ? (s & 3) * (ntiles >> 2) : 0;
  auto tile_key = [&](int i) {
    int j = i + rot;
    if (j >= ntiles) j -= ntiles;
    return c0 + j * kSplitTileKeys;
  };

  SubTileRegs<D> R0, R1;
  if (ntiles > 0) {
    load_subtile<D, T, true>(R0, kr, vr, p.k.ss, p.v.ss, tile_key(0), c1, t);
    load_subtile<D, T, true>(R1, kr, vr, p.k.ss, p.v.ss, tile_key(0) + 64, c1, t);
  }
  const int sub = wave >> 1, mb = wave & 1;
  const char* mytile = smem + sub * ST::kBytes;

  // Issue priority falls with progress (3 for the first quarter of the
  // chunk, then 2, 1, 0).  Two workgroups share a compute unit; at equal
  // priority the older one's waves issue first and it streams its chunk up
  // to ~25 % ahead of its neighbour, which then finishes alone at a lower
  // memory rate.  Ranking by progress keeps the two within a quarter of each
  // other (the two end 5 instead of 19 µs apart at 131072 keys, ~2 % faster).
  int prio_lvl = -1;
  for (int it = 0; it < ntiles; ++it) {
    const int key0 = tile_key(it);
    const int lvl = (4 * it) / ntiles;  // wave-uniform
    if (lvl != prio_lvl) {
      prio_lvl = lvl;
      if (lvl == 0) __builtin_amdgcn_s_setprio(3);
      else if (lvl == 1) __builtin_amdgcn_s_setprio(2);
      else if (lvl == 2) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    __syncthreads();  // previous tile fully consumed
    store_subtile<D>(smem, R0, t);
    store_subtile<D>(smem + ST::kBytes, R1, t);
    __syncthreads();
    if (it + 1 < ntiles) {
      load_subtile<D, T, true>(R0, kr, vr, p.k.ss, p.v.ss, tile_key(it + 1), c1, t);
      load_subtile<D, T, true>(R1, kr, vr, p.k.ss, p.v.ss, tile_key(it + 1) + 64, c1, t);
    }

    const int kb0 = key0 + 32 * wave;  // this wave's 32 keys
    if (kb0 >= c1) continue;           // wave-uniform: nothing visible here
    f32x16 sc = qk_block<DT, D>(mytile, qreg, mb, lane);
    const bool need_mask = (kb0 + 32 > c1) || (dm.causal && kb0 + 31 > qpos_lo);
    if (need_mask) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int key = kb0 + key_of(v, hh);
        if (key >= c1 || (dm.causal && key > qpos)) sc[v] = -__builtin_inff();
      }
    }
    float mx = sc[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) mx = fmaxf(mx, sc[v]);
    mx = xhalf_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
    const float alpha = fast_exp2((m_run - m_use) * c);
    const float nmc = -m_use * c;
    float pv[16];
    float rs = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      pv[v] = fast_exp2(__builtin_fmaf(sc[v], c, nmc));
      rs += pv[v];
    }
    u32x4 pk[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int e = 0; e < 4; ++e) pk[kk][e] = E::pack2(pv[8 * kk + 2 * e], pv[8 * kk + 2 * e + 1]);
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[db][v] *= alpha;
    pv_block<DT, D>(mytile, pk, acc, mb, lane);
  }

  __builtin_amdgcn_s_setprio(0);
  // Merge the 4 waves' states in LDS: m_s/l_s [wave][row], acc (reusing the
  // tile buffer, exactly 4 * D * 32 floats) as f32x4 at
  // [((wave * D/32 + db) * 4 + j) * 64 + lane].
  static_assert(4 * D * 32 * sizeof(float) <= 2 * ST::kBytes, "merge buffer");
  const float l_tot = xhalf_sum(l_run);
  __syncthreads();
  f32x4* a_s = reinterpret_cast<f32x4*>(smem);
  if (hh == 0) {
    m_s[wave * 32 + i] = m_run;
    l_s[wave * 32 + i] = l_tot;
  }
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f32x4 x = {acc[db][4 * j], acc[db][4 * j + 1], acc[db][4 * j + 2], acc[db][4 * j + 3]};
      a_s[((wave * (D / 32) + db) * 4 + j) * 64 + lane] = x;
    }
  __syncthreads();
  if (wave < D / 32) {
    const int db = wave;
    float mw[4];
    float mstar = -__builtin_inff();
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      mw[ww] = m_s[ww * 32 + i];
      mstar = fmaxf(mstar, mw[ww]);
    }
    const float mstar_use = (mstar == -__builtin_inff()) ? 0.f : mstar;
    float lsum = 0.f;
    f32x4 o[4] = {};
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float f = fast_exp2((mw[ww] - mstar_use) * c);
      lsum += f * l_s[ww * 32 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] += f * a_s[((ww * (D / 32) + db) * 4 + j) * 64 + lane];
    }
    if (valid) {
      // Device-coherent stores: the fused combine may read them from another
      // XCD within this launch.
      const int64_t row = (((int64_t)b * dm.Hq + head) * dm.Sq + pos) * p.splits + s;
      float* wa = p.ws_acc + row * D;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) store_coherent(wa + 32 * db + 8 * j + 4 * hh + e, o[j][e]);
      // A sequence without keys stores m = 0, l = 0 (never produced
      // otherwise: the chunk's largest score contributes exp2(0) = 1 to l),
      // which the combine turns into a zero row.
      if (db == 0 && hh == 0) {
        store_coherent(p.ws_m + row, skv == 0 ? 0.f : mstar * c);
        store_coherent(p.ws_l + row, lsum);
      }
    }
  }

  if (PAGED || p.counters == nullptr) return;
  // Fused combine: count this partial once its stores have completed, and let
  // the workgroup that completes the count for this (b, kv head, row block)
  // combine all splits.
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are done
  __syncthreads();
  if (t == 0) {
    const int idx = (b * dm.Hkv + kvh) * p.n_rblk + rb;
    const int prev = __hip_atomic_fetch_add(&p.counters[idx], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == p.splits - 1);
    // Every increment of this call has landed: leave the counter zero.
    if (s_last) __hip_atomic_store(&p.counters[idx], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  combine_rows<DT, D>(p, b, kvh, rb, t, reinterpret_cast<float*>(smem));
}

// LSE combine.  256 threads: thread (d4, sg) owns output columns
// [4*d4, 4*d4 + 4) and the splits sg, sg + NSG, ...  One round of loads:
// each thread requests m, l and the accumulators of its splits together
// (up to BATCH splits at a time: 1 when every thread has at most one split,
// else 8) and combines them against its own running maximum; the NSG split
// groups are then merged in LDS against the row maximum m*:
//   m* = max m_s, a_s = exp2(m_s - m*), l* = sum a_s l_s,
//   o = sum a_s acc_s / l*                           (gqa_split.py:134-147)
template <int DT, int D, int BATCH>
__global__ __launch_bounds__(256) void gqa_split_reduce_kernel(ReduceParams p) {
  constexpr int kReduceBatch = BATCH;
  using E = Elem<DT>;
  using T = typename E::T;
  constexpr int ND4 = D / 4;
  constexpr int NSG = 256 / ND4;
  __shared__ float red_m[NSG][ND4];
  __shared__ float red_l[NSG][ND4];
  __shared__ f32x4 red_o[NSG][ND4];

  const int t = threadIdx.x;
  // Row ((b * Hq + h) * Sq + pos), dealt to the XCDs in contiguous ranges:
  // rows are ordered by (b, kv head) as the first passes' work items are,
  // so a row is combined on the XCD whose L2 holds its partials (decode
  // 8192 keys 10.89 -> 10.72 us, a 16-token verify step at 131072 keys
  // 92.25 -> 91.28 us, bit-identical).
  const int row = xcd_remap(blockIdx.x, gridDim.x);
  const int S = p.splits;
  const int pos = row % p.Sq;
  const int bh = row / p.Sq;
  const int h = bh % p.Hq, b = bh / p.Hq;
  // Variable query lengths: rows past this sequence's queries hold no
  // partials; o and lse are token-major.
  const bool varlen = p.q_len != nullptr;
  if (varlen && pos >= p.q_len[b]) return;
  const int64_t tok = varlen ? (int64_t)load_uniform(p.q_start + b) + pos : 0;
  const float* wm = p.ws_m + (int64_t)row * S;
  const float* wl = p.ws_l + (int64_t)row * S;
  const float* wa = p.ws_acc + (int64_t)row * S * D;

  const int d4 = t % ND4, sg = t / ND4;
  float m_loc = -__builtin_inff(), l_loc = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = sg; s0 < S; s0 += kReduceBatch * NSG) {
    float mv[kReduceBatch], lv[kReduceBatch];
    f32x4 av[kReduceBatch];
#pragma unroll
    for (int k = 0; k < kReduceBatch; ++k) {
      const int s = s0 + k * NSG;
      mv[k] = -__builtin_inff();
      lv[k] = 0.f;
      av[k] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (s < S) {
        mv[k] = wm[s];
        lv[k] = wl[s];
        av[k] = *reinterpret_cast<const f32x4*>(wa + (int64_t)s * D + 4 * d4);
      }
    }
    float mb = m_loc;
#pragma unroll
    for (int k = 0; k < kReduceBatch; ++k) mb = fmaxf(mb, mv[k]);
    // Nothing visible yet (every split so far empty): keep (-inf, 0, 0).
    if (mb == -__builtin_inff()) continue;
    const float r = fast_exp2(m_loc - mb);  // 0 while m_loc is -inf
    l_loc *= r;
    o *= r;
#pragma unroll
    for (int k = 0; k < kReduceBatch; ++k) {
      const float a = fast_exp2(mv[k] - mb);
      l_loc += a * lv[k];
      o += a * av[k];
    }
    m_loc = mb;
  }
  red_m[sg][d4] = m_loc;
  red_l[sg][d4] = l_loc;
  red_o[sg][d4] = o;
  __syncthreads();
  if (sg == 0) {
    float mstar = red_m[0][d4];
#pragma unroll
    for (int k = 1; k < NSG; ++k) mstar = fmaxf(mstar, red_m[k][d4]);
    // exp2(-inf - -inf) = NaN when every chunk is empty, as gqa_split.py:138;
    // a group with no visible key (m = -inf, l = 0, o = 0) adds nothing.
    float l = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < NSG; ++k) {
      const float a = fast_exp2(red_m[k][d4] - mstar);
      l += a * red_l[k][d4];
      acc += a * red_o[k][d4];
    }
    // Optional LSE side output (natural log; m* and l* are log2-domain);
    // -inf for a row with no visible key (whose o stays NaN).
    if (p.lse != nullptr && d4 == 0)
      p.lse[varlen ? tok * p.Hq + h : row] =
          mstar == -__builtin_inff() ? -__builtin_inff() : (mstar + __log2f(l)) * kLn2;
    T* orow = static_cast<T*>(const_cast<void*>(p.o.ptr)) +
              (varlen ? tok * p.o.ss + (int64_t)h * p.o.sh
                      : (int64_t)b * p.o.sb + (int64_t)h * p.o.sh + (int64_t)pos * p.o.ss);
    // A sequence without keys (finite m*, l* = 0, o = 0): 0 / inf = 0.
    if (l == 0.f && mstar > -__builtin_inff()) l = __builtin_inff();
    u32x2 x;
    x[0] = E::pack2(acc[0] / l, acc[1] / l);
    x[1] = E::pack2(acc[2] / l, acc[3] / l);
    *reinterpret_cast<u32x2*>(orow + 4 * d4) = x;
  }
}

template <int DT, int D, int KV>
static hipError_t launch_split_first_t(const SplitParams& p, hipStream_t stream) {
  const int64_t total = (int64_t)p.dm.B * p.dm.Hkv * p.n_rblk * p.splits;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL((gqa_split_first_kernel<DT, D, KV>), dim3((unsigned)total), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <int DT, int D>
static hipError_t launch_split_reduce_t(const ReduceParams& p, hipStream_t stream) {
  const int64_t rows = (int64_t)p.B * p.Hq * p.Sq;
  if (rows <= 0) return hipSuccess;
  if (p.splits <= 256 / (D / 4))  // at most one split per thread
    hipLaunchKernelGGL((gqa_split_reduce_kernel<DT, D, 1>), dim3((unsigned)rows), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((gqa_split_reduce_kernel<DT, D, 8>), dim3((unsigned)rows), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_split_first(const SplitParams& p, int dtype, hipStream_t stream) {
  if (decode_kernel_fits(p)) return launch_decode_first(p, dtype, stream);
  if (dtype == 0)
    return p.dm.D == 128 ? launch_split_first_t<0, 128, 0>(p, stream) : launch_split_first_t<0, 64, 0>(p, stream);
  return p.dm.D == 128 ? launch_split_first_t<1, 128, 0>(p, stream) : launch_split_first_t<1, 64, 0>(p, stream);
}

template <int KV>
static hipError_t launch_paged_t(const SplitParams& p, int dtype, hipStream_t stream) {
  if (dtype == 0)
    return p.dm.D == 128 ? launch_split_first_t<0, 128, KV>(p, stream) : launch_split_first_t<0, 64, KV>(p, stream);
  return p.dm.D == 128 ? launch_split_first_t<1, 128, KV>(p, stream) : launch_split_first_t<1, 64, KV>(p, stream);
}

// Requires p.chunk to be a multiple of 64 (sub-tiles start 64-aligned).
hipError_t launch_paged_split_first(const SplitParams& p, int dtype, hipStream_t stream) {
  if (decode_kernel_fits(p)) return launch_decode_first(p, dtype, stream);
  return p.block_shift >= 6 ? launch_paged_t<1>(p, dtype, stream) : launch_paged_t<2>(p, dtype, stream);
}

hipError_t launch_split_reduce(const ReduceParams& p, int dtype, hipStream_t stream) {
  if (dtype == 0)
    return p.D == 128 ? launch_split_reduce_t<0, 128>(p, stream) : launch_split_reduce_t<0, 64>(p, stream);
  return p.D == 128 ? launch_split_reduce_t<1, 128>(p, stream) : launch_split_reduce_t<1, 64>(p, stream);
}

}  // namespace gqa
