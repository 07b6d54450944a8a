// gqa_common.hpp — device-side building blocks shared by the gfx950 kernels.
//
// MFMA layout used throughout (v_mfma_f32_32x32x16_{bf16,f16}, wave64):
//   A operand (32 x 16, M x K): lane l holds A[l % 32][8*(l/32) + e], e = 0..7
//   B operand (16 x 32, K x N): lane l holds B[8*(l/32) + e][l % 32]
//   C/D       (32 x 32)       : lane l, register v holds
//                               C[8*(v/4) + 4*(l/32) + (v%4)][l % 32]
//
// The attention tile is computed transposed, S^T = K * Q^T and O^T = V^T * P^T,
// so that the query row is the N index: every lane then owns one query row
// (row = l % 32) and its softmax statistics are per-lane scalars, and the C
// layout of S^T is already the B-operand layout P^T needs for the second
// product (no register shuffle between the two MFMA chains).
//
// v_mfma_f32_16x16x32_{bf16,f16} (Elem::mfma16, the 16-row decode pass),
// confirmed on the MI355X with a one-wave probe:
//   A operand (16 x 32, M x K): lane l holds A[l % 16][8*(l/16) + e], e = 0..7
//   B operand (32 x 16, K x N): lane l holds B[8*(l/16) + e][l % 16]
//   C/D       (16 x 16)       : lane l, register v holds C[4*(l/16) + v][l % 16]
//
// Key order inside a 32-key block: the M index m of S^T is mapped to key
// pi(m) = m with bits 2 and 3 swapped.  With that map, register v of the
// S^T accumulator in lane l holds key 16*(v/8) + 8*(l/32) + (v%8), so the 8
// probabilities a lane feeds to one PV MFMA are 8 consecutive keys and the
// matching V^T operand is one 16-byte LDS read.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gqa {

constexpr int kWave = 64;

typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8 __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef uint32_t u32x4 __attribute__((__vector_size__(4 * sizeof(uint32_t))));
typedef uint32_t u32x2 __attribute__((__vector_size__(2 * sizeof(uint32_t))));

// ---------------------------------------------------------------------------
// Element-type traits: storage type, MFMA call and fp32 -> 2x16-bit packing.
// ---------------------------------------------------------------------------
template <int DT> struct Elem;

template <> struct Elem<0> {  // bf16
  using T = __bf16;
  __device__ static inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // v_mfma_f32_16x16x32_bf16 (layout in the header comment).
  __device__ static inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even conversion of two floats, packed lo | hi << 16.
  __device__ static inline uint32_t pack2(float lo, float hi) {
    typedef __bf16 bf16x2 __attribute__((__vector_size__(2 * sizeof(__bf16))));
    bf16x2 r;
    r[0] = (__bf16)lo;
    r[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, r);
  }
};

template <> struct Elem<1> {  // fp16
  using T = _Float16;
  __device__ static inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    typedef _Float16 f16x2 __attribute__((__vector_size__(2 * sizeof(_Float16))));
    f16x2 r;
    r[0] = (_Float16)lo;
    r[1] = (_Float16)hi;
    return __builtin_bit_cast(uint32_t, r);
  }
};

// ---------------------------------------------------------------------------
// Small helpers
// ---------------------------------------------------------------------------
__device__ inline int lane_id() { return __lane_id(); }

// Key offset (0..31) inside a 32-key block held by register v of lane half h.
__device__ constexpr int key_of(int v, int h) { return 16 * (v >> 3) + 8 * h + (v & 7); }

// pi: M index of S^T -> key inside a 32-key block (swap bits 2 and 3).
__device__ constexpr int pi_key(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

// Value of x in lane (l ^ 32), combined with x by `op`.  v_permlane32_swap
// exchanges the upper half of its first operand with the lower half of its
// second; feeding x twice leaves {x[l%32], x[l%32+32]} in the two results.
__device__ inline float xhalf_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xhalf_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The same for lane (l ^ 16): v_permlane16_swap exchanges the odd 16-lane
// rows of its first operand with the even rows of its second.
__device__ inline float xquad_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xquad_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------
// LDS tile of 64 keys x D (one "sub-tile").  K is stored row-major [key][d]
// in 16-byte chunks with an XOR swizzle; V is stored transposed [d][key] in
// 16-byte chunks of 8 keys with a second XOR swizzle.  Both swizzles make the
// MFMA operand reads (8 lanes per LDS cycle) and the tile writes hit distinct
// banks.
// ---------------------------------------------------------------------------
template <int D> struct SubTile {
  static constexpr int kKeys = 64;
  static constexpr int kKBytes = kKeys * D * 2;  // K part
  static constexpr int kVBytes = D * kKeys * 2;  // V^T part
  static constexpr int kBytes = kKBytes + kVBytes;

  // K: row r (key), 16-byte chunk cd (d = 8*cd .. 8*cd+7).
  __device__ static constexpr int k_off(int r, int cd) {
    const int g = (r & 3) | (((r >> 3) & 1) << 2);
    return r * (D * 2) + ((cd ^ g) << 4);
  }
  // V^T: row d, chunk c (keys 8*c .. 8*c+7).
  __device__ static constexpr int v_off(int d, int c) {
    const int f = (d + (d >> 3)) & 7;
    return kKBytes + d * (kKeys * 2) + ((c ^ f) << 4);
  }
};

// Per-thread staging registers for one 64-key sub-tile, loaded from global
// memory with 16-byte (K) and 8-byte (V) coalesced loads by 256 threads.
//   K: chunk ci = t + 256*j (j < KCH): row ci / (D/8), chunk ci % (D/8).
//   V: thread owns keys [KPT*kg, KPT*kg + KPT) x d [4*d4, 4*d4 + 4),
//      d4 = t % (D/4), kg = t / (D/4), KPT = D/16 keys.
template <int D> struct SubTileRegs {
  static constexpr int KCH = (64 * D / 8) / 256;  // 16-byte K chunks per thread
  static constexpr int KPT = D / 16;              // keys per thread for V
  u32x4 k[KCH];
  u32x2 v[KPT];
};

// 16- and 8-byte global loads; kStream selects the non-temporal form
// (global_load ... nt), which streams data that is read exactly once at a
// markedly higher rate than cached loads on MI355X HBM.
template <bool kStream>
__device__ inline u32x4 ld16(const void* p) {
  if constexpr (kStream) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return *reinterpret_cast<const u32x4*>(p);
}
template <bool kStream>
__device__ inline u32x2 ld8(const void* p) {
  if constexpr (kStream) return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
  return *reinterpret_cast<const u32x2*>(p);
}

// Wave-uniform read of a value that no work-item writes during the launch
// (block tables, per-sequence lengths) through the scalar cache.  Read as an
// ordinary global load it would be a vector load whose s_waitcnt vmcnt(0)
// also waits for every LDS-DMA tile load in flight.
__device__ inline int load_uniform(const int* p) {
  // Global and constant address-space pointers share one 64-bit address.
  typedef const __attribute__((address_space(4))) int ConstInt;
  return *(ConstInt*)(uintptr_t)p;
}

// Where the K or V row of key j of one (b, kv head) lives.
//   Contiguous: base + j * row stride (the (B, H, S, D) tensors).
//   Paged: a block table maps key j to slot j % block_size of block
//   table[j / block_size] of a cache laid out (num_blocks, block_size,
//   heads, D) in any strides; block_size is a power of two.
// run64(key0): keys [key0, key0 + 64) form one strided run, so the first
// row's address and the row stride locate all 64.  With pages of >= 64 keys
// this holds for every 64-aligned key0 (the paged first pass starts its
// chunks on 64-key boundaries); with smaller pages every row resolves its own
// page.  The two paged cases are separate types so each kernel instantiation
// carries only one load path.
template <typename T>
struct ContigRows {
  const T* base;  // key 0 of this (b, kv head)
  int64_t ss;     // key stride (elements)
  __device__ const T* row(int key) const { return base + (int64_t)key * ss; }
  __device__ const T* row_uniform(int key) const { return row(key); }
  __device__ static constexpr bool run64() { return true; }
};
template <typename T, bool kBigPages>
struct PagedRows {
  const T* base;      // the cache at this kv head (block 0, slot 0)
  const int* table;   // this sequence's block-table entries from page tab0 on
  int64_t sblk, sss;  // block and slot strides (elements)
  int shift;          // log2(block_size)
  int tab0;           // page index of table[0] (a slice of the row staged in LDS)
  __device__ const T* row(int key) const {
    return base + (int64_t)table[(key >> shift) - tab0] * sblk + (int64_t)(key & ((1 << shift) - 1)) * sss;
  }
  // The same for a key that is equal in every lane (scalar table read).
  __device__ const T* row_uniform(int key) const {
    return base + (int64_t)load_uniform(table + ((key >> shift) - tab0)) * sblk +
           (int64_t)(key & ((1 << shift) - 1)) * sss;
  }
  __device__ static constexpr bool run64() { return kBigPages; }
};

// Load keys [key0, key0 + 64) of one (b, kv head) into registers; rows at or
// beyond `key_lim` read as zero.  kr/vr locate K and V rows (see run64 for
// the alignment key0 needs).  A tile that lies entirely below key_lim (all
// but the last) takes the unpredicated path.
template <int D, typename T, bool kStream, typename KR>
__device__ inline void load_subtile(SubTileRegs<D>& R, const KR& kr, const KR& vr, int64_t kss, int64_t vss,
                                    int key0, int key_lim, int t) {
  const int d4 = t % (D / 4), kg = t / (D / 4);
  constexpr int KPT = SubTileRegs<D>::KPT;
  if (key0 + 64 <= key_lim) {
    if constexpr (KR::run64()) {
      const T* kb = kr.row_uniform(key0);
      const T* vb = vr.row_uniform(key0);
#pragma unroll
      for (int j = 0; j < SubTileRegs<D>::KCH; ++j) {
        const int ci = t + 256 * j;
        const int r = ci / (D / 8), cd = ci % (D / 8);
        R.k[j] = ld16<kStream>(kb + (int64_t)r * kss + cd * 8);
      }
#pragma unroll
      for (int j = 0; j < KPT; ++j) R.v[j] = ld8<kStream>(vb + (int64_t)(kg * KPT + j) * vss + d4 * 4);
      return;
    }
#pragma unroll
    for (int j = 0; j < SubTileRegs<D>::KCH; ++j) {
      const int ci = t + 256 * j;
      const int r = ci / (D / 8), cd = ci % (D / 8);
      R.k[j] = ld16<kStream>(kr.row(key0 + r) + cd * 8);
    }
#pragma unroll
    for (int j = 0; j < KPT; ++j) R.v[j] = ld8<kStream>(vr.row(key0 + kg * KPT + j) + d4 * 4);
    return;
  }
#pragma unroll
  for (int j = 0; j < SubTileRegs<D>::KCH; ++j) {
    const int ci = t + 256 * j;
    const int r = ci / (D / 8), cd = ci % (D / 8);
    const int key = key0 + r;
    u32x4 x = {0u, 0u, 0u, 0u};
    if (key < key_lim) x = ld16<kStream>(kr.row(key) + cd * 8);
    R.k[j] = x;
  }
#pragma unroll
  for (int j = 0; j < KPT; ++j) {
    const int key = key0 + kg * KPT + j;
    u32x2 x = {0u, 0u};
    if (key < key_lim) x = ld8<kStream>(vr.row(key) + d4 * 4);
    R.v[j] = x;
  }
}

// Write staged registers into an LDS sub-tile (K row-major, V transposed).
template <int D>
__device__ inline void store_subtile(char* __restrict__ lds, const SubTileRegs<D>& R, int t) {
  using ST = SubTile<D>;
#pragma unroll
  for (int j = 0; j < SubTileRegs<D>::KCH; ++j) {
    const int ci = t + 256 * j;
    const int r = ci / (D / 8), cd = ci % (D / 8);
    *reinterpret_cast<u32x4*>(lds + ST::k_off(r, cd)) = R.k[j];
  }
  const int d4 = t % (D / 4), kg = t / (D / 4);
  constexpr int KPT = SubTileRegs<D>::KPT;
  // Transpose KPT keys x 4 d (16-bit) into 4 rows of KPT keys.
#pragma unroll
  for (int dd = 0; dd < 4; ++dd) {
    const uint32_t sel = (dd & 1) ? 0x07060302u : 0x05040100u;
    uint32_t w[KPT / 2];
#pragma unroll
    for (int i = 0; i < KPT / 2; ++i)
      w[i] = __builtin_amdgcn_perm(R.v[2 * i + 1][dd >> 1], R.v[2 * i][dd >> 1], sel);
    const int d = 4 * d4 + dd;
    if constexpr (KPT == 8) {
      u32x4 o = {w[0], w[1], w[2], w[3]};
      *reinterpret_cast<u32x4*>(lds + ST::v_off(d, kg)) = o;
    } else {  // KPT == 4: half a chunk
      u32x2 o = {w[0], w[1]};
      *reinterpret_cast<u32x2*>(lds + ST::v_off(d, kg >> 1) + ((kg & 1) << 3)) = o;
    }
  }
}

// S^T block (32 keys x 32 query rows) for keys [32*mb, 32*mb + 32) of a
// sub-tile: A = K rows pi(l%32), B = Q^T held in registers (qreg[ks] =
// q[row][16*ks + 8*h .. +8]).
template <int DT, int D>
__device__ inline f32x16 qk_block(const char* __restrict__ lds, const u32x4* qreg, int mb, int lane) {
  using ST = SubTile<D>;
  const int i = lane & 31, h = lane >> 5;
  const int r = 32 * mb + pi_key(i);
  f32x16 s = {};
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    const u32x4 a = *reinterpret_cast<const u32x4*>(lds + ST::k_off(r, 2 * ks + h));
    s = Elem<DT>::mfma(a, qreg[ks], s);
  }
  return s;
}

// O^T += V^T * P^T for keys [32*mb, 32*mb + 32) of a sub-tile.  p[kk] holds
// the 8 probabilities (packed 16-bit) of keys 16*kk + 8*h + 0..7.
template <int DT, int D>
__device__ inline void pv_block(const char* __restrict__ lds, const u32x4 p[2], f32x16* acc, int mb,
                                int lane) {
  using ST = SubTile<D>;
  const int i = lane & 31, h = lane >> 5;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(lds + ST::v_off(32 * db + i, 4 * mb + 2 * kk + h));
      acc[db] = Elem<DT>::mfma(a, p[kk], acc[db]);
    }
  }
}

// Buffer resource over `bytes` bytes at `base` (raw buffer, stride 0): loads
// at offsets at or beyond `bytes` return zero instead of touching memory.
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// ---------------------------------------------------------------------------
// Device-coherent (agent scope) 32-bit stores and loads.  On gfx950 they are
// plain global stores/loads with sc1 set: they write through to / read from
// the point where all XCDs are coherent, so data passed between workgroups
// of one launch needs no L2 write-back or invalidate (which a release or
// acquire fence at agent scope performs for the whole L2 of the XCD).
// ---------------------------------------------------------------------------
__device__ inline void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Four consecutive floats at byte offset `off` of buffer `r`, read the same
// way (a 16-byte buffer load with sc1 set: cache-policy bit 4 on gfx950).
__device__ inline f32x4 load_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16));
}

// ---------------------------------------------------------------------------
// Workgroup-id remap: hardware hands consecutive workgroup ids to the 8 XCDs
// round-robin.  Remap so that each XCD receives a contiguous range of work
// items (work items sharing K/V then share that XCD's L2).
// ---------------------------------------------------------------------------
__device__ inline int xcd_remap(int bid, int total) {
  constexpr int kXcd = 8;
  const int q = total / kXcd, r = total % kXcd;
  const int x = bid % kXcd, local = bid / kXcd;
  return x * q + (x < r ? x : r) + local;
}

}  // namespace gqa
