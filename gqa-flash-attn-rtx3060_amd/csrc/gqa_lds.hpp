// gqa_lds.hpp — LDS tile staging shared by the single-pass and decode kernels:
// 64-key K/V tiles written straight from global memory into LDS (buffer
// loads in their LDS-DMA form), read back as MFMA operands (K row-major, V
// transposed by ds_read_b64_tr_b16), plus the wait/barrier helpers around
// them.
#pragma once

#include "gqa_common.hpp"

namespace gqa {

// ---------------------------------------------------------------------------
// One pipeline stage in LDS: a 64-key K tile and a 64-key V tile, both
// row-major [key][d] in 16-byte chunks, written by direct-to-LDS loads
// (64 lanes write 1 KiB contiguous per instruction), so both swizzles are
// applied on the global side: the lane that lands on chunk pc of row r
// fetches chunk pc ^ swizzle(r).
//
// K: gk is chosen so that the S^T A-operand reads (row pi(i), chunk 2ks+h)
// hit distinct bank groups in every 16 consecutive lanes; the chunk lane i
// reads is (2ks+h) ^ gk(pi(i)).
//
// V: read transposed by ds_read_b64_tr_b16.  In each 16-lane group of such a
// read, lane j addresses V[r0 + j/4][d0 + 4*(j%4)] and receives
// V[r0 + k][d0 + j] for k = 0..3: 4 keys of one d, the layout of the V^T
// A operand.  A group touches 4 rows x 32 bytes; sv moves the 4 rows to
// distinct bank groups and keeps the two groups of a half-wave (d0 and
// d0 + 16) apart, so the read is conflict-free.
// ---------------------------------------------------------------------------
template <int D> struct FwdStage {
  static constexpr int kKeys = 64;
  static constexpr int CPR = D / 8;                 // 16-byte chunks per row
  static constexpr int kTileBytes = kKeys * D * 2;  // one K or V tile
  static constexpr int RPI = 64 / CPR;              // rows per LDS-DMA instruction
  static constexpr int NI = (kKeys * CPR) / 256;    // LDS-DMA instructions per wave of a group

  // D = 128 (256-byte rows): gk(pi(i)) = i & 15.  D = 64 (128-byte rows,
  // bank group 8 (r & 1) + chunk): gk(pi(i)) = (i >> 1) & 7, so the 16 lanes
  // of a 128-bit read (rows pi(0..15)) hit 16 distinct bank groups.
  __device__ static constexpr int gk(int r) {
    return CPR == 16 ? ((r & 3) | (((r >> 3) & 1) << 2) | (((r >> 2) & 1) << 3))
                     : (((r >> 1) & 1) | (((r >> 3) & 1) << 1) | (((r >> 2) & 1) << 2));
  }
  __device__ static constexpr int sv(int r) { return CPR == 16 ? 4 * (r & 3) : 4 * ((r >> 1) & 1); }
};

// Direct-to-LDS loads of tile rows [key0, key0 + 64) by the 4 waves of one
// group (wave index gw): NI instructions each, 64 lanes x 16 bytes per
// instruction.  Not predicated: the descriptor's extent ends at the last row
// of this (b, kv head), so rows past it read as zero (and are masked, or
// belong to a tile that is never used).  k0b = key0 * row stride in bytes;
// off: this lane's row in the instruction times the row stride plus its
// swizzled chunk.
// kAux: the loads' cache policy (0: cached; kDmaStream: non-temporal, for
// data read exactly once).
constexpr int kDmaStream = 2;
template <int D, int kAux = 0>
__device__ inline void issue_tile_dma(char* __restrict__ lds, __amdgpu_buffer_rsrc_t rsrc, uint32_t k0b,
                                      uint32_t rowb, uint32_t off, int gw) {
  using ST = FwdStage<D>;
  typedef __attribute__((address_space(3))) void lds_void;
#pragma unroll
  for (int j = 0; j < ST::NI; ++j) {
    const int step = j * 4 + gw;  // instruction index within the tile
    lds_void* l = (lds_void*)(lds + step * 1024);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, l, 16, off, k0b + (uint32_t)(step * ST::RPI) * rowb, 0, kAux);
  }
}

typedef short s16x4 __attribute__((__vector_size__(4 * sizeof(short))));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ inline u32x2 ld_tr(const char* p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p)));
}

// s_waitcnt immediates (gfx9 encoding): vmcnt(n) alone, and lgkmcnt(0) alone.
__device__ constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }
constexpr int kLgkm0 = 0xC07F;

// Workgroup barrier between phases, without a memory fence: this wave's LDS
// reads are complete (lgkmcnt(0)); completion of its LDS-DMA loads is waited
// for explicitly, where the schedule needs it.  The empty asm statements keep
// the compiler from moving memory accesses across the barrier.
__device__ inline void phase_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(kLgkm0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

// Keep a value computed in the current phase: without it the compiler may
// sink the computation past the barrier, next to its use in the next phase,
// which would move VALU work into an MFMA phase.
template <typename V>
__device__ inline void pin(V& x) {
  asm volatile("" : "+v"(x));
}

// v_max3_f32 without the canonicalising moves the compiler adds in front of
// fmaxf on MFMA results (finite or -inf here; no NaN handling needed).
__device__ inline float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

}  // namespace gqa
