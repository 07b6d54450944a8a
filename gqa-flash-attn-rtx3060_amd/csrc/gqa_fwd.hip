// gqa_fwd.hip — single-pass group-packed GQA forward for gfx950.
//
// Replaces the Triton kernel gqa_fwd_kernel (reference
// gqa_kernels/gqa_fwd.py:33-109).  One workgroup = 4 waves = 128 packed
// query rows of ONE (batch, kv head): G query heads x block_m positions
// (row r -> head r / block_m, position r % block_m, as gqa_fwd.py:58-63), so
// each K/V tile staged in LDS feeds the whole query group.  Per 64-key tile:
//   S^T = K Q^T        (bf16/f16 MFMA 32x32x16, fp32 accumulate)
//   online softmax     (exp2 domain, scale applied in fp32, gqa_fwd.py:98-101)
//   O^T += V^T P^T     (P rounded to the input type, gqa_fwd.py:103)
// K/V tiles are double-buffered in LDS; the next tile's global loads are in
// flight while the current one is computed (K straight into LDS by buffer
// loads with the LDS-DMA form, V through registers and a transposing store).  Causal: the key loop stops at
// the workgroup's last visible key (gqa_fwd.py:70-73) and masks only the
// tiles that cross the diagonal or the end of the keys.
#include <type_traits>

#include "gqa_common.hpp"
#include "gqa_params.hpp"

namespace gqa {

template <int DT, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gqa_fwd_kernel(FwdParams p) {
  using E = Elem<DT>;
  using T = typename E::T;
  using FT = FwdTile<D>;
  constexpr int CPR = FT::CPR;
  constexpr int RPI = 64 / CPR;
  constexpr int KPT = VRegs<D>::KPT;
  // Two separate arrays (not one array of two halves): the compiler can then
  // tell the DMA target of the next tile from the buffer being read, and does
  // not wait for the in-flight loads before the reads of the current tile.
  __shared__ __attribute__((aligned(1024))) char smem0[FT::kBytes];
  __shared__ __attribute__((aligned(1024))) char smem1[FT::kBytes];

  const Dims& dm = p.dm;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6) & 3;  // wave-uniform (SGPR), 0..3
  const int i = lane & 31, hh = lane >> 5;

  // Work item: heavy (late) query blocks first under causal, and every XCD
  // gets a contiguous range of items (same kv head -> same L2).
  const int total = p.n_mblk * dm.Hkv * dm.B;
  const int w = xcd_remap(blockIdx.x, total);
  const int bh = w / p.n_mblk;
  const int mrank = w - bh * p.n_mblk;
  const int pid_m = dm.causal ? (p.n_mblk - 1 - mrank) : mrank;
  const int b = bh / dm.Hkv, kvh = bh - b * dm.Hkv;

  // This lane's query row.
  const int r = wave * 32 + i;
  const int g = r / p.block_m, ml = r - g * p.block_m;
  const int pos = pid_m * p.block_m + ml;
  const bool valid = (g < dm.G) && (pos < dm.Sq);
  const int head = kvh * dm.G + (g < dm.G ? g : 0);
  const int qpos = pos + (dm.Skv - dm.Sq);

  u32x4 qreg[D / 16];
  {
    const T* qrow = static_cast<const T*>(p.q.ptr) + (int64_t)b * p.q.sb + (int64_t)head * p.q.sh +
                    (int64_t)(valid ? pos : 0) * p.q.ss;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      u32x4 x = {0u, 0u, 0u, 0u};
      if (valid) x = *reinterpret_cast<const u32x4*>(qrow + 16 * ks + 8 * hh);
      qreg[ks] = x;
    }
  }

  // Key range of this workgroup.
  const int pos_lo = pid_m * p.block_m;
  const int pos_hi = min(pos_lo + p.block_m, dm.Sq) - 1;
  int kv_end = dm.Skv;
  if (dm.causal) kv_end = min(dm.Skv, pos_hi + (dm.Skv - dm.Sq) + 1);
  kv_end = max(kv_end, 0);
  const int ntiles = (kv_end + FT::kKeys - 1) / FT::kKeys;
  const int qpos_lo = pos_lo + (dm.Skv - dm.Sq);

  // Global side: buffer descriptors over this (b, kv head)'s K and V rows,
  // each ending at the last byte of row seq_kv - 1 so that rows past the end
  // read as zero (the host guarantees seq_kv * key stride * 2 < 2^31), and
  // per-lane offsets.
  const uint32_t kssb = (uint32_t)(2 * p.k.ss), vssb = (uint32_t)(2 * p.v.ss);
  const char* kbh = static_cast<const char*>(p.k.ptr) + 2 * ((int64_t)b * p.k.sb + (int64_t)kvh * p.k.sh);
  const char* vbh = static_cast<const char*>(p.v.ptr) + 2 * ((int64_t)b * p.v.sb + (int64_t)kvh * p.v.sh);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbh, (uint32_t)(dm.Skv - 1) * kssb + 2 * D);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbh, (uint32_t)(dm.Skv - 1) * vssb + 2 * D);
  const int lrow = lane / CPR;
  const uint32_t koff =
      (uint32_t)(lrow * kssb) + 16u * (uint32_t)((lane % CPR) ^ FT::gk((wave * RPI + lrow) & 15));
  const int d4 = t % (D / 4), kg = t / (D / 4);
  const uint32_t voff = (uint32_t)(kg * KPT * vssb) + 8u * (uint32_t)d4;

  // LDS side: per-lane read offsets (the tile buffer, the 32-key block and
  // the 32-row d block are immediate offsets on top of these).  The masks are
  // no-ops on the values; they give the compiler known bounds, so it can prove
  // that reads of one buffer never touch the other and does not wait for the
  // next tile's in-flight loads.
  constexpr uint32_t kKMask = (FT::kKBytes / 2 - 1) & ~15u;  // rows 0..31 of K
  constexpr uint32_t kVMask = (FT::kBytes - 1) & ~15u;
  uint32_t ka[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
    ka[ks] = (uint32_t)(pi_key(i) * (2 * D) + 16 * ((2 * ks + hh) ^ (i & (CPR - 1)))) & kKMask;
  uint32_t va[2][2];
  {
    const int z = hh ^ FT::f0(i);
#pragma unroll
    for (int mp = 0; mp < 2; ++mp)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        va[mp][kk] = (uint32_t)(FT::kKBytes + 128 * i + 16 * ((4 * mp + 2 * kk) ^ z)) & kVMask;
  }

  f32x16 acc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) acc[db] = f32x16{};
  float m_run = -__builtin_inff();
  float l_run = 0.f;
  const float c = dm.c;

  VRegs<D> R;
  if (ntiles > 0) {
    issue_k_dma<D>(smem0, rk, 0u, kssb, koff, wave);
    load_v_regs<D>(R, rv, 0u, vssb, voff);
    store_v_lds<D>(smem0, R, t);
  }
  __syncthreads();

  auto step = [&](auto bufc, int it) {
    constexpr int BUF = decltype(bufc)::value;
    const char* cur = BUF ? smem1 : smem0;
    char* nxt = BUF ? smem0 : smem1;
    const int key0 = it * FT::kKeys;
    const bool has_next = it + 1 < ntiles;
    if (has_next) {
      const uint32_t k1 = (uint32_t)(key0 + FT::kKeys);
      issue_k_dma<D>(nxt, rk, k1 * kssb, kssb, koff, wave);
      load_v_regs<D>(R, rv, k1 * vssb, vssb, voff);
    }
    __builtin_amdgcn_sched_barrier(0);

    // S^T = K Q^T for the two 32-key blocks, the chains interleaved and each
    // K operand read from LDS four MFMAs ahead of its use.
    f32x16 sc[2];
    sc[0] = f32x16{};
    sc[1] = f32x16{};
    {
      u32x4 ak[D / 16][2];
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
          ak[ks][mb] = *reinterpret_cast<const u32x4*>(cur + mb * 32 * (2 * D) + ka[ks]);
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) sc[mb] = E::mfma(ak[ks][mb], qreg[ks], sc[mb]);
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // 4 LDS reads
#pragma unroll
      for (int j = 0; j < D / 8 - 4; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // last 4 MFMAs
    }

    const bool need_mask = (key0 + FT::kKeys > dm.Skv) || (dm.causal && key0 + FT::kKeys - 1 > qpos_lo);
    if (need_mask) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = key0 + 32 * mb + key_of(v, hh);
          const bool off = key >= dm.Skv || (dm.causal && key > qpos);
          sc[mb][v] = off ? -__builtin_inff() : sc[mb][v];
        }
    }
    const float nmc = softmax_rescale<D / 32>(sc, m_run, l_run, acc, c);
    // P of block 0 feeds its PV MFMAs while block 1 is exponentiated.
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      u32x4 pk[2];
      softmax_exp<DT>(sc[mb], nmc, l_run, c, pk);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(cur + 4096 * db + va[mb ^ (db & 1)][kk]);
          acc[db] = E::mfma(a, pk[kk], acc[db]);
        }
    }

    if (has_next) store_v_lds<D>(nxt, R, t);
    __syncthreads();
  };

  int it = 0;
  for (; it + 2 <= ntiles; it += 2) {
    step(std::integral_constant<int, 0>{}, it);
    step(std::integral_constant<int, 1>{}, it + 1);
  }
  if (it < ntiles) step(std::integral_constant<int, 0>{}, it);

  // Epilogue: o = acc / l (0/0 = NaN for a row with no visible key, as the
  // reference's acc / l_i at gqa_fwd.py:106).
  const float l_tot = xhalf_sum(l_run);
  const float inv = 1.0f / l_tot;
  if (valid) {
    T* orow = static_cast<T*>(const_cast<void*>(p.o.ptr)) + (int64_t)b * p.o.sb +
              (int64_t)head * p.o.sh + (int64_t)pos * p.o.ss;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x2 x;
        x[0] = E::pack2(acc[db][4 * j] * inv, acc[db][4 * j + 1] * inv);
        x[1] = E::pack2(acc[db][4 * j + 2] * inv, acc[db][4 * j + 3] * inv);
        *reinterpret_cast<u32x2*>(orow + 32 * db + 8 * j + 4 * hh) = x;
      }
  }
}

template <int DT, int D>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
  const int total = p.n_mblk * p.dm.Hkv * p.dm.B;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL((gqa_fwd_kernel<DT, D>), dim3(total), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_fwd(const FwdParams& p, int dtype, hipStream_t stream) {
  if (dtype == 0) return p.dm.D == 128 ? launch_fwd_t<0, 128>(p, stream) : launch_fwd_t<0, 64>(p, stream);
  return p.dm.D == 128 ? launch_fwd_t<1, 128>(p, stream) : launch_fwd_t<1, 64>(p, stream);
}

}  // namespace gqa
