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
// flight while the current one is computed.  Causal: the key loop stops at
// the workgroup's last visible key (gqa_fwd.py:70-73) and masks only the
// tiles that cross the diagonal or the end of the keys.
#include "gqa_common.hpp"
#include "gqa_params.hpp"

namespace gqa {

template <int DT, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gqa_fwd_kernel(FwdParams p) {
  using E = Elem<DT>;
  using T = typename E::T;
  using ST = SubTile<D>;
  __shared__ __attribute__((aligned(16))) char smem[2 * ST::kBytes];

  const Dims& dm = p.dm;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
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
  const int ntiles = (kv_end + kFwdTileKeys - 1) / kFwdTileKeys;
  const int qpos_lo = pos_lo + (dm.Skv - dm.Sq);

  const T* kbase = static_cast<const T*>(p.k.ptr) + (int64_t)b * p.k.sb + (int64_t)kvh * p.k.sh;
  const T* vbase = static_cast<const T*>(p.v.ptr) + (int64_t)b * p.v.sb + (int64_t)kvh * p.v.sh;

  f32x16 acc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) acc[db] = f32x16{};
  float m_run = -__builtin_inff();
  float l_run = 0.f;
  const float c = dm.c;

  SubTileRegs<D> R;
  if (ntiles > 0) {
    load_subtile<D, T>(R, kbase, vbase, p.k.ss, p.v.ss, 0, dm.Skv, t);
    store_subtile<D>(smem, R, t);
  }
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const char* cur = smem + (it & 1) * ST::kBytes;
    const int key0 = it * kFwdTileKeys;
    const bool has_next = it + 1 < ntiles;
    if (has_next) load_subtile<D, T>(R, kbase, vbase, p.k.ss, p.v.ss, key0 + kFwdTileKeys, dm.Skv, t);

    const bool need_mask =
        (key0 + kFwdTileKeys > dm.Skv) || (dm.causal && key0 + kFwdTileKeys - 1 > qpos_lo);
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      f32x16 s = qk_block<DT, D>(cur, qreg, mb, lane);
      if (need_mask) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = key0 + 32 * mb + key_of(v, hh);
          const bool off = key >= dm.Skv || (dm.causal && key > qpos);
          s[v] = off ? -__builtin_inff() : s[v];
        }
      }
      u32x4 pk[2];
      softmax_block<DT, D / 32>(s, m_run, l_run, acc, c, pk);
      pv_block<DT, D>(cur, pk, acc, mb, lane);
    }

    if (has_next) store_subtile<D>(smem + ((it + 1) & 1) * ST::kBytes, R, t);
    __syncthreads();
  }

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
