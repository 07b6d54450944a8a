// gqa_cache.hip — paged KV cache write for gfx950.
//
// Stores the K and V rows of new tokens into the paged caches
// (num_blocks, block_size, Hkv, D) at the slots the caller assigned
// (slot = block * block_size + offset; negative slots are padding and are
// skipped).  Pure data movement: each thread moves one 16-byte chunk of K and
// the matching chunk of V, so consecutive threads read consecutive bytes of
// one token's rows and write consecutive bytes of its cache slot.
#include <hip/hip_runtime.h>

#include "gqa_common.hpp"
#include "gqa_params.hpp"

namespace gqa {

__global__ __launch_bounds__(256) void gqa_paged_cache_write_kernel(CacheWriteParams p) {
  const int cpr = p.D * p.elem_bytes / 16;  // 16-byte chunks per (token, head) row
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)p.n_tokens * p.Hkv * cpr;
  if (idx >= total) return;
  const int c = (int)(idx % cpr);
  const int64_t th = idx / cpr;
  const int h = (int)(th % p.Hkv);
  const int64_t tok = th / p.Hkv;
  const int64_t slot = p.slots[tok];
  if (slot < 0) return;
  const int64_t blk = slot >> p.block_shift;
  const int64_t off = slot & ((1 << p.block_shift) - 1);
  const int64_t eb = p.elem_bytes;
  const char* ks = static_cast<const char*>(p.k) + (tok * p.k_st + h * p.k_sh) * eb + 16 * c;
  const char* vs = static_cast<const char*>(p.v) + (tok * p.v_st + h * p.v_sh) * eb + 16 * c;
  char* kd = const_cast<char*>(static_cast<const char*>(p.kc.ptr)) +
             (blk * p.kc.sb + off * p.kc.ss + h * p.kc.sh) * eb + 16 * c;
  char* vd = const_cast<char*>(static_cast<const char*>(p.vc.ptr)) +
             (blk * p.vc.sb + off * p.vc.ss + h * p.vc.sh) * eb + 16 * c;
  const u32x4 kx = *reinterpret_cast<const u32x4*>(ks);
  const u32x4 vx = *reinterpret_cast<const u32x4*>(vs);
  *reinterpret_cast<u32x4*>(kd) = kx;
  *reinterpret_cast<u32x4*>(vd) = vx;
}

hipError_t launch_paged_cache_write(const CacheWriteParams& p, hipStream_t stream) {
  const int64_t total = (int64_t)p.n_tokens * p.Hkv * (p.D * p.elem_bytes / 16);
  if (total <= 0) return hipSuccess;
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL(gqa_paged_cache_write_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace gqa
