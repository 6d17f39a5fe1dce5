// K1: frame-major <-> token-major layout permutation of [BH, S, D] tensors.
//
// Reference: svg/models/hyvideo/placement.py — closed forms :6-31, forward
// (temporal-head) kernel branch :73-100, inverse kernel branch :320-343.  The
// reference walks source rows and scatters; here each thread owns one 16-byte
// chunk of a DESTINATION row and gathers it, so every wavefront writes whole,
// contiguous destination rows (coalesced stores) and reads whole source rows.
// Up to three tensors share one launch, one tensor per workgroup (blockIdx.z): a
// wavefront that moved the same chunk of all three at once ran at 5.6 TB/s, one tensor
// at a time at 6.2 TB/s (c2 forward, [40, 75600, 128] bf16 x 3).
#include "common.h"
#include "kernels.h"

namespace pasa {

__global__ __launch_bounds__(256) void k1_permute(
    const u32x4_t* __restrict__ s0, const u32x4_t* __restrict__ s1,
    const u32x4_t* __restrict__ s2, u32x4_t* __restrict__ d0, u32x4_t* __restrict__ d1,
    u32x4_t* __restrict__ d2,
    int S, int F, int P, int ctx, int chunks_per_row, int rows_per_wg,
    const int32_t* __restrict__ head_is_temporal, int inverse) {
  const int bh = blockIdx.y;
  const int t = blockIdx.z;  // which tensor
  const u32x4_t* __restrict__ src_t = t == 0 ? s0 : (t == 1 ? s1 : s2);
  u32x4_t* __restrict__ dst_t = t == 0 ? d0 : (t == 1 ? d1 : d2);
  const int local_row = threadIdx.x / chunks_per_row;
  const int chunk = threadIdx.x - local_row * chunks_per_row;
  const int r = blockIdx.x * rows_per_wg + local_row;
  if (local_row >= rows_per_wg || r >= S) return;

  int src = r;
  const bool permute = head_is_temporal == nullptr || head_is_temporal[bh] != 0;
  if (permute && r < S - ctx) {
    if (!inverse) {  // dst r = p*F + f  <-  src f*P + p
      const int p = r / F;
      const int f = r - p * F;
      src = f * P + p;
    } else {         // dst r = f*P + p  <-  src p*F + f
      const int f = r / P;
      const int p = r - f * P;
      src = p * F + f;
    }
  }
  const int64_t base = (int64_t)bh * S * chunks_per_row;
  const int64_t so = base + (int64_t)src * chunks_per_row + chunk;
  const int64_t dof = base + (int64_t)r * chunks_per_row + chunk;
  __builtin_nontemporal_store(__builtin_nontemporal_load(src_t + so), dst_t + dof);
}

hipError_t launch_permute(const void* s0, const void* s1, const void* s2, void* d0, void* d1,
                          void* d2, int ntens, int bh, int S, int F, int P, int ctx,
                          int row_bytes, const int32_t* head_is_temporal, int inverse,
                          hipStream_t stream) {
  const int cpr = row_bytes / 16;
  const int threads = 256;
  const int rows_per_wg = cpr >= threads ? 1 : threads / cpr;
  if (cpr > threads) return hipErrorInvalidValue;  // rejected by the host validation
  if (ntens < 1 || ntens > 3) return hipErrorInvalidValue;
  dim3 grid((S + rows_per_wg - 1) / rows_per_wg, bh, ntens);
  hipLaunchKernelGGL(k1_permute, grid, dim3(threads), 0, stream, (const u32x4_t*)s0, (const u32x4_t*)s1,
                     (const u32x4_t*)s2, (u32x4_t*)d0, (u32x4_t*)d1, (u32x4_t*)d2, S, F, P, ctx, cpr,
                     rows_per_wg, head_is_temporal, inverse);
  return hipGetLastError();
}

}  // namespace pasa
