// K1: frame-major <-> token-major layout permutation of [BH, S, D] tensors.
//
// Reference: svg/models/hyvideo/placement.py — closed forms :6-31, forward
// (temporal-head) kernel branch :73-100, inverse kernel branch :320-343.  The
// reference walks source rows and scatters; here each thread owns one 16-byte
// chunk of a DESTINATION row and gathers it, so every wavefront writes whole,
// contiguous destination rows (coalesced stores) and reads whole source rows.
// Up to three tensors share one launch (the index math is computed once).
#include "common.h"
#include "kernels.h"

namespace pasa {

template <int NTENS>
__global__ __launch_bounds__(256) void k1_permute(
    const u32x4_t* __restrict__ s0, const u32x4_t* __restrict__ s1,
    const u32x4_t* __restrict__ s2, u32x4_t* __restrict__ d0, u32x4_t* __restrict__ d1,
    u32x4_t* __restrict__ d2,
    int S, int F, int P, int ctx, int chunks_per_row, int rows_per_wg,
    const int32_t* __restrict__ head_is_temporal, int inverse) {
  const int bh = blockIdx.y;
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
  u32x4_t a = __builtin_nontemporal_load(s0 + so);
  u32x4_t b, c;
  if (NTENS > 1) b = __builtin_nontemporal_load(s1 + so);
  if (NTENS > 2) c = __builtin_nontemporal_load(s2 + so);
  __builtin_nontemporal_store(a, d0 + dof);
  if (NTENS > 1) __builtin_nontemporal_store(b, d1 + dof);
  if (NTENS > 2) __builtin_nontemporal_store(c, d2 + dof);
}

hipError_t launch_permute(const void* s0, const void* s1, const void* s2, void* d0, void* d1,
                          void* d2, int ntens, int bh, int S, int F, int P, int ctx,
                          int row_bytes, const int32_t* head_is_temporal, int inverse,
                          hipStream_t stream) {
  const int cpr = row_bytes / 16;
  const int threads = 256;
  const int rows_per_wg = cpr >= threads ? 1 : threads / cpr;
  if (cpr > threads) return hipErrorInvalidValue;  // rejected by the host validation
  dim3 grid((S + rows_per_wg - 1) / rows_per_wg, bh);
  auto a0 = (const u32x4_t*)s0;
  auto a1 = (const u32x4_t*)s1;
  auto a2 = (const u32x4_t*)s2;
  auto b0 = (u32x4_t*)d0;
  auto b1 = (u32x4_t*)d1;
  auto b2 = (u32x4_t*)d2;
  if (ntens == 1)
    hipLaunchKernelGGL(k1_permute<1>, grid, dim3(threads), 0, stream, a0, a1, a2, b0, b1, b2, S, F,
                       P, ctx, cpr, rows_per_wg, head_is_temporal, inverse);
  else if (ntens == 2)
    hipLaunchKernelGGL(k1_permute<2>, grid, dim3(threads), 0, stream, a0, a1, a2, b0, b1, b2, S, F,
                       P, ctx, cpr, rows_per_wg, head_is_temporal, inverse);
  else
    hipLaunchKernelGGL(k1_permute<3>, grid, dim3(threads), 0, stream, a0, a1, a2, b0, b1, b2, S, F,
                       P, ctx, cpr, rows_per_wg, head_is_temporal, inverse);
  return hipGetLastError();
}

}  // namespace pasa
