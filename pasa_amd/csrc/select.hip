// K3: covariance-aware block scores and deterministic per-row top-k.
//
// Reference: svg/kernels/triton/group_pisa_attention.py:365-375
//   score = einsum(qc, kc * scale) + log(h_norm + 1e-6) [+ randn per key block]
//   indices = topk(score, NS).indices  (descending)
// Scores are fp32 here (the reference's einsum runs in the input dtype; parity
// is defined against fp32 math).  torch.topk leaves the order of equal scores
// unspecified; this kernel fixes it: (score desc, index asc), -0.0 == +0.0.
//
// Stage 1 (k3_scores): a 64x64-tile fp32 GEMM per (slice, tile) on the fp32 MFMA,
//   with a fixed d-order, plus the per-key-block log bias.
// Stage 2 (k3_topk): one wavefront per row finds the NS-th largest score with a
//   4-pass radix select over the orderable 32-bit score, takes the ties at it by
//   lowest index, sorts the NS selected 64-bit keys (orderable(score) << 32 | ~index)
//   with a bitonic network in LDS, and emits the indices and the selection bitmask
//   (one bit per key block).
#include "common.h"
#include "kernels.h"

namespace pasa {

constexpr int kScoreTile = 64;

// One workgroup per 64 x 64 tile of one slice's score matrix, one 32 x 32 sub-tile per
// wave, on the fp32 MFMA (v_mfma_f32_32x32x2_f32: twice the rate of scalar fp32 FMAs).
// The dot product over d is taken in a fixed permuted order: in step s the lanes of
// half-wave hh supply d = hh * D/2 + s, so a lane walks contiguous d and one 16-byte LDS
// read feeds four MFMAs.  Rows are staged in LDS as fp32 with a 4-float pad; kc * scale is
// rounded to fp32 before the product, as the reference computes it.
template <int D>
__global__ __launch_bounds__(256) void k3_scores(const float* __restrict__ qc,
                                                 const float* __restrict__ kc,
                                                 const float* __restrict__ hnorm,
                                                 const float* __restrict__ noise, float scale,
                                                 int use_cov_bias, float* __restrict__ scores, int NT) {
  constexpr int RS = D + 4;  // padded row stride (floats)
  __shared__ __attribute__((aligned(16))) float As[kScoreTile * RS];
  __shared__ __attribute__((aligned(16))) float Bs[kScoreTile * RS];
  const int bh = blockIdx.z;
  const int i0 = blockIdx.y * kScoreTile;
  const int j0 = blockIdx.x * kScoreTile;
  const int tid = threadIdx.x;
  const float* qb = qc + (int64_t)bh * NT * D;
  const float* kb = kc + (int64_t)bh * NT * D;
  // Stage 64 rows of qc and of scale * kc, 16 bytes per thread per step.
  constexpr int C4 = D / 4;  // float4 per row
  for (int u = tid; u < kScoreTile * C4; u += 256) {
    const int r = u / C4;
    const int c4 = u - r * C4;
    const int gi = i0 + r;
    const int gj = j0 + r;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    if (gi < NT) a = *reinterpret_cast<const float4*>(qb + (int64_t)gi * D + 4 * c4);
    if (gj < NT) {
      b = *reinterpret_cast<const float4*>(kb + (int64_t)gj * D + 4 * c4);
      b = make_float4(scale * b.x, scale * b.y, scale * b.z, scale * b.w);  // kc * scale first
    }
    *reinterpret_cast<float4*>(As + r * RS + 4 * c4) = a;
    *reinterpret_cast<float4*>(Bs + r * RS + 4 * c4) = b;
  }
  __syncthreads();
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int ar = (wave >> 1) * 32 + l32;  // row of A (query block) this lane supplies
  const int br = (wave & 1) * 32 + l32;   // row of B (key block)
  const float* ap = As + ar * RS + hh * (D / 2);
  const float* bp = Bs + br * RS + hh * (D / 2);
  f32x16_t acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
  for (int s4 = 0; s4 < D / 8; ++s4) {
    const float4 a = *reinterpret_cast<const float4*>(ap + 4 * s4);
    const float4 b = *reinterpret_cast<const float4*>(bp + 4 * s4);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, acc, 0, 0, 0);
  }
  // C: row (query block) 8(r>>2) + 4hh + (r&3) of the wave's sub-tile, column (key block) l32.
  const int gj = j0 + (wave & 1) * 32 + l32;
  if (gj >= NT) return;
  float bias = 0.f;
  if (use_cov_bias) {
    bias = logf(hnorm[(int64_t)bh * NT + gj] + 1e-6f);
    if (noise) bias = bias + noise[(int64_t)bh * NT + gj];
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int gi = i0 + (wave >> 1) * 32 + mfma32_row(r, hh);
    if (gi < NT) scores[((int64_t)bh * NT + gi) * NT + gj] = acc[r] + bias;
  }
}

// Inclusive prefix sum over the 64 lanes of a wavefront.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t t = __shfl_up(x, d, 64);
    if (lane >= d) x += t;
  }
  return x;
}

// Order-preserving map of fp32 scores to uint32 (-0.0 == +0.0).
__device__ __forceinline__ uint32_t score_ord(float s) {
  uint32_t bits = __float_as_uint(s);
  if ((bits & 0x7fffffffu) == 0) bits = 0;
  return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}

// One wavefront per row.  The row's ordered scores stay in registers (KPL per lane,
// index j = 64 i + lane).  An MSB-first radix select over the 32-bit ordered score
// (4 passes of 8 bits; each pass histograms the keys still matching the prefix, in
// kCopies LDS copies picked by lane so that equal digits spread their atomics) finds
// the NS-th largest score T and how many of the scores equal to T are taken; those
// are the lowest indices (ties go to the lowest index).  The NS selected keys
// (score << 32 | ~index) are compacted into LDS and sorted descending there with a
// bitonic network.  Dynamic LDS: NSP * 8 bytes (NSP = pow2 >= NS).
template <int KPL>
__global__ __launch_bounds__(64) void k3_topk(const float* __restrict__ scores, int NT, int NS, int NSP,
                                              int NW, int32_t* __restrict__ idx,
                                              uint32_t* __restrict__ selmask) {
  constexpr int kCopies = 2;
  extern __shared__ uint64_t sel[];
  __shared__ uint32_t hist[kCopies][256];
  __shared__ uint32_t words[kMaxSelectBlocks / 32];
  const int row = blockIdx.x;
  const int bh = blockIdx.y;
  const int lane = threadIdx.x;
  const float* srow = scores + ((int64_t)bh * NT + row) * NT;

  uint32_t ok[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int j = i * 64 + lane;
    ok[i] = j < NT ? score_ord(srow[j]) : 0u;
  }
  for (int w = lane; w < NW; w += 64) words[w] = 0u;

  uint32_t prefix = 0u, mask = 0u;
  uint32_t need = (uint32_t)NS;  // rank of the threshold among the scores matching prefix
  uint32_t* myhist = hist[lane & (kCopies - 1)];
#pragma unroll 1
  for (int shift = 24; shift >= 0; shift -= 8) {
#pragma unroll
    for (int t = 0; t < 4 * kCopies; ++t) (&hist[0][0])[t * 64 + lane] = 0u;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < KPL; ++i)
      if (i * 64 + lane < NT && (ok[i] & mask) == prefix) atomicAdd(&myhist[(ok[i] >> shift) & 255u], 1u);
    __syncthreads();
    uint32_t hb[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint32_t x = 0u;
#pragma unroll
      for (int cp = 0; cp < kCopies; ++cp) x += hist[cp][4 * lane + t];
      hb[t] = x;
    }
    const uint32_t s = hb[0] + hb[1] + hb[2] + hb[3];
    const uint32_t incl = wave_incl_scan(s);
    const uint32_t total = __shfl(incl, 63, 64);
    uint32_t cum = total - incl;  // candidates in the bins of higher lanes
    int found = -1;
    uint32_t above = 0u;
#pragma unroll
    for (int t = 3; t >= 0; --t) {
      if (found < 0 && cum < need && need <= cum + hb[t]) {
        found = 4 * lane + t;
        above = cum;
      }
      cum += hb[t];
    }
    const uint64_t hit = __ballot(found >= 0);
    const int src = __ffsll((long long)hit) - 1;
    const uint32_t bin = (uint32_t)__shfl(found, src, 64);
    need -= (uint32_t)__shfl((int)above, src, 64);
    prefix |= bin << shift;
    mask |= 0xffu << shift;
  }
  // prefix = T, the NS-th largest ordered score; every score above T is selected and,
  // of the scores equal to T, the `need` with the lowest indices.
  uint32_t taken = 0u;  // ties at T taken so far (in index order)
  uint32_t cnt = 0u;
  uint64_t lt = (1ull << lane) - 1ull;
  bool pick[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const bool valid = i * 64 + lane < NT;
    const bool tie = valid && ok[i] == prefix;
    const uint64_t tb = __ballot(tie);
    const uint32_t rank = taken + (uint32_t)__popcll(tb & lt);
    pick[i] = valid && (ok[i] > prefix || (tie && rank < need));
    taken += (uint32_t)__popcll(tb);
    cnt += pick[i] ? 1u : 0u;
  }
  uint32_t pos = wave_incl_scan(cnt) - cnt;
#pragma unroll
  for (int i = 0; i < KPL; ++i)
    if (pick[i]) sel[pos++] = ((uint64_t)ok[i] << 32) | (uint64_t)(0xffffffffu - (uint32_t)(i * 64 + lane));
  for (int i = NS + lane; i < NSP; i += 64) sel[i] = 0ull;
  __syncthreads();

  for (int kk = 2; kk <= NSP; kk <<= 1) {
    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
      for (int p = lane; p < (NSP >> 1); p += 64) {
        const int i = ((p & ~(jj - 1)) << 1) | (p & (jj - 1));
        const int l = i + jj;
        const uint64_t a = sel[i];
        const uint64_t b = sel[l];
        const bool desc = (i & kk) == 0;
        if (desc ? (a < b) : (a > b)) {
          sel[i] = b;
          sel[l] = a;
        }
      }
      __syncthreads();
    }
  }

  int32_t* irow = idx + ((int64_t)bh * NT + row) * NS;
  for (int i = lane; i < NS; i += 64) {
    const int j = (int)(0xffffffffu - (uint32_t)(sel[i] & 0xffffffffull));
    irow[i] = j;
    atomicOr(&words[j >> 5], 1u << (j & 31));
  }
  __syncthreads();
  uint32_t* mrow = selmask + ((int64_t)bh * NT + row) * NW;
  for (int w = lane; w < NW; w += 64) mrow[w] = words[w];
}

hipError_t launch_scores(const float* qc, const float* kc, const float* hnorm, const float* noise,
                         float scale, int use_cov_bias, float* scores, int bh, int NT, int D,
                         hipStream_t stream) {
  dim3 grid((NT + kScoreTile - 1) / kScoreTile, (NT + kScoreTile - 1) / kScoreTile, bh);
  if (D == 128)
    hipLaunchKernelGGL(k3_scores<128>, grid, dim3(256), 0, stream, qc, kc, hnorm, noise, scale, use_cov_bias,
                       scores, NT);
  else if (D == 64)
    hipLaunchKernelGGL(k3_scores<64>, grid, dim3(256), 0, stream, qc, kc, hnorm, noise, scale, use_cov_bias,
                       scores, NT);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_topk(const float* scores, int bh, int NT, int NS, int32_t* idx,
                       uint32_t* selmask, hipStream_t stream) {
  int NSP = 1;
  while (NSP < NS) NSP <<= 1;
  if (NSP < 2) NSP = 2;
  const int NW = (NT + 31) / 32;
  dim3 grid(NT, bh);
  const size_t lds = (size_t)NSP * sizeof(uint64_t);
#define PASA_TOPK(K) \
  hipLaunchKernelGGL((k3_topk<K>), grid, dim3(64), lds, stream, scores, NT, NS, NSP, NW, idx, selmask)
  if (NT <= 64 * 4)
    PASA_TOPK(4);
  else if (NT <= 64 * 8)
    PASA_TOPK(8);
  else if (NT <= 64 * 16)
    PASA_TOPK(16);
  else if (NT <= 64 * 32)
    PASA_TOPK(32);
  else if (NT <= 64 * 64)
    PASA_TOPK(64);
  else
    return hipErrorInvalidValue;
#undef PASA_TOPK
  return hipGetLastError();
}

}  // namespace pasa
