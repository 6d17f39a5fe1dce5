// K3: covariance-aware block scores and deterministic per-row top-k.
//
// Reference: svg/kernels/triton/group_pisa_attention.py:365-375
//   score = einsum(qc, kc * scale) + log(h_norm + 1e-6) [+ randn per key block]
//   indices = topk(score, NS).indices  (descending)
// Scores are fp32 here (the reference's einsum runs in the input dtype; parity
// is defined against fp32 math).  torch.topk leaves the order of equal scores
// unspecified; this kernel fixes it: (score desc, index asc), -0.0 == +0.0.
//
// Stage 1 (k3_scores): a 64x64-tile fp32 GEMM per (slice, tile), VALU FMA with
//   a fixed d-order, plus the per-key-block log bias.
// Stage 2 (k3_topk): one wavefront per row sorts 64-bit keys
//   (orderable(score) << 32 | ~index) with a bitonic network in LDS, emits the
//   first NS indices and the selection bitmask (one bit per key block).
#include "common.h"
#include "kernels.h"

namespace pasa {

constexpr int kScoreTile = 64;
constexpr int kScoreKC = 32;

__global__ __launch_bounds__(256) void k3_scores(const float* __restrict__ qc,
                                                 const float* __restrict__ kc,
                                                 const float* __restrict__ hnorm,
                                                 const float* __restrict__ noise, float scale,
                                                 int use_cov_bias, float* __restrict__ scores,
                                                 int NT, int D) {
  __shared__ float As[kScoreTile][kScoreKC + 1];
  __shared__ float Bs[kScoreTile][kScoreKC + 1];
  const int bh = blockIdx.z;
  const int i0 = blockIdx.y * kScoreTile;
  const int j0 = blockIdx.x * kScoreTile;
  const int tid = threadIdx.x;
  const int tx = tid & 15;
  const int ty = tid >> 4;
  const float* qb = qc + (int64_t)bh * NT * D;
  const float* kb = kc + (int64_t)bh * NT * D;

  float acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = 0.f;

  for (int d0 = 0; d0 < D; d0 += kScoreKC) {
    __syncthreads();
    for (int u = tid; u < kScoreTile * kScoreKC; u += 256) {
      const int r = u / kScoreKC;
      const int c = u - r * kScoreKC;
      const int gi = i0 + r;
      const int gj = j0 + r;
      As[r][c] = gi < NT ? qb[(int64_t)gi * D + d0 + c] : 0.f;
      Bs[r][c] = gj < NT ? scale * kb[(int64_t)gj * D + d0 + c] : 0.f;  // kc * scale first
    }
    __syncthreads();
#pragma unroll 8
    for (int c = 0; c < kScoreKC; ++c) {
      float av[4], bv[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) av[a] = As[ty + 16 * a][c];
#pragma unroll
      for (int b = 0; b < 4; ++b) bv[b] = Bs[tx + 16 * b][c];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = fmaf(av[a], bv[b], acc[a][b]);
    }
  }
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int gj = j0 + tx + 16 * b;
    if (gj >= NT) continue;
    float bias = 0.f;
    if (use_cov_bias) {
      bias = logf(hnorm[(int64_t)bh * NT + gj] + 1e-6f);
      if (noise) bias = bias + noise[(int64_t)bh * NT + gj];
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int gi = i0 + ty + 16 * a;
      if (gi < NT) scores[((int64_t)bh * NT + gi) * NT + gj] = acc[a][b] + bias;
    }
  }
}

__device__ __forceinline__ uint64_t topk_key(float s, int j) {
  uint32_t bits = __float_as_uint(s);
  if ((bits & 0x7fffffffu) == 0) bits = 0;  // -0.0 == +0.0
  const uint32_t ord = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - (uint32_t)j);
}

// One wavefront per (slice, query block).  Dynamic LDS: NTP * 8 bytes.
__global__ __launch_bounds__(64) void k3_topk(const float* __restrict__ scores, int NT, int NTP,
                                              int NS, int NW, int32_t* __restrict__ idx,
                                              uint32_t* __restrict__ selmask) {
  extern __shared__ uint64_t keys[];
  __shared__ uint32_t words[kMaxSelectBlocks / 32];
  const int row = blockIdx.x;
  const int bh = blockIdx.y;
  const int lane = threadIdx.x;
  const float* srow = scores + ((int64_t)bh * NT + row) * NT;

  for (int i = lane; i < NTP; i += 64) keys[i] = i < NT ? topk_key(srow[i], i) : 0ull;
  for (int w = lane; w < NW; w += 64) words[w] = 0u;
  __syncthreads();

  for (int kk = 2; kk <= NTP; kk <<= 1) {
    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
      for (int p = lane; p < (NTP >> 1); p += 64) {
        const int i = ((p & ~(jj - 1)) << 1) | (p & (jj - 1));
        const int l = i + jj;
        const uint64_t a = keys[i];
        const uint64_t b = keys[l];
        const bool desc = (i & kk) == 0;
        if (desc ? (a < b) : (a > b)) {
          keys[i] = b;
          keys[l] = a;
        }
      }
      __syncthreads();
    }
  }

  int32_t* irow = idx + ((int64_t)bh * NT + row) * NS;
  for (int i = lane; i < NS; i += 64) {
    const int j = (int)(0xffffffffu - (uint32_t)(keys[i] & 0xffffffffull));
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
  hipLaunchKernelGGL(k3_scores, grid, dim3(256), 0, stream, qc, kc, hnorm, noise, scale,
                     use_cov_bias, scores, NT, D);
  return hipGetLastError();
}

hipError_t launch_topk(const float* scores, int bh, int NT, int NS, int32_t* idx,
                       uint32_t* selmask, hipStream_t stream) {
  int NTP = 1;
  while (NTP < NT) NTP <<= 1;
  if (NTP < 2) NTP = 2;
  const int NW = (NT + 31) / 32;
  dim3 grid(NT, bh);
  hipLaunchKernelGGL(k3_topk, grid, dim3(64), (size_t)NTP * sizeof(uint64_t), stream, scores, NT,
                     NTP, NS, NW, idx, selmask);
  return hipGetLastError();
}

}  // namespace pasa
