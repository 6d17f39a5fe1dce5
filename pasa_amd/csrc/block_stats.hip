// K2: per-key-block statistics and the per-group first-order moment.
//
// Reference: fused_chunk_reduce_kernel, svg/kernels/triton/group_pisa_attention.py:66-129
// (means :101-102, value sum :103, H = K^T V - kc vc^T :106-107, ||H||^2 :110),
// sqrt on the host :287, and compute_h_group :291-301 (zero-padded mean over G).
//
// One workgroup (4 wavefronts) owns one group of G consecutive key blocks of one
// (batch, head) slice and walks its blocks in order.  Per block it streams the
// Q, K, V tiles from HBM once, forms the column sums with in-register partials
// reduced by shuffles and LDS (fixed order, deterministic), computes
// H_j = K_j^T V_j on bf16 MFMA (each wave owns one quadrant of the D x D
// matrix), subtracts kc vc^T, reduces ||H_j||_F and adds H_j into the group
// accumulator held in registers.  H_j is never written to memory; the group
// mean is written once per group.  All statistics are fp32.
#include "common.h"
#include "kernels.h"

namespace pasa {

template <int D, int BT>
__global__ __launch_bounds__(256, 1) void k2_block_stats(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, float* __restrict__ qc, float* __restrict__ kc,
    float* __restrict__ vc, float* __restrict__ hnorm, float* __restrict__ hgroup, int T, int Tslice,
    int NT, int G) {
  constexpr int CH = D / 8;                 // 16-byte chunks per row
  constexpr int ROWS_PER_PASS = 256 / CH;   // rows loaded per pass by the workgroup
  constexpr int PASSES = BT / ROWS_PER_PASS;
  constexpr int QD = D / 2;                 // quadrant side owned by one wave
  constexpr int TL = QD / 32;               // 32x32 MFMA tiles per quadrant side
  static_assert(PASSES >= 1 && BT % ROWS_PER_PASS == 0, "tile shape");

  using TL_ = PadTile<D>;
  __shared__ __attribute__((aligned(16))) unsigned char Ks[TL_::bytes(BT)];
  __shared__ __attribute__((aligned(16))) unsigned char Vs[TL_::bytes(BT)];
  __shared__ float red_sum[4][3 * D];
  __shared__ float colstat[3 * D];
  __shared__ float red_norm[4];

  const int g = blockIdx.x;
  const int bh = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;
  const int l32 = lane & 31;
  const int dq = (wave >> 1) * QD;
  const int eq = (wave & 1) * QD;

  const int j0 = g * G;
  const int j1 = min(j0 + G, NT);
  // Slices are Tslice rows apart; only the first T rows (the blocked segment) are
  // addressable through the buffer resources, so rows >= T read as zero.
  const int64_t slice = (int64_t)bh * Tslice * D;
  const uint32_t slice_bytes = (uint32_t)T * D * 2u;
  const rsrc_t qr = make_rsrc(q + slice, slice_bytes);
  const rsrc_t kr = make_rsrc(k + slice, slice_bytes);
  const rsrc_t vr = make_rsrc(v + slice, slice_bytes);

  f32x16_t gacc[TL][TL];
#pragma unroll
  for (int a = 0; a < TL; ++a)
#pragma unroll
    for (int b = 0; b < TL; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) gacc[a][b][r] = 0.f;

  const int prow = tid / CH;  // row within a pass
  const int pc = tid % CH;    // chunk within the row

  for (int j = j0; j < j1; ++j) {
    const int n = min(BT, T - j * BT);
    __syncthreads();  // previous block finished with Ks/Vs/colstat/red_sum

    float ps[3][8];
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int i = 0; i < 8; ++i) ps[a][i] = 0.f;

#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int t = p * ROWS_PER_PASS + prow;
      const uint32_t off = ((uint32_t)(j * BT + t) * D + pc * 8) * 2u;
      const uint4 cq = buf_load16(qr, off);
      const uint4 ck = buf_load16(kr, off);
      const uint4 cv = buf_load16(vr, off);
      float f[8];
      unpack8(cq, f);
#pragma unroll
      for (int i = 0; i < 8; ++i) ps[0][i] += f[i];
      unpack8(ck, f);
#pragma unroll
      for (int i = 0; i < 8; ++i) ps[1][i] += f[i];
      unpack8(cv, f);
#pragma unroll
      for (int i = 0; i < 8; ++i) ps[2][i] += f[i];
      lds_st(Ks, TL_::chunk_byte(t, pc), ck);
      lds_st(Vs, TL_::chunk_byte(t, pc), cv);
    }
    // Lanes holding the same chunk column differ in the bits >= log2(CH).
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float x = ps[a][i];
#pragma unroll
        for (int m = CH; m < 64; m <<= 1) x += __shfl_xor(x, m, 64);
        ps[a][i] = x;
      }
    if (lane < CH) {
#pragma unroll
      for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int i = 0; i < 8; ++i) red_sum[wave][a * D + lane * 8 + i] = ps[a][i];
    }
    __syncthreads();
    const float nf = (float)n;
    for (int idx = tid; idx < 3 * D; idx += 256) {
      float s = ((red_sum[0][idx] + red_sum[1][idx]) + red_sum[2][idx]) + red_sum[3][idx];
      const int a = idx / D;
      const int d = idx - a * D;
      if (a < 2) s = s / nf;
      colstat[idx] = s;
      float* dst = a == 0 ? qc : (a == 1 ? kc : vc);
      dst[((int64_t)bh * NT + j) * D + d] = s;
    }
    __syncthreads();

    // H_j quadrant = K^T V over the block's tokens (rows >= n are zero).
    f32x16_t acc[TL][TL];
#pragma unroll
    for (int a = 0; a < TL; ++a)
#pragma unroll
      for (int b = 0; b < TL; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

#pragma unroll
    for (int ks = 0; ks < BT / 16; ++ks) {
      bf16x8_t af[TL], bfr[TL];
#pragma unroll
      for (int mt = 0; mt < TL; ++mt) {
        const int d = dq + mt * 32 + l32;
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t0 = ks * 16 + h * 8 + 2 * i;
          const uint32_t lo = lds_ld<uint16_t>(Ks, TL_::elem_byte(t0, d));
          const uint32_t hi = lds_ld<uint16_t>(Ks, TL_::elem_byte(t0 + 1, d));
          w[i] = lo | (hi << 16);
        }
        af[mt] = __builtin_bit_cast(bf16x8_t, (u32x4_t){w[0], w[1], w[2], w[3]});
      }
#pragma unroll
      for (int nt = 0; nt < TL; ++nt) {
        const int e = eq + nt * 32 + l32;
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t0 = ks * 16 + h * 8 + 2 * i;
          const uint32_t lo = lds_ld<uint16_t>(Vs, TL_::elem_byte(t0, e));
          const uint32_t hi = lds_ld<uint16_t>(Vs, TL_::elem_byte(t0 + 1, e));
          w[i] = lo | (hi << 16);
        }
        bfr[nt] = __builtin_bit_cast(bf16x8_t, (u32x4_t){w[0], w[1], w[2], w[3]});
      }
#pragma unroll
      for (int mt = 0; mt < TL; ++mt)
#pragma unroll
        for (int nt = 0; nt < TL; ++nt) acc[mt][nt] = mfma32(af[mt], bfr[nt], acc[mt][nt]);
    }

    float nrm = 0.f;
#pragma unroll
    for (int mt = 0; mt < TL; ++mt)
#pragma unroll
      for (int nt = 0; nt < TL; ++nt) {
        const int e = eq + nt * 32 + l32;
        const float vsum = colstat[2 * D + e];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = dq + mt * 32 + mfma32_row(r, h);
          const float hv = acc[mt][nt][r] - colstat[D + d] * vsum;
          nrm += hv * hv;
          gacc[mt][nt][r] += hv;
        }
      }
    nrm = wave_sum(nrm);
    if (lane == 0) red_norm[wave] = nrm;
    __syncthreads();
    if (tid == 0) {
      const float s = ((red_norm[0] + red_norm[1]) + red_norm[2]) + red_norm[3];
      hnorm[(int64_t)bh * NT + j] = sqrtf(s);
    }
  }

  // Group mean: divide by G (the reference zero-pads the last group to G blocks).
  const int NG = (NT + G - 1) / G;
  float* hg = hgroup + ((int64_t)bh * NG + g) * D * D;
  const float Gf = (float)G;
#pragma unroll
  for (int mt = 0; mt < TL; ++mt)
#pragma unroll
    for (int nt = 0; nt < TL; ++nt) {
      const int e = eq + nt * 32 + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = dq + mt * 32 + mfma32_row(r, h);
        hg[d * D + e] = gacc[mt][nt][r] / Gf;
      }
    }
}

hipError_t launch_block_stats(const void* q, const void* k, const void* v, float* qc, float* kc,
                              float* vc, float* hnorm, float* hgroup, int bh, int T, int Tslice, int D,
                              int BT, int G, hipStream_t stream) {
  const int NT = (T + BT - 1) / BT;
  const int NG = (NT + G - 1) / G;
  dim3 grid(NG, bh);
  auto a = (const uint16_t*)q;
  auto b = (const uint16_t*)k;
  auto c = (const uint16_t*)v;
  if (D == 128 && BT == 128)
    hipLaunchKernelGGL((k2_block_stats<128, 128>), grid, dim3(256), 0, stream, a, b, c, qc, kc, vc,
                       hnorm, hgroup, T, Tslice, NT, G);
  else if (D == 128 && BT == 64)
    hipLaunchKernelGGL((k2_block_stats<128, 64>), grid, dim3(256), 0, stream, a, b, c, qc, kc, vc,
                       hnorm, hgroup, T, Tslice, NT, G);
  else if (D == 64 && BT == 128)
    hipLaunchKernelGGL((k2_block_stats<64, 128>), grid, dim3(256), 0, stream, a, b, c, qc, kc, vc,
                       hnorm, hgroup, T, Tslice, NT, G);
  else if (D == 64 && BT == 64)
    hipLaunchKernelGGL((k2_block_stats<64, 64>), grid, dim3(256), 0, stream, a, b, c, qc, kc, vc,
                       hnorm, hgroup, T, Tslice, NT, G);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace pasa
