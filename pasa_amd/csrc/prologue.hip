// Attention-processor prologue (K5): RMSNorm and rotary embedding of Q and K,
// fused with the move to the head-major [B, H, S, D] layout PISA-PG reads.
//
// The processors around the PISA-PG path normalise Q and K (RMSNorm over the
// whole hidden row for Wan, per head for HunyuanVideo), split heads, and rotate
// channel pairs (x[2i], x[2i+1]).  Each step is a separate HBM pass in the
// reference; here one pass reads each projection row once and writes the final
// bf16 row once.  The intermediate bf16 roundings of the unfused pipeline are
// reproduced in registers, so the result equals the step-by-step computation:
//  * norm (once):  y = bf16((x * rstd) * w),        rstd = 1 / sqrt(sum(x^2)/N + eps)
//                  (svg/kernels/triton/rmsnorm.py:29-44)
//  * norm (twice): y = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)
//                  (diffusers RMSNorm with a bf16 weight, the fallback at
//                  svg/models/hyvideo/attention.py:198-205)
//  * rope, fp32 cos/sin [rows, D]:  o0 = x0*c0 + (-x1)*s0, o1 = x1*c1 + x0*s1,
//                  each product and sum rounded in fp32, then bf16
//                  (diffusers apply_rotary_emb use_real, hyvideo/attention.py:211-230)
//  * rope, fp64 complex [rows, D/2]: (x0 + i x1)(re + i im) in fp64, then
//                  fp64 -> fp32 -> bf16 as torch's cast does
//                  (svg/models/wan/attention.py:49-57)
// Rows at or past rope_rows (trailing text tokens) are normalised but not rotated.
//
// Work split: a workgroup owns 4 tokens of one tensor, one wave per token; lane
// l handles the 16-byte chunks l, l+64, l+128, ... of the token's H*D row, so
// every chunk of a lane has the same position c inside its head and the lane
// loads its rotary coefficients once.  All of a lane's chunks are read before
// any is written, and each chunk is written by the lane that read it, so the
// operation may run in place when input and output share one layout.
#include <math.h>

#include "common.h"
#include "kernels.h"

namespace pasa {

namespace {

constexpr int kTokPerWg = 4;
constexpr int kLanesPerTok = 64;

__device__ __forceinline__ float bf16r(float x) { return __uint_as_float(f32_to_bf16_bits(x) << 16); }

// Workgroup n runs on XCD n % 8.  The three tensors of one token tile take slots
// 3g, 3g+1, 3g+2 of the same XCD, so K's workgroup finds the rotary table Q's
// workgroup just read in that XCD's L2.
template <int CPT>
__global__ __launch_bounds__(256) void k5_prologue(PrologueParams p, int64_t tiles) {
  const int64_t n = blockIdx.x;
  const int64_t slot = n >> 3;
  const int t = (int)(slot % 3);
  const int64_t tile = (slot / 3) * 8 + (n & 7);
  const PrologueTensor T = p.t[t];
  if (T.in == nullptr || tile >= tiles) return;  // uniform over the workgroup

  const int tid = threadIdx.x;
  const int l = tid & (kLanesPerTok - 1);
  const int64_t s = tile * kTokPerWg + __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t b = blockIdx.y;
  const bool tok_ok = s < p.S;  // uniform over the wave
  const int D = p.D;
  const int DC = D >> 3;            // chunks per head (8 or 16); divides 64
  const int NC = (int)p.H * DC;     // chunks per token row
  const int c = l & (DC - 1);       // this lane's chunk position inside every head
  const int h0 = l / DC;            // head of chunk i is h0 + i * (64 / DC)
  const int64_t hstep = kLanesPerTok / DC;
  // Element offsets of chunk 0 and the step between successive chunks of the lane.
  const uint16_t* in0 = T.in + (p.in_bshd ? ((b * p.S + s) * p.H + h0) * D : ((b * p.H + h0) * p.S + s) * D) + 8 * c;
  const int64_t in_step = p.in_bshd ? hstep * D : hstep * p.S * D;
  const int64_t row = p.row0 + s;
  uint16_t* out0 = T.out + (p.out_bshd ? ((b * p.OS + row) * p.H + h0) * D : ((b * p.H + h0) * p.OS + row) * D) + 8 * c;
  const int64_t out_step = p.out_bshd ? hstep * D : hstep * p.OS * D;
  const int nmine = tok_ok ? (NC - l + kLanesPerTok - 1) / kLanesPerTok : 0;  // chunks this lane owns

  // ---- load the lane's chunks --------------------------------------------------
  uint4 raw[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    raw[i] = uint4{0u, 0u, 0u, 0u};
    if (i < nmine) raw[i] = *reinterpret_cast<const uint4*>(in0 + i * in_step);
  }

  // ---- RMSNorm ------------------------------------------------------------------
  const int norm = T.weight != nullptr ? p.norm : 0;
  float rstd[CPT];
  if (norm != 0) {
    float ss[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      float f[8];
      unpack8(raw[i], f);
      float a = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) a = add_rn(a, mul_rn(f[e], f[e]));  // squares rounded, as x*x is
      ss[i] = a;
    }
    if (norm == kNormRow) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < CPT; ++i) a += ss[i];
#pragma unroll
      for (int m = 1; m < kLanesPerTok; m <<= 1) a += __shfl_xor(a, m, kLanesPerTok);
      const float var = div_rn(a, (float)(p.H * D));
      const float r = p.round_twice ? rsqrtf(var + p.eps) : div_rn(1.0f, sqrt_rn(add_rn(var, p.eps)));
#pragma unroll
      for (int i = 0; i < CPT; ++i) rstd[i] = r;
    } else {  // per head: the head's DC chunks sit on DC consecutive lanes
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        float a = ss[i];
        for (int m = 1; m < DC; m <<= 1) a += __shfl_xor(a, m, kLanesPerTok);
        const float var = div_rn(a, (float)D);
        rstd[i] = p.round_twice ? rsqrtf(var + p.eps) : div_rn(1.0f, sqrt_rn(add_rn(var, p.eps)));
      }
    }
  }

  // ---- rotary coefficients for this lane's 4 channel pairs -----------------------
  const int rope = (t < 2 && tok_ok && s < p.rope_rows) ? p.rope : 0;
  float cr[8], sr[8];  // fp32 form: cos/sin of the chunk's 8 channels
  double cre[4], cim[4];  // complex form: the chunk's 4 pair coefficients
  if (rope == kRopeCosSinF32) {
    const float* cp = reinterpret_cast<const float*>(p.cos) + s * D + 8 * c;
    const float* sp = reinterpret_cast<const float*>(p.sin) + s * D + 8 * c;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      cr[e] = cp[e];
      sr[e] = sp[e];
    }
  } else if (rope == kRopeComplexF64) {
    const double* rp = reinterpret_cast<const double*>(p.cos) + s * (D / 2) + 4 * c;
    const double* ip = reinterpret_cast<const double*>(p.sin) + s * (D / 2) + 4 * c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      cre[e] = rp[e];
      cim[e] = ip[e];
    }
  }

  // ---- normalise, rotate, store ---------------------------------------------------
  float w[8];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    if (i >= nmine) continue;
    float f[8];
    unpack8(raw[i], f);
    if (norm != 0) {
      const int64_t woff = norm == kNormRow ? (h0 + i * hstep) * D + 8 * c : 8 * c;
      unpack8(*reinterpret_cast<const uint4*>(T.weight + woff), w);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        f[e] = p.round_twice ? bf16r(bf16r(f[e] * rstd[i]) * w[e]) : bf16r(mul_rn(mul_rn(f[e], rstd[i]), w[e]));
    }
    if (rope == kRopeCosSinF32) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = f[2 * e], x1 = f[2 * e + 1];
        f[2 * e] = add_rn(mul_rn(x0, cr[2 * e]), mul_rn(-x1, sr[2 * e]));
        f[2 * e + 1] = add_rn(mul_rn(x1, cr[2 * e + 1]), mul_rn(x0, sr[2 * e + 1]));
      }
    } else if (rope == kRopeComplexF64) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const double x0 = f[2 * e], x1 = f[2 * e + 1];
        f[2 * e] = (float)(x0 * cre[e] - x1 * cim[e]);
        f[2 * e + 1] = (float)(x0 * cim[e] + x1 * cre[e]);
      }
    }
    uint4 o;
    o.x = pack_bf16x2(f[0], f[1]);
    o.y = pack_bf16x2(f[2], f[3]);
    o.z = pack_bf16x2(f[4], f[5]);
    o.w = pack_bf16x2(f[6], f[7]);
    *reinterpret_cast<uint4*>(out0 + i * out_step) = o;
  }
}

}  // namespace

constexpr int kMaxCpt = 16;  // H*D <= 8192
int prologue_max_chunks() { return kMaxCpt * kLanesPerTok; }

hipError_t launch_prologue(const PrologueParams& p, hipStream_t stream) {
  if ((p.D != 64 && p.D != 128) || p.H <= 0 || p.S <= 0 || p.B <= 0) return hipErrorInvalidValue;
  const int64_t nc = p.H * (int64_t)(p.D / 8);
  const int64_t cpt = (nc + kLanesPerTok - 1) / kLanesPerTok;
  if (cpt > kMaxCpt) return hipErrorInvalidValue;
  const int64_t tiles = (p.S + kTokPerWg - 1) / kTokPerWg;
  const int64_t nwg = (tiles + 7) / 8 * 8 * 3;
  if (nwg > 0x7fffffff || p.B > 65535) return hipErrorInvalidValue;
  dim3 grid((unsigned)nwg, (unsigned)p.B, 1);
#define PASA_K5(N) hipLaunchKernelGGL(k5_prologue<N>, grid, dim3(256), 0, stream, p, tiles)
  if (cpt <= 2) PASA_K5(2);
  else if (cpt <= 4) PASA_K5(4);
  else if (cpt <= 6) PASA_K5(6);
  else if (cpt <= 8) PASA_K5(8);
  else if (cpt <= 10) PASA_K5(10);
  else if (cpt <= 12) PASA_K5(12);
  else PASA_K5(16);
#undef PASA_K5
  return hipGetLastError();
}

}  // namespace pasa
