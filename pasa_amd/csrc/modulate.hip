// DiT block row operations (K6): gated residual, LayerNorm and shift/scale modulation
// of token rows, fused into one pass per row.
//
// The Wan block around the PASA processors (svg/models/wan/custom_models.py:23-115)
// runs, per token row of width N:
//   stage A (optional):  h = r + x * gate      (gated residual, gate fp32 [N] per batch)
//                        h = r + x             (plain residual, gate absent)
//   stage B (optional), on h (or on x without stage A):
//                        v = (v - mean) * rstd,  mean = sum(v)/N,
//                            rstd = 1/sqrt(sum((v-mean)^2)/N + eps)        (LayerNorm)
//                        v = v * w + b                                     (affine)
//                        v = v * (1 + scale) + shift                       (modulation)
// Each product and sum is rounded in fp32 as the reference's PyTorch fallback rounds
// it (one operation per step), and h is rounded to its storage type before stage B
// reads it, as the reference stores h between the two steps.  The reference runs these
// as separate passes with an fp32 tensor between LayerNorm and modulation
// (svg/kernels/triton/layernorm.py:9-63, :110-161 and modulate.py:12-122); fused, a row
// is read once and its results written once.
//
// Work split: one wave per row, four rows per workgroup; lane l owns the 8-element
// chunks l, l+64, l+128, ... of the row.  Every chunk is read before any is written and
// is written by the lane that read it, so h may alias r (in-place residual update).
#include <math.h>

#include "common.h"
#include "kernels.h"

namespace pasa {

namespace {

constexpr int kRowsPerWg = 4;

__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float(f32_to_bf16_bits(x) << 16); }

// 8 consecutive elements of a bf16 or fp32 row into fp32.
__device__ __forceinline__ void load8(const void* base, int64_t elem, bool f32, float (&f)[8]) {
  if (f32) {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + elem);
    const float4 a = p[0], b = p[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
    unpack8(*reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + elem), f);
  }
}

// 16-byte row chunks, streamed (nontemporal: not kept in L2 or the last-level cache) when
// NT, for rows of tensors too large for those caches to help their next reader.
template <bool NT>
__device__ __forceinline__ uint4 ld16(const void* ptr) {
  if constexpr (NT) {
    const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(ptr));
    return uint4{t[0], t[1], t[2], t[3]};
  } else {
    return *reinterpret_cast<const uint4*>(ptr);
  }
}
template <bool NT>
__device__ __forceinline__ void st16(void* ptr, const uint4& v) {
  if constexpr (NT)
    __builtin_nontemporal_store((u32x4_t){v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t*>(ptr));
  else
    *reinterpret_cast<uint4*>(ptr) = v;
}

template <bool NT = false>
__device__ __forceinline__ void store8(void* base, int64_t elem, bool f32, const float (&f)[8]) {
  if (f32) {
    float4* p = reinterpret_cast<float4*>(reinterpret_cast<float*>(base) + elem);
    p[0] = make_float4(f[0], f[1], f[2], f[3]);
    p[1] = make_float4(f[4], f[5], f[6], f[7]);
  } else {
    uint4 o;
    o.x = pack_bf16x2(f[0], f[1]);
    o.y = pack_bf16x2(f[2], f[3]);
    o.z = pack_bf16x2(f[4], f[5]);
    o.w = pack_bf16x2(f[6], f[7]);
    st16<NT>(reinterpret_cast<uint16_t*>(base) + elem, o);
  }
}

// Stage B's input row, CPT chunks of 8 per lane: packed bf16 when it is a bf16 value
// (x in bf16 without stage A, or h stored as bf16), else fp32.  Every pass rebuilds
// the fp32 values from it exactly, so the packed form changes no result and holds a
// row in half the registers.
template <int CPT, bool PACKED>
struct RowStore;
template <int CPT>
struct RowStore<CPT, true> {
  uint4 c[CPT];
  __device__ __forceinline__ void get(int i, float (&f)[8]) const { unpack8(c[i], f); }
  __device__ __forceinline__ void set(int i, const float (&f)[8]) {
    c[i] = make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                      pack_bf16x2(f[6], f[7]));
  }
  __device__ __forceinline__ void zero(int i) { c[i] = make_uint4(0u, 0u, 0u, 0u); }
};
template <int CPT>
struct RowStore<CPT, false> {
  float v[CPT][8];
  __device__ __forceinline__ void get(int i, float (&f)[8]) const {
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = v[i][e];
  }
  __device__ __forceinline__ void set(int i, const float (&f)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[i][e] = f[e];
  }
  __device__ __forceinline__ void zero(int i) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[i][e] = 0.f;
  }
};

// NT (packed rows only): the row tensors x, the residual, h and y are streamed.
template <int CPT, bool PACKED, bool NT>
__global__ __launch_bounds__(256) void k6_row_ops(RowOpParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWg + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= p.M) return;  // uniform over the wave
  const int N = p.N;
  const int nc = N >> 3;
  const int nmine = (nc - lane + 63) >> 6;  // chunks this lane owns (<= CPT)
  const int64_t base = row * (int64_t)N;
  const int64_t pb = (row / p.rows_per_batch) * p.param_stride;  // batch offset of gate/scale/shift

  RowStore<CPT, PACKED> st;
  if (p.r == nullptr) {
    // stage B reads x itself
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      if (i >= nmine) {
        st.zero(i);
      } else if constexpr (PACKED) {
        reinterpret_cast<uint4*>(&st)[i] =
            ld16<NT>(reinterpret_cast<const uint16_t*>(p.x) + base + 8 * (lane + 64 * i));
      } else {
        float f[8];
        load8(p.x, base + 8 * (lane + 64 * i), p.x_f32, f);
        st.set(i, f);
      }
    }
  } else if constexpr (PACKED) {
    // ---- stage A, all bf16: raw 16-byte chunks in registers, all loads issued first -----
    uint4 xr[CPT], rr[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      if (i >= nmine) continue;
      const int c0 = 8 * (lane + 64 * i);
      xr[i] = ld16<NT>(reinterpret_cast<const uint16_t*>(p.x) + base + c0);
      rr[i] = ld16<NT>(reinterpret_cast<const uint16_t*>(p.r) + base + c0);
    }
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      if (i >= nmine) {
        st.zero(i);
        continue;
      }
      const int c0 = 8 * (lane + 64 * i);
      float xs[8], rs[8], h[8];
      unpack8(xr[i], xs);
      unpack8(rr[i], rs);
      if (p.gate != nullptr) {
        float g[8];
        load8(p.gate, pb + c0, true, g);
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = add_rn(rs[e], mul_rn(xs[e], g[e]));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = add_rn(rs[e], xs[e]);
      }
      st.set(i, h);  // h rounded to bf16, its storage type
      if (p.h != nullptr)
        st16<NT>(reinterpret_cast<uint16_t*>(p.h) + base + c0, reinterpret_cast<uint4*>(&st)[i]);
    }
  } else {
    // ---- stage A, other types ---------------------------------------------------------
    float xs[CPT][8], rs[CPT][8];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      if (i >= nmine) continue;
      const int c0 = 8 * (lane + 64 * i);
      load8(p.x, base + c0, p.x_f32, xs[i]);
      load8(p.r, base + c0, p.r_f32, rs[i]);
    }
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      if (i >= nmine) {
        st.zero(i);
        continue;
      }
      const int c0 = 8 * (lane + 64 * i);
      float h[8];
      if (p.gate != nullptr) {
        float g[8];
        load8(p.gate, pb + c0, true, g);
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = add_rn(rs[i][e], mul_rn(xs[i][e], g[e]));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = add_rn(rs[i][e], xs[i][e]);
      }
      if (!p.h_f32) {
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = bf16_round(h[e]);
      }
      st.set(i, h);
      if (p.h != nullptr) store8(p.h, base + c0, p.h_f32, h);
    }
  }
  if (p.y == nullptr) return;

  // ---- stage B: LayerNorm, affine, modulation -----------------------------------------
  float mean = 0.f, rstd = 1.f;
  if (p.ln) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      float f[8];
      st.get(i, f);  // padding chunks hold 0
#pragma unroll
      for (int e = 0; e < 8; ++e) a = add_rn(a, f[e]);
    }
    mean = div_rn(wave_sum_xor(a), (float)N);
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      if (i >= nmine) continue;
      float f[8];
      st.get(i, f);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = sub_rn(f[e], mean);
        q = add_rn(q, mul_rn(d, d));
      }
    }
    const float var = div_rn(wave_sum_xor(q), (float)N);
    rstd = div_rn(1.0f, sqrt_rn(add_rn(var, p.eps)));
  }
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    if (i >= nmine) continue;
    const int c0 = 8 * (lane + 64 * i);
    float v[8];
    st.get(i, v);
    if (p.ln) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = mul_rn(sub_rn(v[e], mean), rstd);
    }
    if (p.w != nullptr) {
      float w[8];
      load8(p.w, c0, p.wb_f32, w);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = mul_rn(v[e], w[e]);
    }
    if (p.b != nullptr) {
      float b[8];
      load8(p.b, c0, p.wb_f32, b);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = add_rn(v[e], b[e]);
    }
    if (p.scale != nullptr) {
      float sc[8], sh[8];
      load8(p.scale, pb + c0, true, sc);
      load8(p.shift, pb + c0, true, sh);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = add_rn(mul_rn(v[e], add_rn(1.0f, sc[e])), sh[e]);
    }
    store8<NT>(p.y, base + c0, p.y_f32, v);
  }
}

}  // namespace

constexpr int kRowOpsMaxCpt = 16;  // N <= 8192
constexpr int64_t kStreamBytes = int64_t(256) << 20;  // MI355X last-level (Infinity) cache
int row_ops_max_cols() { return kRowOpsMaxCpt * 64 * 8; }

hipError_t launch_row_ops(const RowOpParams& p, hipStream_t stream) {
  if (p.M <= 0 || p.N <= 0 || p.N % 8 != 0 || p.N > row_ops_max_cols() || p.rows_per_batch <= 0)
    return hipErrorInvalidValue;
  const int cpt = (p.N / 8 + 63) / 64;
  const int64_t nwg = (p.M + kRowsPerWg - 1) / kRowsPerWg;
  if (nwg > 0x7fffffff) return hipErrorInvalidValue;
  dim3 grid((unsigned)nwg);
  // Packed: stage B's input is bf16 and, with stage A, x and the residual are bf16 too
  // (every call of the Wan block).  Other type mixes keep the row in fp32 registers.
  const bool packed = p.r != nullptr ? (!p.h_f32 && !p.x_f32 && !p.r_f32) : !p.x_f32;
  // Rows of a tensor larger than the 256 MB last-level cache are streamed: its next reader
  // cannot find them there anyway, and nontemporal accesses move them 15% faster (75,600 x
  // 5120 bf16: 0.58 against 0.68 ms).  Smaller tensors stay cached for their reader.
  const bool stream_rows = packed && (int64_t)p.M * p.N * 2 >= kStreamBytes;
#define PASA_K6(C)                                                                              \
  do {                                                                                          \
    if (stream_rows) hipLaunchKernelGGL((k6_row_ops<C, true, true>), grid, dim3(256), 0, stream, p); \
    else if (packed) hipLaunchKernelGGL((k6_row_ops<C, true, false>), grid, dim3(256), 0, stream, p); \
    else hipLaunchKernelGGL((k6_row_ops<C, false, false>), grid, dim3(256), 0, stream, p);     \
  } while (0)
  if (cpt <= 1) PASA_K6(1);
  else if (cpt <= 2) PASA_K6(2);
  else if (cpt <= 3) PASA_K6(3);
  else if (cpt <= 4) PASA_K6(4);
  else if (cpt <= 6) PASA_K6(6);
  else if (cpt <= 8) PASA_K6(8);
  else if (cpt <= 10) PASA_K6(10);
  else if (cpt <= 12) PASA_K6(12);
  else PASA_K6(16);
#undef PASA_K6
  return hipGetLastError();
}

}  // namespace pasa
