// The PISA-PG path for shapes the tuned kernels do not take: fp32 q, k, v; any head
// dim up to 128; any group size; block sizes 16 .. 256.  Same mathematics, plain VALU
// arithmetic, one WG per (slice, group) or per (slice, 64-row query tile).
//
// Reference: svg/kernels/triton/group_pisa_attention.py
//   k2_block_stats_any   fused_chunk_reduce_kernel :66-129 (+ sqrt :287) and
//                        compute_h_group :291-301
//   k3_scores_any        the selection scores :365-371
//   k4_sparse_attn_any   pisa_pg_fwd_kernel :135-262
// The reference accepts any float dtype (o = torch.empty_like(v), :380; statistics
// stored like q, :275-278), any group size (:312) and any power-of-two block size
// (:311; Triton's tl.arange needs a power of two).  These kernels round where the
// reference rounds for 16-bit inputs (kc, vc and Hbar in the input type at their use,
// P and P-bar cast to it before their products, the output store) and not at all for
// fp32 inputs, so an fp32 call is the reference's mathematics in fp32.
//
// Layout of a query tile: 64 rows, eight lanes per pair of rows (rows r and r + 32; lane & 7
// owns features 16 (lane & 7) .. + 15 of both); a row's dot products are reduced over its
// eight lanes by DPP, which gives all eight lanes the same bits.
#include "common.h"
#include "kernels.h"

namespace pasa {

namespace {

// Element access for the three input types.  round(x): x rounded to the type and back.
struct F32E {
  __device__ static float load(const void* p, int64_t i) { return ((const float*)p)[i]; }
  __device__ static float round(float x) { return x; }
  __device__ static void store(void* p, int64_t i, float x) { ((float*)p)[i] = x; }
};
struct Bf16E {
  __device__ static float load(const void* p, int64_t i) {
    return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  }
  __device__ static float round(float x) { return bf16_bits_to_f32(f32_to_bf16_bits(x)); }
  __device__ static void store(void* p, int64_t i, float x) { ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16_bits(x); }
};
struct F16E {
  __device__ static float load(const void* p, int64_t i) { return (float)((const _Float16*)p)[i]; }
  __device__ static float round(float x) { return (float)(_Float16)x; }
  __device__ static void store(void* p, int64_t i, float x) { ((_Float16*)p)[i] = (_Float16)x; }
};

constexpr int kAnyChunk = 32;   // rows of a staged K/V chunk
constexpr int kAnyLd = 132;     // LDS row stride (floats) of staged rows: 16-byte aligned, so
                                // row pieces are ds_read_b128
constexpr int kAnyTile = 64;    // query rows per attention workgroup

// Sum of x over the eight lanes 8r .. 8r + 7: ((x0 + x1) + (x2 + x3)) + ((x4 + x5) + (x6 + x7)) on
// all eight (addition commutes, so every lane gets the same bits), by DPP: two quad
// permutations (lane ^ 1, lane ^ 2), then the half-row mirror (lane 7 - i of the eight).
__device__ __forceinline__ float oct_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false));   // lane ^ 1
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false));   // lane ^ 2
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, false));  // 7 - i
  return x;
}

}  // namespace

// ---- block statistics ---------------------------------------------------------
// One workgroup (256 threads) per (group of G key blocks, slice); the group's blocks in
// ascending order, each in 32-row chunks of k and v staged in LDS as fp32 (132-float rows,
// feature columns D .. 127 zero).  Thread t owns an 8 x 8 tile of the D x D moment, rows
// d = 8 (t >> 4) .. + 7 and columns e = 8 (t & 15) .. + 7: per staged row, four 16-byte
// reads feed 64 FMAs.  H_j[d][e] = sum_t k_t[d] v_t[e] - kbar_j[d] V^_j[e] (:106-107), the
// sum over the block's rows in order; entries past D stay zero and are not stored.  Threads
// t < D own column t of the block sums of q, k and v.  The group sum adds H_j in block order,
// then / G.
template <typename EL>
__global__ __launch_bounds__(256) void k2_block_stats_any(const void* __restrict__ q, const void* __restrict__ k,
                                                          const void* __restrict__ v, float* __restrict__ qc,
                                                          float* __restrict__ kc, float* __restrict__ vc,
                                                          float* __restrict__ hnorm, float* __restrict__ hgroup,
                                                          int T, int Tslice, int D, int BT, int NT, int G) {
  constexpr int CH = kAnyChunk, LD = kAnyLd;
  __shared__ __attribute__((aligned(16))) float ks[CH * LD];
  __shared__ __attribute__((aligned(16))) float vs[CH * LD];
  __shared__ float qsm[CH * 128];  // the chunk's q rows (only their column sums are needed)
  __shared__ float kbar[128];
  __shared__ float vhat[128];
  __shared__ float red[4];
  const int g = blockIdx.x;
  const int bh = blockIdx.y;
  const int tid = threadIdx.x;
  const int NG = (NT + G - 1) / G;
  const int64_t base = (int64_t)bh * Tslice * D;
  const int d0 = 8 * (tid >> 4);
  const int e0 = 8 * (tid & 15);
  const bool owns = d0 < D && e0 < D;  // the tile holds at least one entry of the moment
  for (int i = tid; i < CH * LD; i += 256) {
    ks[i] = 0.f;
    vs[i] = 0.f;
  }
  if (tid < 128) {
    kbar[tid] = 0.f;
    vhat[tid] = 0.f;
  }
  float gacc[64];
#pragma unroll
  for (int m = 0; m < 64; ++m) gacc[m] = 0.f;
  const int j1 = min(NT, (g + 1) * G);
  for (int j = g * G; j < j1; ++j) {
    const int r0 = j * BT;
    const int n = min(BT, T - r0);
    float hacc[64];
#pragma unroll
    for (int m = 0; m < 64; ++m) hacc[m] = 0.f;
    float qs = 0.f, ksum = 0.f, vsum = 0.f;
    for (int c0 = 0; c0 < n; c0 += CH) {
      const int cn = min(CH, n - c0);
      __syncthreads();  // the previous chunk's reads are done (and the zero fill landed)
      for (int i = tid; i < cn * D; i += 256) {
        const int t = i / D;
        const int d = i - t * D;
        const int64_t off = base + (int64_t)(r0 + c0 + t) * D + d;
        ks[t * LD + d] = EL::load(k, off);
        vs[t * LD + d] = EL::load(v, off);
        qsm[t * 128 + d] = EL::load(q, off);
      }
      __syncthreads();
      if (tid < D) {
        for (int t = 0; t < cn; ++t) {
          ksum += ks[t * LD + tid];
          vsum += vs[t * LD + tid];
          qs += qsm[t * 128 + tid];
        }
      }
      if (owns) {
        for (int t = 0; t < cn; ++t) {
          const float4 k0 = *reinterpret_cast<const float4*>(ks + t * LD + d0);
          const float4 k1 = *reinterpret_cast<const float4*>(ks + t * LD + d0 + 4);
          const float4 v0 = *reinterpret_cast<const float4*>(vs + t * LD + e0);
          const float4 v1 = *reinterpret_cast<const float4*>(vs + t * LD + e0 + 4);
          const float kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
          const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
          for (int a = 0; a < 8; ++a)
#pragma unroll
            for (int b = 0; b < 8; ++b) hacc[8 * a + b] = fmaf(kk[a], vv[b], hacc[8 * a + b]);
        }
      }
    }
    __syncthreads();
    if (tid < D) {
      const float kb = ksum / (float)n;
      kbar[tid] = kb;
      vhat[tid] = vsum;
      const int64_t so = ((int64_t)bh * NT + j) * D + tid;
      qc[so] = qs / (float)n;  // :101
      kc[so] = kb;             // :102
      vc[so] = vsum;           // :103 (a sum, not a mean)
    }
    __syncthreads();
    float nsq = 0.f;
    if (owns) {
#pragma unroll
      for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const float h = hacc[8 * a + b] - kbar[d0 + a] * vhat[e0 + b];  // :107 (zero past D)
          nsq = fmaf(h, h, nsq);
          gacc[8 * a + b] += h;
        }
    }
    nsq = wave_sum(nsq);
    if ((tid & 63) == 0) red[tid >> 6] = nsq;
    __syncthreads();
    if (tid == 0) hnorm[(int64_t)bh * NT + j] = sqrt_rn((red[0] + red[1]) + (red[2] + red[3]));  // :110, :287
  }
  // hbar_g = (1/G) sum over the group, the missing blocks of the last group counting as zeros (:294-299).
  if (owns) {
    float* hg = hgroup + ((int64_t)bh * NG + g) * D * D;
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
      for (int b = 0; b < 8; ++b)
        if (d0 + a < D && e0 + b < D) hg[(d0 + a) * D + e0 + b] = gacc[8 * a + b] / (float)G;
  }
}

// ---- selection scores -----------------------------------------------------------
// score[I][j] = sum_d qc[I][d] * fl(scale * kc[j][d]) + log(hnorm[j] + 1e-6) [+ noise[j]],
// one thread per score, features in ascending order; one row per grid x index.
__global__ __launch_bounds__(256) void k3_scores_any(const float* __restrict__ qc, const float* __restrict__ kc,
                                                     const float* __restrict__ hnorm, const float* __restrict__ noise,
                                                     float scale, int use_cov_bias, float* __restrict__ scores, int NT,
                                                     int D) {
  const int j = blockIdx.y * 256 + threadIdx.x;
  const int I = blockIdx.x;  // the row on grid x: NT may exceed grid y's 65,535
  const int bh = blockIdx.z;
  if (j >= NT) return;
  const float* qi = qc + ((int64_t)bh * NT + I) * D;
  const float* kj = kc + ((int64_t)bh * NT + j) * D;
  float acc = 0.f;
  for (int d = 0; d < D; ++d) acc = fmaf(qi[d], mul_rn(scale, kj[d]), acc);
  float bias = 0.f;
  if (use_cov_bias) {
    bias = logf(hnorm[(int64_t)bh * NT + j] + 1e-6f);
    if (noise) bias = bias + noise[(int64_t)bh * NT + j];
  }
  scores[((int64_t)bh * NT + I) * NT + j] = acc + bias;
}

// ---- attention -----------------------------------------------------------------
// One workgroup per 64-row query tile of a slice.  Video tiles (a block of BT rows is
// ceil(BT / 64) tiles) visit the selected key blocks in ascending order (every block
// when `all`), then the prompt keys [T, T + text_valid); then phase 2 over the groups
// (not when `all`).  Text tiles attend densely within their segment ([0, seg) for the
// prompt rows, [seg, T + text) for the padding rows).  Keys go in chunks of 32 staged in
// LDS, each chunk one online-softmax step (exact: rescaled whenever a row's max rises).
// Lane mapping: eight lanes per pair of rows (rows rp and rp + 32, rp = tid / 8), lane
// tid & 7 owning features 16 (tid & 7) .. + 15 of both; a 16-byte LDS read of a key row
// feeds eight FMAs.  Feature columns D .. 127 of every LDS row hold zeros (written once,
// never overwritten), as do a lane's q features past D, so the dot products run over all
// 16 features of a lane with no per-feature test: the extra terms are 0 * 0.
template <typename EL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k4_sparse_attn_any(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v,
    const float* __restrict__ kc, const float* __restrict__ vc, const float* __restrict__ hgroup,
    const uint32_t* __restrict__ selmask, void* __restrict__ o, float scale, float c, int T, int text,
    int text_valid, int D, int BT, int NT, int G, int NG, int NW, int gamma_literal, int all) {
  constexpr int CH = kAnyChunk, LD = kAnyLd, TR = kAnyTile;
  static_assert(2 * CH * LD >= TR * LD, "an Hbar slab of 64 rows fits the K/V chunk buffers");
  static_assert(LD % 4 == 0 && TR == 64, "16-byte LDS rows; two rows per lane, 32 apart");
  __shared__ __attribute__((aligned(16))) float kv[2 * CH * LD];  // K chunk, V chunk; phase 2: 64 rows of Hbar
  __shared__ __attribute__((aligned(16))) float qsh[TR * LD];     // the tile's q rows
  float* ks = kv;
  float* vs = kv + CH * LD;
  const int tid = threadIdx.x;
  const int rp = tid >> 3;        // rows rp and rp + 32 of the tile
  const int f0 = 16 * (tid & 7);  // this lane's first feature
  const int bh = blockIdx.y;
  const int Ttot = T + text;
  const int seg = T + text_valid;
  const int tpb = (BT + TR - 1) / TR;
  const int nvt = NT * tpb;
  int tile = blockIdx.x;
  int row0, rows, I = -1, kbeg = 0, kend = 0;
  if (tile < nvt) {
    I = tile / tpb;
    const int sub = tile - I * tpb;
    row0 = I * BT + sub * TR;
    rows = min(TR, min(BT - sub * TR, T - row0));
  } else {
    tile -= nvt;
    const int ptiles = (text_valid + TR - 1) / TR;
    if (tile < ptiles) {
      row0 = T + tile * TR;
      rows = min(TR, seg - row0);
      kbeg = 0;
      kend = seg;
    } else {
      row0 = seg + (tile - ptiles) * TR;
      rows = min(TR, Ttot - row0);
      kbeg = seg;
      kend = Ttot;
    }
  }
  if (rows <= 0) return;  // a video tile past the last block's rows
  const int64_t sbase = (int64_t)bh * Ttot * D;
  // The tile's q rows, zeros past D and past its last row; the K/V buffers start as zeros.
  for (int i = tid; i < TR * 128; i += 256) {
    const int rr = i >> 7;
    const int d = i & 127;
    qsh[rr * LD + d] = (rr < rows && d < D) ? EL::load(q, sbase + (int64_t)(row0 + rr) * D + d) : 0.f;
  }
  for (int i = tid; i < 2 * CH * LD; i += 256) kv[i] = 0.f;
  __syncthreads();
  float qp[2][16], op[2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int d4 = 0; d4 < 4; ++d4) {
      const float4 qq = *reinterpret_cast<const float4*>(qsh + (rp + 32 * i) * LD + f0 + 4 * d4);
      qp[i][4 * d4] = qq.x;
      qp[i][4 * d4 + 1] = qq.y;
      qp[i][4 * d4 + 2] = qq.z;
      qp[i][4 * d4 + 3] = qq.w;
    }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int dd = 0; dd < 16; ++dd) op[i][dd] = 0.f;
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f}, gam[2] = {0.f, 0.f};

  // Rows 0 .. 31 of ks / vs against this lane's features.  Each loop reads one LDS row ahead
  // (its four 16-byte reads in flight while the current row's 32 FMAs run) and keeps the
  // scheduler from hoisting further (register pressure).  Rows past the staged ones hold
  // earlier rows or zeros: their scores are computed and replaced by -inf, and P.V skips them.
  float x[2][CH];
  // x[i][t] = c q_i . ks[t] where keep(t), else -inf; mx[i] = the max over t.
  auto scores = [&](auto keep, float (&mx)[2]) __attribute__((always_inline)) {
    mx[0] = mx[1] = -INFINITY;
    float4 rb[4], rn[4];
    const float* kr = ks + f0;
#pragma unroll
    for (int d4 = 0; d4 < 4; ++d4) rb[d4] = *reinterpret_cast<const float4*>(kr + 4 * d4);
#pragma unroll
    for (int t = 0; t < CH; ++t) {
      if (t + 1 < CH) {
#pragma unroll
        for (int d4 = 0; d4 < 4; ++d4) rn[d4] = *reinterpret_cast<const float4*>(kr + (t + 1) * LD + 4 * d4);
      }
      const bool kp = keep(t);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        float a = 0.f;
#pragma unroll
        for (int d4 = 0; d4 < 4; ++d4) {
          a = fmaf(qp[i][4 * d4], rb[d4].x, a);
          a = fmaf(qp[i][4 * d4 + 1], rb[d4].y, a);
          a = fmaf(qp[i][4 * d4 + 2], rb[d4].z, a);
          a = fmaf(qp[i][4 * d4 + 3], rb[d4].w, a);
        }
        a = oct_sum(a);
        x[i][t] = kp ? a * c : -INFINITY;
        mx[i] = fmaxf(mx[i], x[i][t]);
      }
#pragma unroll
      for (int d4 = 0; d4 < 4; ++d4) rb[d4] = rn[d4];
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // For the rows t where use(t): p_i = exp2(x[i][t] - mn[i]), f(t, p_0, p_1),
  // o_i += round(p_i) * vs[t] (P cast to v's type before P.V, :185).
  auto pv = [&](const float (&mn)[2], auto use, auto f) __attribute__((always_inline)) {
    float4 rb[4], rn[4];
    const float* vr = vs + f0;
#pragma unroll
    for (int d4 = 0; d4 < 4; ++d4) rb[d4] = *reinterpret_cast<const float4*>(vr + 4 * d4);
#pragma unroll
    for (int t = 0; t < CH; ++t) {
      if (t + 1 < CH) {
#pragma unroll
        for (int d4 = 0; d4 < 4; ++d4) rn[d4] = *reinterpret_cast<const float4*>(vr + (t + 1) * LD + 4 * d4);
      }
      if (use(t)) {
        const float p0 = fast_exp2(x[0][t] - mn[0]);
        const float p1 = fast_exp2(x[1][t] - mn[1]);
        f(t, p0, p1);
        const float pr[2] = {EL::round(p0), EL::round(p1)};
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int d4 = 0; d4 < 4; ++d4) {
            op[i][4 * d4] = fmaf(pr[i], rb[d4].x, op[i][4 * d4]);
            op[i][4 * d4 + 1] = fmaf(pr[i], rb[d4].y, op[i][4 * d4 + 1]);
            op[i][4 * d4 + 2] = fmaf(pr[i], rb[d4].z, op[i][4 * d4 + 2]);
            op[i][4 * d4 + 3] = fmaf(pr[i], rb[d4].w, op[i][4 * d4 + 3]);
          }
      }
#pragma unroll
      for (int d4 = 0; d4 < 4; ++d4) rb[d4] = rn[d4];
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // The running max of row i rises to mn: rescale its accumulators (and Gamma unless literal).
  auto rescale = [&](const float (&mn)[2], bool with_gamma) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float al = fast_exp2(m[i] - mn[i]);  // 0 on the first step
      l[i] *= al;
      if (with_gamma) gam[i] *= al;
#pragma unroll
      for (int dd = 0; dd < 16; ++dd) op[i][dd] *= al;
      m[i] = mn[i];
    }
  };

  // Keys [key0, key0 + cn), cn <= 32, all valid: one online-softmax step (:174-186).
  auto chunk = [&](int key0, int cn) __attribute__((always_inline)) {
    __syncthreads();
    for (int i = tid; i < cn * D; i += 256) {
      const int t = i / D;
      const int d = i - t * D;
      const int64_t off = sbase + (int64_t)(key0 + t) * D + d;
      ks[t * LD + d] = EL::load(k, off);
      vs[t * LD + d] = EL::load(v, off);
    }
    __syncthreads();
    auto valid = [&](int t) { return t < cn; };
    float mx[2];
    scores(valid, mx);
    const float mn[2] = {fmaxf(m[0], mx[0]), fmaxf(m[1], mx[1])};
    rescale(mn, false);
    pv(mn, valid, [&](int, float p0, float p1) {
      l[0] += p0;
      l[1] += p1;
    });
  };
  auto keys = [&](int a, int b) __attribute__((always_inline)) {
    for (int k0 = a; k0 < b; k0 += CH) chunk(k0, min(CH, b - k0));
  };

  if (I >= 0) {
    const uint32_t* mrow = all ? nullptr : selmask + ((int64_t)bh * NT + I) * NW;
    if (all) {
      keys(0, T);
    } else {
      for (int w = 0; w < NW; ++w) {
        uint32_t bits = mrow[w];
        while (bits) {
          const int j = 32 * w + __builtin_ctz(bits);
          bits &= bits - 1u;
          keys(j * BT, min(T, (j + 1) * BT));
        }
      }
    }
    keys(T, seg);  // the prompt keys, exact for every video row
    if (!all) {
      // Phase 2 (:212-253): per group, the blocks not selected.
      const int last_len = T - (NT - 1) * BT;
      const float* kcb = kc + (int64_t)bh * NT * D;
      const float* vcb = vc + (int64_t)bh * NT * D;
      const float* hgb = hgroup + (int64_t)bh * NG * D * D;
      auto selected = [&](int j) { return (mrow[j >> 5] >> (j & 31)) & 1u; };
      // Bit t set: block jc + t (t < cn) is approximated, i.e. not selected.
      auto unselected_bits = [&](int jc, int cn) -> uint32_t {
        const int w = jc >> 5;
        const int sh = jc & 31;
        uint32_t sel = mrow[w] >> sh;
        if (sh != 0 && w + 1 < NW) sel |= mrow[w + 1] << (32 - sh);
        return ~sel & (cn >= 32 ? 0xffffffffu : (1u << cn) - 1u);
      };
      // kbar and V^ rows jc .. jc + cn - 1 into ks / vs, in the input type (:216-217, :238).
      auto zstage = [&](int jc, int cn, bool with_v) __attribute__((always_inline)) {
        __syncthreads();
        for (int i = tid; i < cn * D; i += 256) {
          const int t = i / D;
          const int d = i - t * D;
          const int64_t off = (int64_t)(jc + t) * D + d;
          ks[t * LD + d] = EL::round(kcb[off]);
          if (with_v) vs[t * LD + d] = EL::round(vcb[off]);
        }
        __syncthreads();
      };
      for (int g = 0; g < NG; ++g) {
        const int j0 = g * G;
        const int j1 = min(NT, j0 + G);
        int napprox = 0;
        for (int j = j0; j < j1; ++j) napprox += selected(j) ? 0 : 1;
        if (napprox == 0) continue;  // nothing approximated: alpha = 1 and no contribution
        // Zero order over the group's unselected blocks, 32 at a time: the group max first
        // (a group of at most 32 blocks keeps its scores and rows for the second pass).
        const bool one = j1 - j0 <= CH;
        float gm[2] = {-INFINITY, -INFINITY};
        for (int jc = j0; jc < j1; jc += CH) {
          const int cn = min(CH, j1 - jc);
          zstage(jc, cn, one);
          const uint32_t ub = unselected_bits(jc, cn);
          float mx[2];
          scores([&](int t) { return ((ub >> t) & 1u) != 0u; }, mx);
          gm[0] = fmaxf(gm[0], mx[0]);
          gm[1] = fmaxf(gm[1], mx[1]);
        }
        const float mn[2] = {fmaxf(m[0], gm[0]), fmaxf(m[1], gm[1])};
        rescale(mn, !gamma_literal);  // the literal form never rescales Gamma (:231-235)
        float ps[2] = {0.f, 0.f};
        for (int jc = j0; jc < j1; jc += CH) {
          const int cn = min(CH, j1 - jc);
          const uint32_t ub = unselected_bits(jc, cn);
          auto keep = [&](int t) { return ((ub >> t) & 1u) != 0u; };
          if (!one) {
            zstage(jc, cn, true);
            float mx[2];
            scores(keep, mx);
          }
          pv(mn, keep, [&](int t, float p0, float p1) {
            const float len = (float)(jc + t == NT - 1 ? last_len : BT);  // :242-243
            ps[0] += p0;
            ps[1] += p1;
            gam[0] += p0 * len;
            gam[1] += p1 * len;
          });
        }
        // First order (:246-253): r = q . Hbar_g (Hbar in q's type), o += r * (sum p * scale).
        float rr[2][16];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int dd = 0; dd < 16; ++dd) rr[i][dd] = 0.f;
        for (int d0 = 0; d0 < D; d0 += TR) {
          const int dn = min(TR, D - d0);
          __syncthreads();
          for (int i = tid; i < dn * D; i += 256) {
            const int dr = i / D;
            const int e = i - dr * D;
            kv[dr * LD + e] = EL::round(hgb[((int64_t)g * D + d0 + dr) * D + e]);
          }
          __syncthreads();
          for (int dr = 0; dr < dn; ++dr) {
            const float qv[2] = {qsh[rp * LD + d0 + dr], qsh[(rp + 32) * LD + d0 + dr]};
            const float4* hr = reinterpret_cast<const float4*>(kv + dr * LD + f0);
#pragma unroll
            for (int d4 = 0; d4 < 4; ++d4) {
              const float4 hh = hr[d4];
#pragma unroll
              for (int i = 0; i < 2; ++i) {
                rr[i][4 * d4] = fmaf(qv[i], hh.x, rr[i][4 * d4]);
                rr[i][4 * d4 + 1] = fmaf(qv[i], hh.y, rr[i][4 * d4 + 1]);
                rr[i][4 * d4 + 2] = fmaf(qv[i], hh.z, rr[i][4 * d4 + 2]);
                rr[i][4 * d4 + 3] = fmaf(qv[i], hh.w, rr[i][4 * d4 + 3]);
              }
            }
          }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const float f = ps[i] * scale;
#pragma unroll
          for (int dd = 0; dd < 16; ++dd) op[i][dd] = fmaf(rr[i][dd], f, op[i][dd]);
        }
      }
    }
  } else {
    keys(kbeg, kend);
  }
  // o = A / (L + Gamma) (:258-259), stored in the input type (:262).
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = rp + 32 * i;
    if (r < rows) {
      const float den = l[i] + gam[i];
#pragma unroll
      for (int dd = 0; dd < 16; ++dd) {
        const int e = f0 + dd;
        if (e < D) EL::store(o, sbase + (int64_t)(row0 + r) * D + e, op[i][dd] / den);
      }
    }
  }
}

namespace {

template <typename F>
hipError_t by_dtype(int dtype, F&& f) {
  switch (dtype) {
    case kAnyF32: f(F32E{}); break;
    case kAnyBf16: f(Bf16E{}); break;
    case kAnyF16: f(F16E{}); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_block_stats_any(const void* q, const void* k, const void* v, float* qc, float* kc, float* vc,
                                  float* hnorm, float* hgroup, int bh, int T, int Tslice, int D, int BT, int G,
                                  int dtype, hipStream_t stream) {
  if (D < 1 || D > 128 || BT < 1 || G < 1) return hipErrorInvalidValue;
  const int NT = (T + BT - 1) / BT;
  const int NG = (NT + G - 1) / G;
  const dim3 grid(NG, bh);
  return by_dtype(dtype, [&](auto el) {
    hipLaunchKernelGGL(k2_block_stats_any<decltype(el)>, grid, dim3(256), 0, stream, q, k, v, qc, kc, vc, hnorm,
                       hgroup, T, Tslice, D, BT, NT, G);
  });
}

hipError_t launch_scores_any(const float* qc, const float* kc, const float* hnorm, const float* noise, float scale,
                             int use_cov_bias, float* scores, int bh, int NT, int D, hipStream_t stream) {
  if (D < 1 || D > 128) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k3_scores_any, dim3(NT, (NT + 255) / 256, bh), dim3(256), 0, stream, qc, kc, hnorm, noise,
                     scale, use_cov_bias, scores, NT, D);
  return hipGetLastError();
}

int64_t sparse_attn_any_tiles(int T, int text, int text_valid, int BT) {
  const int64_t NT = (T + BT - 1) / BT;
  const int64_t tpb = (BT + kAnyTile - 1) / kAnyTile;
  return NT * tpb + (text_valid + kAnyTile - 1) / kAnyTile + (text - text_valid + kAnyTile - 1) / kAnyTile;
}

hipError_t launch_sparse_attn_any(const void* q, const void* k, const void* v, const float* kc, const float* vc,
                                  const float* hgroup, const uint32_t* selmask, void* o, float scale, int bh, int T,
                                  int text, int text_valid, int D, int BT, int G, int gamma_literal, int all,
                                  int dtype, hipStream_t stream) {
  if (D < 1 || D > 128 || BT < 1 || G < 1 || text_valid < 0 || text_valid > text) return hipErrorInvalidValue;
  if (!all && (kc == nullptr || vc == nullptr || hgroup == nullptr || selmask == nullptr)) return hipErrorInvalidValue;
  const int NT = (T + BT - 1) / BT;
  const int NG = (NT + G - 1) / G;
  const int NW = (NT + 31) / 32;
  const dim3 grid((unsigned)sparse_attn_any_tiles(T, text, text_valid, BT), bh);
  const float c = scale * kLog2e;
  return by_dtype(dtype, [&](auto el) {
    hipLaunchKernelGGL(k4_sparse_attn_any<decltype(el)>, grid, dim3(256), 0, stream, q, k, v, kc, vc, hgroup,
                       selmask, o, scale, c, T, text, text_valid, D, BT, NT, G, NG, NW, gamma_literal, all);
  });
}

}  // namespace pasa
