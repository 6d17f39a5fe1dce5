// K2: per-key-block statistics and the per-group first-order moment.
//
// Reference: fused_chunk_reduce_kernel, svg/kernels/triton/group_pisa_attention.py:66-129
// (means :101-102, value sum :103, H = K^T V - kc vc^T :106-107, ||H||^2 :110),
// sqrt on the host :287, and compute_h_group :291-301 (zero-padded mean over G).
//
// One workgroup (4 wavefronts) owns one group of G consecutive key blocks of one
// (batch, head) slice and walks its blocks in order.  Per block it streams the
// Q, K, V tiles from HBM once, forms the column sums (fixed order, deterministic),
// computes H_j = K_j^T V_j on the MFMA (each wave owns one quadrant of the D x D
// matrix), subtracts kc vc^T, reduces ||H_j||_F and adds H_j into the group
// accumulator held in registers.  H_j is never written to memory; the group
// mean is written once per group.  All statistics are fp32.
#include <type_traits>

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

// D = 128, BT = 128: the same statistics with the block loads overlapped.  K and V
// tiles go straight into double-buffered LDS (direct loads, 256-byte rows with 16-byte
// chunk c of row r at c ^ 4(r & 3)); Q rows go to registers.  Block j+1's loads are in
// flight while block j is reduced.  H_j = K^T V reads both MFMA operands with the
// transposing ds_read_b64_tr_b16 (K^T as A, V as B; the same token order in both); the K
// and V column sums are two more MFMAs per step against a ones operand, and the Q column
// sums are per-thread sums of its Q rows.  The Q sums and ||H_j||^2 reach LDS as per-wave
// partials that the next block's barrier publishes (one workgroup barrier per block).
// PERM: q, k, v are frame-major; the statistics are those of their token-major view (rm),
// and the token-major view itself is written to qt (unless NULL), kt, vt: each row of a block goes out
// from the registers (Q) and the LDS tiles (K, V), and the workgroup of group 0 copies
// the text rows [T, Tslice), which stay in place.
// E: the 16-bit element type of q, k, v (Bf16 or F16).
// BT 128 (two 64 KB buffer pairs: one workgroup per CU) or 64 (two per CU).
template <int BT, bool PERM, typename E = Bf16>
__global__ __launch_bounds__(256, 128 / BT) void k2_block_stats_dma(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, float* __restrict__ qc, float* __restrict__ kc,
    float* __restrict__ vc, float* __restrict__ hnorm, float* __restrict__ hgroup, int T, int Tslice,
    int NT, int G, RowMap rm, int split, float* __restrict__ partials, uint16_t* __restrict__ qt,
    uint16_t* __restrict__ kt, uint16_t* __restrict__ vt) {
  constexpr int D = 128;
  constexpr int TILE = BT * 256;
  constexpr bool RQ = BT < 128;  // 256 VGPRs (two workgroups per CU): see qv below
  __shared__ __attribute__((aligned(1024))) unsigned char Kb[2 * TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char Vb[2 * TILE];
  __shared__ float qpart[2][4][D];  // per-wave Q column sums of the last two blocks
  __shared__ float npart[2][4];     // per-wave ||H_j||^2

  // Workgroup (g, part) of a split group takes the part-th of `split` equal runs of its blocks.
  const int g = blockIdx.x / split;
  const int part = blockIdx.x - g * split;
  const int bh = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5;
  const int l32 = lane & 31;
  const int dq = (wave >> 1) * 64;
  const int eq = (wave & 1) * 64;
  const int nblk = min(G, NT - g * G);           // blocks in this group
  const int per = (nblk + split - 1) / split;
  const int j0 = g * G + min(part * per, nblk);
  const int j1 = g * G + min((part + 1) * per, nblk);

  const int64_t slice = (int64_t)bh * Tslice * D;
  const uint32_t slice_bytes = (uint32_t)T * D * 2u;  // rows >= T read as zero
  const rsrc_t qr = make_rsrc(q + slice, slice_bytes);
  const u32x4_t kd = make_rsrc_words(k + slice, slice_bytes);
  const u32x4_t vd = make_rsrc_words(v + slice, slice_bytes);
  const uint32_t kb_lds = lds_addr(Kb);
  const uint32_t vb_lds = lds_addr(Vb);

  // Direct loads: load n of wave w covers rows 16n + 4w + lane/16 (chunk lane % 16).
  const int lrow = lane >> 4;
  const int lch = lane & 15;
  const uint32_t t_lane = (uint32_t)((4 * wave + lrow) * 256 + ((lch ^ (4 * lrow)) << 4));
  const bool perm = PERM && slice_permuted(rm, bh);
  // Stored row of logical row r (rows past T are not permuted and read as zero).
  auto st = [&](int r) -> uint32_t { return (uint32_t)(perm ? map_row(r, rm) : r); };
  // Load slot n of block j: K and V rows 16n + 4 wave + lane/16 (direct to LDS buffer
  // buf) and Q rows 16n + t/16, chunk t % 16 (thread t, into registers).  A block's
  // slots are issued spread over the previous block's work, so that no wave stalls
  // issuing a block's worth of loads at once.  Every row is read once here, so the loads
  // are nontemporal (nt): 4-5% faster at c2 and c3 than cached loads, bit-identical.
  const int prow = tid >> 4;
  const int pc = tid & 15;
  auto load_kv = [&](int buf, int j, int n) {
    uint32_t off, soff;
    if (perm) {
      off = st(j * BT + 16 * n + 4 * wave + lrow) * 256u + (t_lane & 255u);
      soff = 0u;
    } else {
      off = t_lane + 16 * n * 256;
      soff = (uint32_t)j * BT * 256u;
    }
    dma_load16_lds_nt(kd, kb_lds + buf * TILE + (16 * n + 4 * wave) * 256, off, soff);
    dma_load16_lds_nt(vd, vb_lds + buf * TILE + (16 * n + 4 * wave) * 256, off, soff);
  };
  auto load_q = [&](int j, int n, uint4& qdst) {
    qdst = buf_load16_nt(qr, (st(j * BT + 16 * n + prow) * D + pc * 8) * 2u);
  };
  auto load_slot = [&](int buf, int j, int n, uint4& qdst) {
    load_kv(buf, j, n);
    load_q(j, n, qdst);
  };

  // Transposing operand reads: lane gets feature 32 ft + l32, tokens 4h + {0..3} (lo)
  // and 8 + 4h + {0..3} (hi) of token step s.
  const int g16 = lane >> 4;
  const int i16 = lane & 15;
  auto tofs = [&](int ft) {
    return (4 * (g16 >> 1) + (i16 >> 2)) * 256 +
           ((4 * (ft ^ (i16 >> 2)) + 2 * (g16 & 1) + ((i16 & 3) >> 1)) << 4) + 8 * (i16 & 1);
  };
  // This wave's feature tiles: K^T rows dq + 32 mt, V columns eq + 32 nt.
  const int kofs[2] = {tofs(dq / 32), tofs(dq / 32 + 1)};
  const int vofs[2] = {tofs(eq / 32), tofs(eq / 32 + 1)};
  auto frag = [&](const unsigned char* base, int ofs, int s) {
    const uint2 lo = lds_read_tr16(base, ofs + s * 16 * 256);
    const uint2 hi = lds_read_tr16(base, ofs + s * 16 * 256 + 8 * 256);
    return as_vec8<E>((u32x4_t){lo.x, lo.y, hi.x, hi.y});
  };

  f32x16_t gacc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) gacc[a][b][r] = 0.f;
  const typename E::vec8 ones = as_vec8<E>((u32x4_t){E::kOne2, E::kOne2, E::kOne2, E::kOne2});

  // The Q column sums and ||H_j||^2 of block j reach LDS as per-wave partials (buffer
  // j & 1) and are finished after the next block's barrier, so a block costs one
  // workgroup barrier.
  auto finish = [&](int jj, int b, int nn) {
    // At BT = 64 the thread's addresses are formed here each time from a fresh copy of its
    // index: kept live across the block loop instead, they are what the compiler spills.
    int t = tid;
    if (RQ) asm volatile("" : "+v"(t));
    if (t < D) {
      const float sm = ((qpart[b][0][t] + qpart[b][1][t]) + qpart[b][2][t]) + qpart[b][3][t];
      qc[((int64_t)bh * NT + jj) * D + t] = sm / (float)nn;
    } else if (t == D) {
      const float sn = ((npart[b][0] + npart[b][1]) + npart[b][2]) + npart[b][3];
      hnorm[(int64_t)bh * NT + jj] = sqrtf(sn);
    }
  };

  // Q rows of the current block (qv) and of the next (qn).  At BT = 64 (two workgroups per
  // CU, 256 VGPRs) a second set does not fit beside the accumulators: the next block's rows
  // land in qv once the column sums have read them (RQ).  At BT = 128 they load into qn
  // from the start of the block, which is 2-3% faster there.
  uint4 qv[BT / 16], qn[RQ ? 1 : BT / 16];
  auto qnext = [&](int n) -> uint4& { return RQ ? qv[n] : qn[RQ ? 0 : n]; };
  if (j0 < j1) {
#pragma unroll
    for (int n = 0; n < BT / 16; ++n) load_slot(0, j0, n, qv[n]);
  }
  // One block.  PRE: block j+1 exists and its loads are issued here, slots 0 and 1 at
  // once and slot s2 + 2 at MFMA step s2 (a compile-time choice, so that the MFMA loop
  // is one basic block).
  auto block = [&](auto pre_c, int j) {
    constexpr bool PRE = decltype(pre_c)::value;
    const int buf = (j - j0) & 1;
    const int n = min(BT, T - j * BT);
    wait_vmcnt<0>();           // block j's K, V (LDS) and Q (registers) landed
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();  // every wave's parts; block j-1's tile reads and partials done
    asm volatile("" ::: "memory");
    if (j > j0) finish(j - 1, buf ^ 1, min(BT, T - (j - 1) * BT));
    if (PRE) {
      load_kv(buf ^ 1, j + 1, 0);
      load_kv(buf ^ 1, j + 1, 1);
      if (!RQ) {
        load_q(j + 1, 0, qnext(0));
        load_q(j + 1, 1, qnext(1));
      }
    }
    const unsigned char* Kt = Kb + buf * TILE;
    const unsigned char* Vt = Vb + buf * TILE;
    if (PERM) {  // the token-major copies (rows past T hold text)
#pragma unroll
      for (int p = 0; p < BT / 16; ++p) {
        const int r = 16 * p + prow;
        if (j * BT + r < T) {
          const int off = r * 256 + ((pc ^ (4 * (r & 3))) << 4);
          const int64_t e = slice + (int64_t)(j * BT + r) * D + pc * 8;
          if (qt != nullptr) *reinterpret_cast<uint4*>(qt + e) = qv[p];
          *reinterpret_cast<uint4*>(kt + e) = lds_ld<uint4>(Kt, off);
          *reinterpret_cast<uint4*>(vt + e) = lds_ld<uint4>(Vt, off);
        }
      }
    }

    // H_j quadrant = K^T V, and on the same fragments the K and V column sums: K^T 1
    // (element r of a lane: feature dq + 32 mt + mfma32_row(r, h), the row layout the
    // correction needs) and 1^T V (every element: feature eq + 32 nt + l32, the lane's
    // column).  Rows >= n are zero in both tiles.  Before it, the Q column sums: thread
    // (prow, pc) adds its rows 16 p + prow of chunk pc.
    f32x16_t acc[2][2], ak[2], av[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
#pragma unroll
      for (int r = 0; r < 16; ++r) ak[a][r] = av[a][r] = 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;
    }
    float ps[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) ps[i] = 0.f;
#pragma unroll
    for (int p = 0; p < BT / 16; ++p) {
      float f[8];
      E::widen8(qv[p], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) ps[i] += f[i];
    }
    // The four 16-lane rows of the wave hold the same chunks: add them with the swaps.  At
    // BT = 64 this runs before the MFMA steps, so that the sums are not live through them.
    auto store_qsum = [&]() {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float x = ps[i];
        {
          const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
          x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
        ps[i] = halves_sum(x);
      }
      if (lane < 16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) qpart[buf][wave][lane * 8 + i] = ps[i];
      }
    };
    if (RQ) store_qsum();
    if (PRE && RQ) {
      load_q(j + 1, 0, qnext(0));
      load_q(j + 1, 1, qnext(1));
    }
#pragma unroll
    for (int s2 = 0; s2 < BT / 16; ++s2) {
      if (PRE && s2 + 2 < BT / 16) load_slot(buf ^ 1, j + 1, s2 + 2, qnext(s2 + 2));
      typename E::vec8 af[2], bfr[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) af[mt] = frag(Kt, kofs[mt], s2);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) bfr[nt] = frag(Vt, vofs[nt], s2);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = E::mfma(af[mt], bfr[nt], acc[mt][nt]);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) ak[mt] = E::mfma(af[mt], ones, ak[mt]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) av[nt] = E::mfma(ones, bfr[nt], av[nt]);
    }
    if (!RQ) store_qsum();
    // Means: sum / n, a product by the exact reciprocal when n is a power of two (every
    // full block), else the correctly rounded division.
    const float nf = (float)n;
    f32x16_t (&km)[2] = ak;  // the sums become the means in place
    if ((n & (n - 1)) == 0) {
      const float rn = 1.f / nf;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) km[mt][r] = ak[mt][r] * rn;
    } else {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) km[mt][r] = ak[mt][r] / nf;
    }
    if (eq == 0 && l32 == 0) {  // waves 0 and 2, lanes 0 and 32: kc of features dq .. dq + 63
      float* dst = kc + ((int64_t)bh * NT + j) * D + dq + 4 * h;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq)
          *reinterpret_cast<float4*>(dst + 32 * mt + 8 * rq) =
              make_float4(km[mt][4 * rq], km[mt][4 * rq + 1], km[mt][4 * rq + 2], km[mt][4 * rq + 3]);
    }
    if (dq == 0 && h == 0) {  // waves 0 and 1: vc of features eq .. eq + 63
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) vc[((int64_t)bh * NT + j) * D + eq + 32 * nt + l32] = av[nt][0];
    }
    float nrm[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float hv = acc[mt][nt][r] - km[mt][r] * av[nt][0];
          nrm[r & 3] += hv * hv;
          gacc[mt][nt][r] += hv;
        }
    const float nsum = wave_sum_xor((nrm[0] + nrm[1]) + (nrm[2] + nrm[3]));
    if (lane == 0) npart[buf][wave] = nsum;
    if (!RQ) {
#pragma unroll
      for (int p = 0; p < BT / 16; ++p) qv[p] = qnext(p);
    }
  };
  for (int j = j0; j < j1; ++j) {
    if (j + 1 < j1)
      block(std::true_type{}, j);
    else
      block(std::false_type{}, j);
  }
  if (j0 < j1) {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();  // the last block's partials
    asm volatile("" ::: "memory");
    finish(j1 - 1, (j1 - 1 - j0) & 1, min(BT, T - (j1 - 1) * BT));
  }

  if (PERM && g == 0 && part == 0) {  // the text rows, in place in both layouts
    const int64_t n16 = (int64_t)(Tslice - T) * (D / 8);
    const int64_t base = slice + (int64_t)T * D;
    for (int64_t i = tid; i < n16; i += 256) {
      if (qt != nullptr)
        *reinterpret_cast<uint4*>(qt + base + 8 * i) = *reinterpret_cast<const uint4*>(q + base + 8 * i);
      *reinterpret_cast<uint4*>(kt + base + 8 * i) = *reinterpret_cast<const uint4*>(k + base + 8 * i);
      *reinterpret_cast<uint4*>(vt + base + 8 * i) = *reinterpret_cast<const uint4*>(v + base + 8 * i);
    }
  }

  // Unsplit: the group mean (the reference zero-pads the last group to G blocks).
  // Split: this part's raw sum, reduced in a fixed order by k2_group_reduce.
  const int NG = (NT + G - 1) / G;
  float* hg = split == 1 ? hgroup + ((int64_t)bh * NG + g) * D * D
                         : partials + (((int64_t)bh * NG + g) * split + part) * D * D;
  const float Gf = split == 1 ? (float)G : 1.0f;
  int t = tid;  // at BT = 64 the lane's indices formed afresh, not kept live through the block loop
  if (RQ) asm volatile("" : "+v"(t));
  const int hx = (t >> 5) & 1;
  const int lx = t & 31;
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int e = eq + nt * 32 + lx;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = dq + mt * 32 + mfma32_row(r, hx);
        hg[d * D + e] = split == 1 ? gacc[mt][nt][r] / Gf : gacc[mt][nt][r];
      }
    }
}

// hgroup[bh, g] = (sum over parts p = 0..split-1 of partials[bh, g, p]) / G, summed in
// part order (deterministic).  One float4 of one group per thread; 256 threads cover a
// 1024-element slab of the group's D*D matrix, so a launch has NG * bh * D*D/1024
// workgroups (1536 at the Wan-1.3B shape) rather than one per group.
__global__ __launch_bounds__(256) void k2_group_reduce(const float* __restrict__ partials,
                                                       float* __restrict__ hgroup, int split, int G, int dd,
                                                       int64_t groups) {
  const int slabs = dd / 1024;
  const int64_t grp = blockIdx.x / slabs;
  if (grp >= groups) return;
  const int i = (int)(blockIdx.x - grp * slabs) * 256 + threadIdx.x;  // float4 index within the group
  const int n4 = dd / 4;
  const float4* src = reinterpret_cast<const float4*>(partials + grp * split * (int64_t)dd);
  float4 a = src[i];
  for (int p = 1; p < split; ++p) {
    const float4 b = src[(int64_t)p * n4 + i];
    a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
  }
  const float Gf = (float)G;
  reinterpret_cast<float4*>(hgroup + grp * (int64_t)dd)[i] = make_float4(a.x / Gf, a.y / Gf, a.z / Gf, a.w / Gf);
}

// Parts per group: enough workgroups for about two per CU (256 CUs) when the grid of
// groups alone is small, at least 4 blocks per part.  Only the D = 128 direct-to-LDS
// kernels split.
int block_stats_split(int bh, int T, int D, int BT, int G) {
  if (D != 128 || (BT != 128 && BT != 64)) return 1;
  const int NT = (T + BT - 1) / BT;
  const int64_t groups = (int64_t)((NT + G - 1) / G) * bh;
  const int nblk = min(G, NT);
  int split = 1;
  while (split < 8 && groups * split < 512 && nblk / (2 * split) >= 4) split *= 2;
  return split;
}

hipError_t launch_block_stats(const void* q, const void* k, const void* v, float* qc, float* kc,
                              float* vc, float* hnorm, float* hgroup, int bh, int T, int Tslice, int D,
                              int BT, int G, const RowMap* rm, void* const* tm_copies, float* partials, int split,
                              bool f16, hipStream_t stream) {
  const int NT = (T + BT - 1) / BT;
  const int NG = (NT + G - 1) / G;
  if (split < 1 || split > G || (split > 1 && (partials == nullptr || D != 128 || (BT != 128 && BT != 64))))
    return hipErrorInvalidValue;
  if (f16 && D != 128) return hipErrorInvalidValue;  // fp16 inputs: the D = 128 kernels only
  dim3 grid(NG * split, bh);
  auto a = (const uint16_t*)q;
  auto b = (const uint16_t*)k;
  auto c = (const uint16_t*)v;
  auto dma = [&](auto kern, const RowMap& map, void* const* cp) {
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, a, b, c, qc, kc, vc, hnorm, hgroup, T, Tslice, NT, G, map,
                       split, partials, cp ? (uint16_t*)cp[0] : nullptr, cp ? (uint16_t*)cp[1] : nullptr,
                       cp ? (uint16_t*)cp[2] : nullptr);
  };
  if (rm != nullptr) {  // token-major view of frame-major slices: D = 128, BT = 128 only
    if (D != 128 || BT != 128 || tm_copies == nullptr) return hipErrorInvalidValue;
    if (f16)
      dma(k2_block_stats_dma<128, true, F16>, *rm, tm_copies);
    else
      dma(k2_block_stats_dma<128, true, Bf16>, *rm, tm_copies);
  } else if (D == 128 && BT == 128) {
    if (f16)
      dma(k2_block_stats_dma<128, false, F16>, RowMap{}, nullptr);
    else
      dma(k2_block_stats_dma<128, false, Bf16>, RowMap{}, nullptr);
  } else if (D == 128 && BT == 64) {
    if (f16)
      dma(k2_block_stats_dma<64, false, F16>, RowMap{}, nullptr);
    else
      dma(k2_block_stats_dma<64, false, Bf16>, RowMap{}, nullptr);
  } else if (D == 64 && BT == 128)
    hipLaunchKernelGGL((k2_block_stats<64, 128>), grid, dim3(256), 0, stream, a, b, c, qc, kc, vc,
                       hnorm, hgroup, T, Tslice, NT, G);
  else if (D == 64 && BT == 64)
    hipLaunchKernelGGL((k2_block_stats<64, 64>), grid, dim3(256), 0, stream, a, b, c, qc, kc, vc,
                       hnorm, hgroup, T, Tslice, NT, G);
  else
    return hipErrorInvalidValue;
  if (split > 1) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t groups = (int64_t)NG * bh;  // D = 128: D*D / 1024 = 16 slabs per group
    hipLaunchKernelGGL(k2_group_reduce, dim3((unsigned)(groups * (D * D / 1024))), dim3(256), 0, stream,
                       (const float*)partials, hgroup, split, G, D * D, groups);
  }
  return hipGetLastError();
}

}  // namespace pasa
