// K4: block-sparse flash attention with per-group first-order correction.
//
// Reference: pisa_pg_fwd_kernel, svg/kernels/triton/group_pisa_attention.py:135-262
//   Phase 1 (:170-186): exact online softmax (base 2) over the selected key
//     blocks; columns >= T masked.
//   Phase 2 (:212-253): per group g of 32 key blocks, the blocks not selected
//     contribute p_j (V^_j + s * Hbar_g^T q) with p_j = 2^(c q.kbar_j - m);
//     A and L are rescaled when the running max rises, Gamma = sum p_j n_j is
//     not (the reference's literal form, :201/:243; gamma_literal = 0 gives the
//     rescaled "consistent" form).
//   Finalize (:258-262): o = A / (L + Gamma).
//
// MI355X mapping.  One workgroup = one (slice, query block) of BT rows; one
// wavefront per 32 query rows.  Everything is computed transposed so that the softmax
// statistics of a query row stay in the lanes that hold it.  In the D = 64 kernel
// (k4_sparse_attn) a lane owns one query (lane % 32):
//   S^T[key][q]  = K  * Q^T   (v_mfma_f32_32x32x16_bf16, K from LDS, Q in VGPRs)
//   O^T[e][q]   += V^T * P^T   (V^T read from the row-major V tile with
//                               ds_read_b64_tr_b16, P from the S^T accumulators)
// The S^T accumulator of a lane holds, per 16-key step s, exactly the 8 keys
// (16s + 8i' + 4h + j) its P^T B-operand slots need; two transposing LDS reads
// fetch the matching V^T slots.  Keys of a block are consumed in halves of 64
// (one online-softmax step each) to bound live accumulators.  The D = 128 kernel
// (k4_sparse_attn_dma) runs the same transposed products on the 16x16x32 MFMA, a lane
// owning two query rows (its lane layout is described at the kernel).
//
// Phase 1 walks the selected blocks in ascending block order (the selection
// bitmask) instead of top-k order: exact online softmax is order-independent up
// to rounding, and the ascending sweep keeps the workgroups of one XCD on
// nearby key blocks at the same time, so the K/V tiles they share hit in L2.
// Workgroups are mapped XCD-aware: each XCD walks a contiguous run of query
// blocks of the same head.
//
// Two kernels.  k4_sparse_attn_dma (D = 128) loads K/V tiles straight into LDS
// (buffer_load ... lds, XOR-swizzled rows), double-buffered between the K and V
// tiles, with an exact online softmax.  At BT = 64 it runs two query blocks per
// four-wave workgroup (PAIR), each wave pair on its own selected tiles in lock
// step: co-resident workgroups on a CU drift into start-time cohorts, each sweeping
// a different region of key space, and pairing halves the number of cohorts (and so
// the L2 working set), while each group's phase-2 operands are loaded once for both
// blocks.  k4_sparse_attn (D = 64) stages tiles through registers; its online
// softmax is the same exact one (rescale whenever a row's max rises).
//
// Both keep the row sum of P in fp32 (adds, not v_dot2c_f32_bf16: on gfx950 a dot
// instruction issues only between the MFMAs of the SIMD's other wave, so it stalls
// its wave behind the partner's MFMA stream).
//
// Phase-2 operands (kbar, V^ transposed, Hbar transposed; in the input's 16-bit type) are
// packed per (slice, group) by k4_pack / k4_pack_xor into the exact LDS image K4 copies in.
// The D = 128 kernels and k4_pack_xor take that type as a template argument (Bf16 or
// F16: the MFMA and the rounding of P, the pack and o); the D = 64 ones are bf16.
#include "common.h"
#include "k4_layout.h"
#include "kernels.h"

namespace pasa {

template <int D, int BT>
struct K4Cfg {
  static constexpr int WAVES = BT / 32;
  static constexpr int THREADS = WAVES * 64;
  static constexpr int CH = D / 8;
  using KT = PadTile<D>;       // K tile:        BT rows x D
  // V tile: BT rows x D, natural chunk order, row stride 2D + 64 bytes, which
  // makes the transposing reads of 32 lanes (4 rows x 2 chunks per 16-lane
  // group, two groups side by side) hit 64 distinct banks.
  static constexpr int VROW = 2 * D + 64;
  using PKB = PadTile<D>;      // kbar:          32 rows x D
  using PVT = PadTile<kGroup>; // V^ transposed: D rows x 32 means (tok_perm order)
  using PHT = PadTile<D>;      // Hbar^T:        D rows (e) x D (d)
  static constexpr int KS_BYTES = KT::bytes(BT);
  static constexpr int P1_BYTES = KS_BYTES + BT * VROW;
  static constexpr int PK_VT_OFF = PKB::bytes(kGroup);
  static constexpr int PK_HT_OFF = PK_VT_OFF + PVT::bytes(D);
  static constexpr int PK_RAW = PK_HT_OFF + PHT::bytes(D);
  static constexpr int PK_BYTES = (PK_RAW + 16 * THREADS - 1) / (16 * THREADS) * (16 * THREADS);
  static constexpr int LDS_BYTES = P1_BYTES > PK_BYTES ? P1_BYTES : PK_BYTES;
  static constexpr int K_LOADS = (BT * D / 8) / THREADS;   // 16-byte K chunks per thread
  static constexpr int V_LOADS = K_LOADS;                  // 16-byte V chunks per thread
  static constexpr int PK_LOADS = PK_BYTES / 16 / THREADS;
  static_assert(K_LOADS * THREADS * 8 == BT * D, "K tile split");
  static_assert(THREADS % CH == 0, "K rows per pass");
};


// ---- phase-2 operand pack ---------------------------------------------------

template <int D, int BT>
__global__ __launch_bounds__(256) void k4_pack(const float* __restrict__ kc,
                                               const float* __restrict__ vc,
                                               const float* __restrict__ hgroup,
                                               unsigned char* __restrict__ pack, int NT, int NG) {
  using C = K4Cfg<D, BT>;
  const int g = blockIdx.x;
  const int bh = blockIdx.y;
  unsigned char* out = pack + ((int64_t)bh * NG + g) * C::PK_BYTES;
  const float* kb = kc + (int64_t)bh * NT * D;
  const float* vb = vc + (int64_t)bh * NT * D;
  const float* hb = hgroup + ((int64_t)bh * NG + g) * D * D;
  for (int u = threadIdx.x; u < kGroup * D; u += 256) {
    const int m = u / D;
    const int d = u - m * D;
    const int jj = g * kGroup + m;
    const float x = jj < NT ? kb[(int64_t)jj * D + d] : 0.f;
    *(uint16_t*)(out + C::PKB::elem_byte(m, d)) = (uint16_t)f32_to_bf16_bits(x);
  }
  for (int u = threadIdx.x; u < D * kGroup; u += 256) {
    const int m = u % kGroup;
    const int e = u / kGroup;
    const int jj = g * kGroup + m;
    const float x = jj < NT ? vb[(int64_t)jj * D + e] : 0.f;
    *(uint16_t*)(out + C::PK_VT_OFF + C::PVT::elem_byte(e, tok_perm(m))) =
        (uint16_t)f32_to_bf16_bits(x);
  }
  for (int u = threadIdx.x; u < D * D; u += 256) {
    const int d = u / D;  // Hbar[d][e] row-major in, Hbar^T[e][d] out
    const int e = u - d * D;
    *(uint16_t*)(out + C::PK_HT_OFF + C::PHT::elem_byte(e, d)) = (uint16_t)f32_to_bf16_bits(hb[u]);
  }
}

// One workgroup per (group, slice).  Every output element is written once, as part of
// a 16-byte chunk: Hbar^T goes through LDS (coalesced fp32 reads of Hbar rows, column
// reads from a padded tile), kbar rows are read as 32-byte runs, V^T columns with the
// token index fastest across lanes.  Rounding is round-to-nearest-even, as everywhere.
template <int BT, typename E = Bf16>
__global__ __launch_bounds__(256) void k4_pack_xor(const float* __restrict__ kc,
                                                   const float* __restrict__ vc,
                                                   const float* __restrict__ hgroup,
                                                   unsigned char* __restrict__ pack, int NT, int NG) {
  using P = K4DPack<BT>;
  constexpr int D = 128;
  constexpr int HS = D + 1;  // padded row of the fp32 Hbar tile
  __shared__ float hs[D * HS];
  const int g = blockIdx.x;
  const int bh = blockIdx.y;
  const int tid = threadIdx.x;
  unsigned char* out = pack + ((int64_t)bh * NG + g) * P::BYTES;
  const float* kb = kc + (int64_t)bh * NT * D;
  const float* vb = vc + (int64_t)bh * NT * D;
  const float* hb = hgroup + ((int64_t)bh * NG + g) * D * D;
#pragma unroll 4
  for (int it = 0; it < D * D / 4 / 256; ++it) {
    const int idx = it * 256 + tid;
    const int d = idx >> 5;
    const int e4 = (idx & 31) * 4;
    const float4 x = *(const float4*)(hb + d * D + e4);
    hs[d * HS + e4 + 0] = x.x;
    hs[d * HS + e4 + 1] = x.y;
    hs[d * HS + e4 + 2] = x.z;
    hs[d * HS + e4 + 3] = x.w;
  }
  // kbar: rows m (block of the group) x 16 chunks of 8 features, XOR layout.
  unsigned char* part2 = out + P::HT_BYTES;
#pragma unroll
  for (int it = 0; it < kGroup * D / 8 / 256; ++it) {
    const int qi = it * 256 + tid;
    const int m = qi >> 4;
    const int cc = qi & 15;
    const int jj = g * kGroup + m;
    float f[8];
    if (jj < NT) {
      const float4 x0 = *(const float4*)(kb + (int64_t)jj * D + cc * 8);
      const float4 x1 = *(const float4*)(kb + (int64_t)jj * D + cc * 8 + 4);
      f[0] = x0.x; f[1] = x0.y; f[2] = x0.z; f[3] = x0.w;
      f[4] = x1.x; f[5] = x1.y; f[6] = x1.z; f[7] = x1.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = 0.f;
    }
    const uint4 w = make_uint4(E::pack2(f[0], f[1]), E::pack2(f[2], f[3]), E::pack2(f[4], f[5]), E::pack2(f[6], f[7]));
    *(uint4*)(part2 + P::KB_OFF + xor_tile_byte(m, cc * 8)) = w;
  }
  // V^T: feature rows e x 4 chunks of 8 blocks (vt_block_of order), kVtRow bytes per row.
#pragma unroll
  for (int it = 0; it < D * kGroup / 8 / 256; ++it) {
    const int qi = it * 256 + tid;
    const int e = qi & (D - 1);
    const int cc = qi >> 7;
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int jj = g * kGroup + vt_block_of(cc, i);
      f[i] = jj < NT ? vb[(int64_t)jj * D + e] : 0.f;
    }
    const uint4 w = make_uint4(E::pack2(f[0], f[1]), E::pack2(f[2], f[3]), E::pack2(f[4], f[5]), E::pack2(f[6], f[7]));
    *(uint4*)(part2 + P::VT_OFF + e * kVtRow + cc * 16) = w;
  }
  __syncthreads();
  // Hbar^T: row e, chunk cc holds Hbar[8 cc .. 8 cc + 7][e].
#pragma unroll 2
  for (int it = 0; it < D * D / 8 / 256; ++it) {
    const int qi = it * 256 + tid;
    const int e = qi >> 4;
    const int cc = qi & 15;
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = hs[(cc * 8 + i) * HS + e];
    const uint4 w = make_uint4(E::pack2(f[0], f[1]), E::pack2(f[2], f[3]), E::pack2(f[4], f[5]), E::pack2(f[6], f[7]));
    *(uint4*)(out + xor_tile_byte(e, cc * 8)) = w;
  }
}

// ---- main kernel ------------------------------------------------------------

template <int D, int BT>
__global__ __attribute__((amdgpu_flat_work_group_size(1, 256), amdgpu_waves_per_eu(2, 2)))
void k4_sparse_attn(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                    const uint16_t* __restrict__ v, const unsigned char* __restrict__ pack,
                    const uint32_t* __restrict__ selmask, uint16_t* __restrict__ o, float scale,
                    float c, int T, int NT, int NG, int NW, int xcd_chunk, int gamma_literal) {
  using C = K4Cfg<D, BT>;
  using KT = typename C::KT;
  __shared__ __attribute__((aligned(16))) unsigned char lds[C::LDS_BYTES];
  unsigned char* Ks = lds;
  unsigned char* Vs = lds + C::KS_BYTES;

  // XCD-aware workgroup -> (slice, query block) map: consecutive workgroup ids
  // go to consecutive XCDs, so slot = wg / 8 indexes within one XCD's run.
  const int wg = blockIdx.x;
  const int xcd = wg & 7;
  const int slot = wg >> 3;
  const int bh = slot / xcd_chunk;
  const int qb = xcd * xcd_chunk + (slot - bh * xcd_chunk);
  if (qb >= NT) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;
  const int l32 = lane & 31;
  const int64_t slice = (int64_t)bh * T * D;
  const int qrow = qb * BT + wave * 32 + l32;  // the query this lane owns

  const uint32_t slice_bytes = (uint32_t)T * D * 2u;
  const rsrc_t qr = make_rsrc(q + slice, slice_bytes);
  const rsrc_t kr = make_rsrc(k + slice, slice_bytes);
  const rsrc_t vr = make_rsrc(v + slice, slice_bytes);

  // Q fragments (B operand of S^T and of r^T): lane holds Q[qrow][16ks + 8h .. +7].
  bf16x8_t qf[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
    qf[ks] = as_bf16x8(buf_load16(qr, ((uint32_t)qrow * D + ks * 16 + h * 8) * 2u));

  f32x16_t oacc[D / 32];
#pragma unroll
  for (int et = 0; et < D / 32; ++et)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[et][r] = 0.f;
  float l_run = 0.f;
  float g_run = 0.f;

  const uint32_t* mrow = selmask + ((int64_t)bh * NT + qb) * NW;

  // Lane-constant parts of the tile load / store / read addresses.
  constexpr int KROWS = C::THREADS / C::CH;  // rows covered per load pass
  const uint32_t goff = (uint32_t)((tid / C::CH) * D + (tid % C::CH) * 8) * 2u;
  const int k_soff = KT::chunk_byte(tid / C::CH, tid % C::CH);
  const int v_soff = (tid / C::CH) * C::VROW + (tid % C::CH) * 16;
  const int ka_base = KT::frag_base(l32, h);
  // Transposing V reads: group g = lane / 16 covers keys +4*(g/2) and columns
  // +16*(g%2); lane i of the group addresses row i/4, columns 4*(i%4) .. +3.
  const int g16 = lane >> 4;
  const int i16 = lane & 15;
  const int vtr_base = (4 * (g16 >> 1) + (i16 >> 2)) * C::VROW + (16 * (g16 & 1) + 4 * (i16 & 3)) * 2;

  // ---------------- Phase 1: exact attention over the selected blocks --------
  uint4 kreg[C::K_LOADS];
  uint4 vreg[C::V_LOADS];
  auto fetch = [&](int blk) {
    const uint32_t base = (uint32_t)blk * BT * D * 2u + goff;
#pragma unroll
    for (int it = 0; it < C::K_LOADS; ++it) kreg[it] = buf_load16(kr, base + it * KROWS * D * 2);
#pragma unroll
    for (int it = 0; it < C::V_LOADS; ++it) vreg[it] = buf_load16(vr, base + it * KROWS * D * 2);
  };
  auto stash = [&]() {
#pragma unroll
    for (int it = 0; it < C::K_LOADS; ++it) lds_st(Ks, k_soff + it * KROWS * KT::ROW_BYTES, kreg[it]);
#pragma unroll
    for (int it = 0; it < C::V_LOADS; ++it) lds_st(Vs, v_soff + it * KROWS * C::VROW, vreg[it]);
  };

  // Selected blocks in ascending order, from the selection bitmask (uniform).
  int wsel = 0;
  uint32_t bits = NW > 0 ? mrow[0] : 0u;
  auto next_selected = [&]() -> int {
    while (bits == 0u) {
      if (++wsel >= NW) return -1;
      bits = mrow[wsel];
    }
    const int j = 32 * wsel + __builtin_ctz(bits);
    bits &= bits - 1u;
    return j;
  };

  float m_run = -INFINITY;  // exact running max of the scores (log2 units)
  int blk = next_selected();
  if (blk >= 0) fetch(blk);
  while (blk >= 0) {
    const int nxt = next_selected();
    __syncthreads();
    stash();
    __syncthreads();
    if (nxt >= 0) fetch(nxt);

    const int nvalid = min(BT, T - blk * BT);
#pragma unroll
    for (int kh = 0; kh < BT / 64; ++kh) {
      if (kh * 64 >= nvalid) break;  // fully masked half (ragged last block)
      f32x16_t sacc[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[mt][r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const bf16x8_t a = as_bf16x8(
              lds_ld<uint4>(Ks, ka_base + (kh * 64 + mt * 32) * KT::ROW_BYTES + ks * 16));
          sacc[mt] = mfma32(a, qf[ks], sacc[mt]);
        }
      if (nvalid < (kh + 1) * 64) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (kh * 64 + mt * 32 + mfma32_row(r, h) >= nvalid) sacc[mt][r] = -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[mt][r]);
      const float mxc = halves_max(mx) * c;
      if (__any(mxc > m_run)) {
        const float m_new = fmaxf(m_run, mxc);
        const float alpha = fast_exp2(m_run - m_new);  // 0 on the first step
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int et = 0; et < D / 32; ++et)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[et][r] *= alpha;
      }
      bf16x8_t pf[4];
      float lsum[4] = {0.f, 0.f, 0.f, 0.f};  // fp32 row sum of p, as gpa.py:182-184
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p0 = fast_exp2(fmaf(sacc[s4 >> 1][8 * (s4 & 1) + 2 * i], c, -m_run));
          const float p1 = fast_exp2(fmaf(sacc[s4 >> 1][8 * (s4 & 1) + 2 * i + 1], c, -m_run));
          w[i] = pack_bf16x2(p0, p1);
          lsum[i] += p0 + p1;
        }
        pf[s4] = __builtin_bit_cast(bf16x8_t, (u32x4_t){w[0], w[1], w[2], w[3]});
      }
      l_run += (lsum[0] + lsum[1]) + (lsum[2] + lsum[3]);
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const int rowk = 16 * (kh * 4 + s4);
#pragma unroll
        for (int et = 0; et < D / 32; ++et) {
          const int off = vtr_base + rowk * C::VROW + et * 64;
          const uint2 lo = lds_read_tr16(Vs, off);
          const uint2 hi = lds_read_tr16(Vs, off + 8 * C::VROW);
          const bf16x8_t a = __builtin_bit_cast(bf16x8_t, (u32x4_t){lo.x, lo.y, hi.x, hi.y});
          oacc[et] = mfma32(a, pf[s4], oacc[et]);
        }
      }
    }
    blk = nxt;
  }

  // ---------------- Phase 2: zero- + first-order correction per group --------
  using PKB = typename C::PKB;
  using PVT = typename C::PVT;
  using PHT = typename C::PHT;
  const unsigned char* Pkb = lds;
  const unsigned char* Pvt = lds + C::PK_VT_OFF;
  const unsigned char* Pht = lds + C::PK_HT_OFF;
  const int kb_base = PKB::frag_base(l32, h);
  const int pv_base = PVT::frag_base(l32, h);
  const int ph_base = PHT::frag_base(l32, h);
  const int last_len = T - (NT - 1) * BT;
  for (int g = 0; g < NG; ++g) {
    // Blocks of this group that take the approximation (uniform over the workgroup).
    const int nin = min(kGroup, NT - g * kGroup);
    const uint32_t inrange = nin >= 32 ? 0xffffffffu : ((1u << nin) - 1u);
    const uint32_t approx = inrange & ~mrow[g];
    if (approx == 0u) continue;  // every block exact or absent: no contribution

    __syncthreads();
    {
      const uint4* src = (const uint4*)(pack + ((int64_t)bh * NG + g) * C::PK_BYTES);
      uint4 preg[C::PK_LOADS];
#pragma unroll
      for (int i = 0; i < C::PK_LOADS; ++i) preg[i] = src[i * C::THREADS + tid];
#pragma unroll
      for (int i = 0; i < C::PK_LOADS; ++i) ((uint4*)lds)[i * C::THREADS + tid] = preg[i];
    }
    __syncthreads();

    f32x16_t sb;
#pragma unroll
    for (int r = 0; r < 16; ++r) sb[r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const bf16x8_t a = as_bf16x8(lds_ld<uint4>(Pkb, kb_base + ks * 16));
      sb = mfma32(a, qf[ks], sb);
    }
    float gmx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int mm = mfma32_row(r, h);
      if (!((approx >> mm) & 1u)) sb[r] = -INFINITY;
      gmx = fmaxf(gmx, sb[r]);
    }
    const float m_new = fmaxf(m_run, halves_max(gmx) * c);
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
    if (!gamma_literal) g_run *= alpha;
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int et = 0; et < D / 32; ++et)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[et][r] *= alpha;
    }
    float psum = 0.f;
    float gsum = 0.f;
    bf16x8_t pbf[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r0 = 8 * s + 2 * i;
        const float p0 = fast_exp2(fmaf(sb[r0], c, -m_new));
        const float p1 = fast_exp2(fmaf(sb[r0 + 1], c, -m_new));
        const int j0 = g * kGroup + mfma32_row(r0, h);
        const int j1 = g * kGroup + mfma32_row(r0 + 1, h);
        psum += p0 + p1;
        gsum += p0 * (float)(j0 == NT - 1 ? last_len : BT) + p1 * (float)(j1 == NT - 1 ? last_len : BT);
        w[i] = pack_bf16x2(p0, p1);
      }
      pbf[s] = __builtin_bit_cast(bf16x8_t, (u32x4_t){w[0], w[1], w[2], w[3]});
    }
    g_run += gsum;
    psum = halves_sum(psum);
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int et = 0; et < D / 32; ++et) {
        const bf16x8_t a = as_bf16x8(lds_ld<uint4>(Pvt, pv_base + et * 32 * PVT::ROW_BYTES + s * 16));
        oacc[et] = mfma32(a, pbf[s], oacc[et]);
      }
    f32x16_t racc[D / 32];
#pragma unroll
    for (int et = 0; et < D / 32; ++et)
#pragma unroll
      for (int r = 0; r < 16; ++r) racc[et][r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
      for (int et = 0; et < D / 32; ++et) {
        const bf16x8_t a = as_bf16x8(lds_ld<uint4>(Pht, ph_base + et * 32 * PHT::ROW_BYTES + ks * 16));
        racc[et] = mfma32(a, qf[ks], racc[et]);
      }
    const float f = psum * scale;
#pragma unroll
    for (int et = 0; et < D / 32; ++et)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[et][r] = fmaf(racc[et][r], f, oacc[et][r]);
  }

  // ---------------- Finalize ---------------------------------------------------
  const float denom = halves_sum(l_run) + halves_sum(g_run);
  if (qrow < T) {
    uint16_t* orow = o + slice + (int64_t)qrow * D;
#pragma unroll
    for (int et = 0; et < D / 32; ++et)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int e0 = et * 32 + 8 * rq + 4 * h;
        uint2 w;
        w.x = pack_bf16x2(oacc[et][4 * rq + 0] / denom, oacc[et][4 * rq + 1] / denom);
        w.y = pack_bf16x2(oacc[et][4 * rq + 2] / denom, oacc[et][4 * rq + 3] / denom);
        *(uint2*)(orow + e0) = w;
      }
  }
}

// ---- D = 128: tiles loaded straight into LDS ----------------------------------
//
// Same computation as k4_sparse_attn, restructured for D = 128 so that the K/V
// tiles never pass through VGPRs: buffer_load_dwordx4 ... lds writes each lane's
// 16 bytes to LDS directly (zeros past the end of the slice), which frees the
// staging registers for deeper LDS-operand prefetching while two workgroups
// still share each CU.  Per block i, with one K and one V buffer, two barriers:
//   wait K_i -> barrier -> load V_i -> S = K_i Q^T -> softmax
//   -> wait V_i -> barrier -> load K_{i+1} -> O += V_i P
// Each barrier both publishes a landed tile and frees the other buffer, so V_i
// streams in during S + softmax and K_{i+1} during P.V.
//
// The products run on the 16x16x32 MFMA (v_mfma_f32_16x16x32_bf16 / _f16).  Under the
// chip's power limit it sustains about 11% more FLOP/s than the 32x32x16 form on
// real-valued operands (1.94 against 1.75 PFLOP/s in a bare MFMA stream, at 1.93
// against 1.72 GHz): the same work per cycle for less energy.  Lane l of a wave owns
// query rows l % 16 and 16 + l % 16 of the wave's 32 (query tiles qt = 0, 1), and holds,
// per 16-key tile kt of S^T = K Q^T, keys 16 kt + 4 (l / 16) + {0..3} of both rows; a
// row's statistics are reduced over its four lanes l % 16 + 16 g.  For P.V the 8 keys of
// a 32-key step s a lane holds (tiles 2s and 2s + 1) are its B-operand k-slots as they
// stand, and two transposing LDS reads fetch the V^T A-operand slots for the same keys.
//
// Tiles use 256-byte rows with XOR-swizzled 16-byte chunks: K chunk c of row r sits at
// c ^ (r & 15) (the A-operand reads of 16 rows by one 16-lane group touch 16 distinct
// chunks), V chunk c at c ^ 2 (r & 7) (the transposing reads of 32 lanes, rows 8 apart,
// touch 16 distinct chunks).  The phase-2 pack image is loaded the same way.

// PAIR: two query blocks per workgroup, one wave group (QWAVES waves) each, with
// their K/V tiles side by side in the K and V buffers.
template <int BT, bool PAIR = false>
struct K4D {
  static constexpr int D = 128;
  static constexpr int QWAVES = BT / 32;                   // waves of one query block
  static constexpr int QBLOCKS = PAIR ? 2 : 1;             // query blocks per workgroup
  static constexpr int WAVES = QWAVES * QBLOCKS;
  static constexpr int THREADS = WAVES * 64;
  static constexpr int TILE = BT * 256;                    // bytes of one K or V tile
  static constexpr int VW = 4 / QWAVES;                    // 4-row load slots per wave per 16 rows
  static constexpr int TILE_LOADS = TILE / 1024 / QWAVES;  // 1 KB direct loads per wave per tile
  static constexpr int KT = BT / 16;                       // 16-key tiles of S per block
  static constexpr int KS = D / 32;                        // 32-feature k-steps
  static constexpr int DT = D / 16;                        // 16-feature tiles of O
  using PK = K4DPack<BT>;
  static constexpr int KBUF = QBLOCKS * TILE > PK::HT_BYTES ? QBLOCKS * TILE : PK::HT_BYTES;
  static constexpr int VBUF = QBLOCKS * TILE > PK::PART2 ? QBLOCKS * TILE : PK::PART2;
  static_assert(TILE_LOADS == 8, "load schedule");
  static_assert(WAVES == 4, "four-wave workgroups (BT = 128, or BT = 64 in pairs)");
  static_assert(PK::PART2 % (1024 * WAVES) == 0 && PK::HT_BYTES % (1024 * WAVES) == 0, "pack split");
};

// Byte offset in a V tile of the 8 bytes lane `lane` reads with ds_read_b64_tr_b16 for
// 16-feature tile dt and key rows row0 + 4 (lane / 16) + {0..3}: row row0 + 4 (lane / 16)
// + (lane % 16) / 4, features 16 dt + 4 (lane % 4) .. + 3 (chunk 2 dt + (lane % 4) / 2,
// half lane % 2), the chunk stored at c ^ 2 (row & 7).  row0 is a multiple of 16.
__device__ __forceinline__ int vtile_tr_byte(int row0, int dt, int lane) {
  const int r = row0 + 4 * (lane >> 4) + ((lane & 15) >> 2);
  const int c = 2 * dt + ((lane & 3) >> 1);
  return r * 256 + ((c ^ (2 * (r & 7))) << 4) + 8 * (lane & 1);
}

// Instruction-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

// ALL: dense attention (every key block exact, no selection read, no correction); a
// separate instantiation so that profiles tell the two launches apart.
// PERM: k and v are the token-major view (as pasa_block_stats_placed writes it), q is
// frame-major, and o is stored frame-major: the load and the store of a query row go
// through map_row.
// PAIR: two consecutive query blocks (or text query tiles) per workgroup (not ALL,
// not PERM).  Video blocks visit NS selected tiles each, so their barriers match
// (a shorter selection row, or a text pair spanning the prompt and the padding
// segment, idles through its partner's extra tiles); a pair past the last block
// repeats it and stores nothing.  Phase 2 visits the groups
// either block approximates; a group the other block approximates and this one
// does not adds exact zeros here (p = 0, alpha = 1), so each block's result is the
// one the unpaired kernel computes.
template <int BT, bool ALL, bool PERM, bool PAIR = false, typename E = Bf16>
__global__ __attribute__((amdgpu_flat_work_group_size(1, 256), amdgpu_waves_per_eu(2, 2)))
void k4_sparse_attn_dma(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                        const uint16_t* __restrict__ v, const unsigned char* __restrict__ pack,
                        const uint32_t* __restrict__ selmask, uint16_t* __restrict__ o,
                        float scale, float c, int T, int NT, int NG, int NW, int xcd_chunk,
                        int gamma_literal, int text, int text_valid, int n_text_wg, int nbh, RowMap rm) {
  static_assert(!PAIR || (!ALL && !PERM), "pairs run selected video blocks only");
  constexpr bool all_tiles = ALL;
  using C = K4D<BT, PAIR>;
  using PK = typename C::PK;
  using vec8 = typename E::vec8;
  constexpr int D = 128;
  constexpr int KT = C::KT, KS = C::KS, DT = C::DT;
  // Two distinct LDS objects, so the compiler can tell loads into one from reads of the other.
  __shared__ __attribute__((aligned(1024))) unsigned char Ks[C::KBUF];
  __shared__ __attribute__((aligned(1024))) unsigned char Vs[C::VBUF];

  // Each slice holds T blocked (video) rows followed by `text` text rows, of which the
  // first text_valid are the prompt and the rest padding.  Two segments attend only
  // within themselves: [0, seg) with seg = T + text_valid, and the padding [seg, T + text).
  // The first n_text_wg workgroups (a multiple of 8) each own one tile of text query
  // rows of one segment and attend densely to that segment's keys; they are the
  // longest-running ones, so they go first.  The rest own one query block (a pair of
  // blocks with PAIR) of the video rows; wg & 7 names their XCD, and each XCD takes a
  // contiguous run of a slice's query blocks (shared K/V tiles in its L2).
  const int wg = blockIdx.x;
  const bool dense = wg < n_text_wg;
  const int seg = T + text_valid;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = PAIR ? wave / C::QWAVES : 0;  // query block (tile) of this wave within the workgroup
  const int qw = PAIR ? wave - half * C::QWAVES : wave;  // wave within its query block
  // A pair's second block (tile) past the last one repeats it and stores nothing.
  bool store_rows = true;
  int bh, qb, qbw = 0, qrow0, row_limit, kbeg = 0, kend = seg;
  int pair_tiles = 0;  // PAIR: tiles of the longer half (the shorter one idles through the rest)
  if (dense) {
    const int vtiles = (text_valid + BT - 1) / BT;
    const int qtiles = vtiles + (text - text_valid + BT - 1) / BT;
    const int units = (qtiles + C::QBLOCKS - 1) / C::QBLOCKS;
    bh = wg / units;
    if (bh >= nbh) return;  // padding of the text range to a multiple of 8
    qb = 0;
    const int t0 = (wg - bh * units) * C::QBLOCKS;
    store_rows = t0 + half < qtiles;
    const int qt = store_rows ? t0 + half : t0;
    auto seg_tiles = [&](int t) { return t < vtiles ? (seg + BT - 1) / BT : (T + text - seg + BT - 1) / BT; };
    if (PAIR) pair_tiles = max(seg_tiles(t0), seg_tiles(min(t0 + 1, qtiles - 1)));
    if (qt < vtiles) {
      qrow0 = T + qt * BT;
      row_limit = seg;
    } else {
      qrow0 = seg + (qt - vtiles) * BT;
      row_limit = T + text;
      kbeg = seg;
      kend = T + text;
    }
  } else {
    const int w = wg - n_text_wg;
    const int xcd = w & 7;
    const int slot = w >> 3;
    bh = slot / xcd_chunk;
    qb = (xcd * xcd_chunk + (slot - bh * xcd_chunk)) * C::QBLOCKS;
    if (qb >= NT) return;
    store_rows = qb + half < NT;
    qbw = qb + (store_rows ? half : 0);
    qrow0 = qbw * BT;
    row_limit = T;
  }

  const int l16 = lane & 15;  // query row within a 16-row query tile; A-operand row
  const int g4 = lane >> 4;   // which 8 k-slots of an operand, which 4 rows of a result
  const int Ttot = T + text;
  const int64_t slice = (int64_t)bh * Ttot * D;
  const bool perm = PERM && slice_permuted(rm, bh);
  // This lane's two query rows (query tiles qt = 0, 1), and the frame-major rows their
  // output goes to (PERM: q is gathered through the same map).
  int qrow[2], qrow_st[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    qrow[qt] = qrow0 + qw * 32 + 16 * qt + l16;
    qrow_st[qt] = perm ? map_row(qrow[qt], rm) : qrow[qt];
  }

  const uint32_t slice_bytes = (uint32_t)Ttot * D * 2u;
  const rsrc_t qr = make_rsrc(q + slice, slice_bytes);
  // Q as B operands: qf[qt][ks] holds features 32 ks + 8 g4 .. + 7 of row qrow[qt].
  vec8 qf[2][KS];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[qt][ks] = as_vec8<E>(buf_load16(qr, ((uint32_t)(perm ? qrow_st[qt] : qrow[qt]) * D + ks * 32 + g4 * 8) * 2u));
  // Complete the Q loads now: vector-memory waits the compiler would place at their
  // first use inside the loop would also wait for the tile loads in flight there.
  wait_vmcnt<0>();

  // O^T accumulators: oacc[dt][qt] element i is feature 16 dt + 4 g4 + i of row qrow[qt].
  f32x4_t oacc[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int i = 0; i < 4; ++i) oacc[dt][qt][i] = 0.f;
  // Running max, row sum and Gamma of the two rows: m is the same on the four lanes of a
  // row; l and Gamma are this lane's partial sums (its keys), added over the four at the end.
  float l_run[2] = {0.f, 0.f};
  float g_run[2] = {0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY};

  // The selection row is read-only here: constant address space -> scalar loads,
  // which wait on lgkmcnt and leave the in-flight tile loads alone.
  typedef const __attribute__((address_space(4))) uint32_t* const_u32_ptr;
  const const_u32_ptr mrow = (const_u32_ptr)(selmask + ((int64_t)bh * NT + qbw) * NW);
  // PAIR: the rows of both blocks (phase 2 visits the groups either approximates).
  const const_u32_ptr mrow0 = (const_u32_ptr)(selmask + ((int64_t)bh * NT + qb) * NW);
  const const_u32_ptr mrow1 = (const_u32_ptr)(selmask + ((int64_t)bh * NT + min(qb + 1, NT - 1)) * NW);

  // Direct-load lane constants.  Load (vw, n) of this wave covers tile rows
  // 16n + 4*(qw + QWAVES*vw) + lane/16 of its query block's tile; the lane's 16 bytes
  // land at chunk lane % 16, so it fetches the logical chunk stored there.
  const int lrow = lane >> 4;
  const int lch = lane & 15;
  uint32_t k_lane[C::VW], v_lane[C::VW];
#pragma unroll
  for (int vw = 0; vw < C::VW; ++vw) {
    const int r = 4 * (qw + C::QWAVES * vw) + lrow;  // row mod 16
    k_lane[vw] = (uint32_t)(r * 256 + ((lch ^ r) << 4));
    v_lane[vw] = (uint32_t)(r * 256 + ((lch ^ (2 * (r & 7))) << 4));
  }

  const u32x4_t kd = make_rsrc_words(k + slice, slice_bytes);
  const u32x4_t vd = make_rsrc_words(v + slice, slice_bytes);
  const uint32_t ks_lds = lds_addr(Ks);
  const uint32_t vs_lds = lds_addr(Vs);
  // This query block's K and V tiles (phase 1); phase 2 uses the whole buffers.
  const int tile_off = half * C::TILE;
  const uint32_t kt_lds = ks_lds + tile_off;
  const uint32_t vt_lds = vs_lds + tile_off;
  // A tile is BT key rows starting at row `row0` of the slice (rows past the slice read as zero).
  auto load_k = [&](int row0) {
    const uint32_t soff = (uint32_t)row0 * 256u;
#pragma unroll
    for (int vw = 0; vw < C::VW; ++vw)
#pragma unroll
      for (int n = 0; n < BT / 16; ++n)
        dma_load16_lds(kd, kt_lds + (16 * n + 4 * (qw + C::QWAVES * vw)) * 256, k_lane[vw] + 16 * n * 256, soff);
  };
  auto load_v = [&](int row0) {
    const uint32_t soff = (uint32_t)row0 * 256u;
#pragma unroll
    for (int vw = 0; vw < C::VW; ++vw)
#pragma unroll
      for (int n = 0; n < BT / 16; ++n)
        dma_load16_lds(vd, vt_lds + (16 * n + 4 * (qw + C::QWAVES * vw)) * 256, v_lane[vw] + 16 * n * 256, soff);
  };

  // MFMA A-operand offsets of K-layout tiles (K, Hbar^T, kbar): row l16 of a 16-row tile,
  // chunk 4 ks + g4 (features 32 ks + 8 g4 .. + 7), stored at chunk ^ l16.
  int kofs[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) kofs[ks] = l16 * 256 + (((4 * ks + g4) ^ l16) << 4);
  // The transposing V reads of 32-key step s: keys 32 s + 16 h2 + 4 g4 + {0..3} (h2 = 0, 1).
  int vofs[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) vofs[dt] = vtile_tr_byte(0, dt, lane);

  int wsel = 0;
  int jall = 0;
  uint32_t bits = (!dense && !all_tiles && NW > 0) ? mrow[0] : 0u;
  auto next_selected = [&]() -> int {
    while (bits == 0u) {
      if (++wsel >= NW) return -1;
      bits = mrow[wsel];
    }
    const int j = 32 * wsel + __builtin_ctz(bits);
    bits &= bits - 1u;
    return j;
  };
  // Exact tiles in visiting order: a video query block takes its selected blocks in
  // ascending order, then the prompt rows [T, seg); a text query tile takes every row
  // of its segment [kbeg, kend).  Returns the tile's first row (-1 when done) and its
  // number of valid rows in nv.
  int tt = 0;
  auto next_tile = [&](int& nv) -> int {
    if (!dense) {
      const int j = all_tiles ? (jall < NT ? jall++ : -1) : next_selected();
      if (j >= 0) {
        nv = min(BT, T - j * BT);
        return j * BT;
      }
      kbeg = T;  // then the prompt rows
    }
    const int r = kbeg + tt * BT;
    if (r >= kend) return -1;
    ++tt;
    nv = min(BT, kend - r);
    return r;
  };

  // ---------------- Phase 1 ------------------------------------------------------
  // PAIR: the tile count of the longer half: for video blocks the longer of the two
  // selection rows (rows written by pasa_select all hold NS bits) plus the prompt
  // tiles; for text tiles, set above from the two segments.  The shorter half idles
  // through its partner's extra tiles below, so that the workgroup barriers match.
  int tiles_done = 0;
  if (PAIR && !dense) {
    int n0 = 0, n1 = 0;
    for (int w = 0; w < NW; ++w) {
      n0 += __builtin_popcount(mrow0[w]);
      n1 += __builtin_popcount(mrow1[w]);
    }
    pair_tiles = max(n0, n1) + (text_valid + BT - 1) / BT;
  }
  int nv_cur = 0;
  int blk = next_tile(nv_cur);
  if (blk >= 0) load_k(blk);
  while (blk >= 0) {
    int nv_nxt = 0;
    const int nxt = next_tile(nv_nxt);
    wait_vmcnt<0>();           // this wave's K_blk loads landed
    barrier_lds_reads_done();  // ... and every wave's; every wave is done reading the V buffer
    load_v(blk);

    // S^T = K Q^T: sacc[kt][qt] element i = key 16 kt + 4 g4 + i against row qrow[qt].
    f32x4_t sacc[KT][2];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sacc[kt][qt][i] = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const vec8 a = as_vec8<E>(lds_ld<uint4>(Ks + tile_off, kofs[ks] + kt * 16 * 256));
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) sacc[kt][qt] = E::mfma16(a, qf[qt][ks], sacc[kt][qt]);
      }
    // Keep 8 fragment reads in flight: each read feeds two MFMAs, consumed ~16 MFMAs
    // (~256 cycles) after it was issued, which covers the LDS latency.
    {
      constexpr int NR = KS * KT;
#pragma unroll
      for (int i = 0; i < 8; ++i) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
#pragma unroll
      for (int i = 0; i < NR - 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
    }

    const int nvalid = nv_cur;
    if (nvalid < BT) {
      // key 16 kt + 4 g4 + i is past the tile's rows iff 16 kt + i reaches lim;
      // comparing against immediates keeps no per-key constants live.
      const int lim = nvalid - 4 * g4;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (kt * 16 + i >= lim) sacc[kt][qt][i] = -INFINITY;
    }
    float mxc[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sacc[kt][qt][i]);
      mxc[qt] = quad16_max(mx) * c;
    }
    // One wave-uniform test per query tile: a tile whose 16 rows all kept their max skips
    // the 32 products of its O (they would multiply by exactly 1).
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      if (__any(mxc[qt] > m_run[qt])) {
        const float m_new = fmaxf(m_run[qt], mxc[qt]);
        const float alpha = fast_exp2(m_run[qt] - m_new);  // 0 on the first block, 1 if the max held
        m_run[qt] = m_new;
        l_run[qt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) oacc[dt][qt][i] *= alpha;
      }
    }
    // P in the B-operand layout of 32-key step s: slots 0-3 = tile 2s, 4-7 = tile 2s + 1.
    // The row sum adds the fp32 p (as gpa.py:182-184 sums `score` before its bf16
    // cast), then adds the tile's sum to the rescaled l.
    vec8 pf[KT / 2][2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float lsum[2] = {0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KT / 2; ++s) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4_t& src = sacc[2 * s + (j >> 1)][qt];
          const float p0 = fast_exp2(fmaf(src[2 * (j & 1)], c, -m_run[qt]));
          const float p1 = fast_exp2(fmaf(src[2 * (j & 1) + 1], c, -m_run[qt]));
          w[j] = E::pack2(p0, p1);
          lsum[j & 1] += p0 + p1;
        }
        pf[s][qt] = as_vec8<E>((u32x4_t){w[0], w[1], w[2], w[3]});
      }
      l_run[qt] += lsum[0] + lsum[1];
    }
    // V_blk is waited for only now, so its load overlaps S and the softmax.
    wait_vmcnt<0>();
    barrier_lds_reads_done();  // every wave's part of V_blk landed; every wave is done reading K_blk
    if (nxt >= 0) load_k(nxt);
#pragma unroll
    for (int s = 0; s < KT / 2; ++s)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint2 lo = lds_read_tr16(Vs + tile_off, vofs[dt] + s * 32 * 256);
        const uint2 hi = lds_read_tr16(Vs + tile_off, vofs[dt] + s * 32 * 256 + 16 * 256);
        const vec8 a = as_vec8<E>((u32x4_t){lo.x, lo.y, hi.x, hi.y});
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) oacc[dt][qt] = E::mfma16(a, pf[s][qt], oacc[dt][qt]);
      }
    // Read-ahead for the transposing V reads: two per A operand, which feeds two MFMAs.
    {
      constexpr int NM = (KT / 2) * DT * 2;
#pragma unroll
      for (int i = 0; i < 8; ++i) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 1);
#pragma unroll
      for (int i = 0; i < NM - 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 1);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 1);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 1);
    }
    blk = nxt;
    nv_cur = nv_nxt;
    if (PAIR) ++tiles_done;
  }
  if (PAIR) {
    for (; tiles_done < pair_tiles; ++tiles_done)
#pragma unroll
      for (int b = 0; b < 2; ++b) barrier_lds_reads_done();  // the loop's barriers per tile
  }
  barrier_lds_reads_done();  // every wave is done reading the V buffer

  // ---------------- Phase 2 ------------------------------------------------------
  const int last_len = T - (NT - 1) * BT;
  const u32x4_t pd = make_rsrc_words(pack + (int64_t)bh * NG * PK::BYTES, (uint32_t)(NG * PK::BYTES));
  // V^T of the group: row 16 dt + l16, chunk g4 (blocks 4 g4 + {0..3}, 16 + 4 g4 + {0..3}).
  const int pv_base = PK::VT_OFF + l16 * kVtRow + g4 * 16;
  const int ng_run = (dense || all_tiles) ? 0 : NG;  // text rows and dense attention: no correction term
  // Groups with at least one unselected in-range block (of either block of a pair),
  // in ascending order.
  auto inrange_of = [&](int g) -> uint32_t {
    const int nin = min(kGroup, NT - g * kGroup);
    return nin >= 32 ? 0xffffffffu : ((1u << nin) - 1u);
  };
  auto approx_of = [&](int g) -> uint32_t { return inrange_of(g) & ~mrow[g]; };
  auto visit_of = [&](int g) -> uint32_t {
    return PAIR ? inrange_of(g) & ~(mrow0[g] & mrow1[g]) : approx_of(g);
  };
  auto next_group = [&](int g) -> int {
    for (++g; g < ng_run; ++g)
      if (visit_of(g) != 0u) return g;
    return -1;
  };
  // A group's pack is two parts: kbar + V^T (part 2, into Vs) and Hbar^T (into Ks).
  // Part 2 of the next group loads while this group's Hbar^T product runs, and the
  // next Hbar^T loads while the next group's scores and P.V^ run.  Two barriers per
  // group: after P.V^ (part 2 of g read everywhere, Hbar^T of g landed) and after the
  // Hbar^T product (Hbar^T of g read everywhere, part 2 of the next group landed).
  constexpr int HT_LOADS = PK::HT_BYTES / 1024 / C::WAVES;
  constexpr int P2_LOADS = PK::PART2 / 1024 / C::WAVES;
  auto load_part2 = [&](int g) {
    const uint32_t gsoff = (uint32_t)(g * PK::BYTES);
#pragma unroll
    for (int n = 0; n < P2_LOADS; ++n) {
      const int kb = n * C::WAVES + wave;
      dma_load16_lds(pd, vs_lds + kb * 1024, (uint32_t)(PK::HT_BYTES + kb * 1024 + lane * 16), gsoff);
    }
  };
  auto load_ht = [&](int g) {
    const uint32_t gsoff = (uint32_t)(g * PK::BYTES);
#pragma unroll
    for (int n = 0; n < HT_LOADS; ++n) {
      const int kb = n * C::WAVES + wave;  // 1 KB piece of Hbar^T
      dma_load16_lds(pd, ks_lds + kb * 1024, (uint32_t)(kb * 1024 + lane * 16), gsoff);
    }
  };
  int g = next_group(-1);
  if (g >= 0) {  // phase 1 ended with a barrier after the last reads of Ks and Vs
    load_part2(g);
    load_ht(g);
    wait_vmcnt<HT_LOADS>();    // this wave's part 2 of group g landed (Hbar^T may be in flight)
    barrier_lds_reads_done();  // ... and every wave's
  }
  while (g >= 0) {
    const int gn = next_group(g);
    const uint32_t approx = approx_of(g);

    // s-bar^T = kbar Q^T: sb[bt][qt] element i = block 16 bt + 4 g4 + i of the group.
    f32x4_t sb[2][2];
#pragma unroll
    for (int bt = 0; bt < 2; ++bt)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sb[bt][qt][i] = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int bt = 0; bt < 2; ++bt) {
        const vec8 a = as_vec8<E>(lds_ld<uint4>(Vs, PK::KB_OFF + kofs[ks] + bt * 16 * 256));
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) sb[bt][qt] = E::mfma16(a, qf[qt][ks], sb[bt][qt]);
      }
    // Blocks of the group that are selected (or past NT) drop out: element i of sb[bt]
    // is block 16 bt + 4 g4 + i, so its keep mask is one sign-extended bit of approx >> 4 g4.
    const uint32_t ah = approx >> (4 * g4);
    float m_new[2], alpha[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float gmx = -INFINITY;
#pragma unroll
      for (int bt = 0; bt < 2; ++bt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t keep = (uint32_t)__builtin_amdgcn_sbfe((int)ah, 16 * bt + i, 1);
          sb[bt][qt][i] = __uint_as_float((__float_as_uint(sb[bt][qt][i]) & keep) | (~keep & 0xff800000u));  // -inf if dropped
          gmx = fmaxf(gmx, sb[bt][qt][i]);
        }
      m_new[qt] = fmaxf(m_run[qt], quad16_max(gmx) * c);
      alpha[qt] = fast_exp2(m_run[qt] - m_new[qt]);
      m_run[qt] = m_new[qt];
      l_run[qt] *= alpha[qt];
      if (!gamma_literal) g_run[qt] *= alpha[qt];
    }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
      if (__any(alpha[qt] != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) oacc[dt][qt][i] *= alpha[qt];
      }
    float psum[2];
    vec8 pbf[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4_t& src = sb[j >> 1][qt];
        const float p0 = fast_exp2(fmaf(src[2 * (j & 1)], c, -m_new[qt]));
        const float p1 = fast_exp2(fmaf(src[2 * (j & 1) + 1], c, -m_new[qt]));
        psum[qt] = j == 0 ? p0 + p1 : psum[qt] + (p0 + p1);  // no 0 + x: x may be -0
        w[j] = E::pack2(p0, p1);
      }
      pbf[qt] = as_vec8<E>((u32x4_t){w[0], w[1], w[2], w[3]});
    }
    // Gamma += sum_j p_j * n_j.  Every block holds BT rows except the last one, NT - 1,
    // which holds last_len: BT * sum(p) (exact, BT being a power of two), corrected for
    // that block in the one group holding it.
    float gsum[2] = {psum[0] * (float)BT, psum[1] * (float)BT};
    if (g == NG - 1 && last_len != BT) {
      const int mm_last = (NT - 1) - g * kGroup;  // block 16 bt + 4 g4 + i of the group
      if (g4 == ((mm_last >> 2) & 3)) {
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          float sl = sb[0][qt][0];
#pragma unroll
          for (int bt = 0; bt < 2; ++bt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (16 * bt + i == (mm_last & 16) + (mm_last & 3)) sl = sb[bt][qt][i];
          gsum[qt] += fast_exp2(fmaf(sl, c, -m_new[qt])) * (float)(last_len - BT);
        }
      }
    }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      g_run[qt] += gsum[qt];
      psum[qt] = quad16_sum(psum[qt]);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const vec8 a = as_vec8<E>(lds_ld<uint4>(Vs, pv_base + dt * 16 * kVtRow));
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) oacc[dt][qt] = E::mfma16(a, pbf[qt], oacc[dt][qt]);
    }
    wait_vmcnt<0>();           // this wave's Hbar^T of group g landed (nothing else is in flight)
    barrier_lds_reads_done();  // every wave is done reading part 2 of group g; Hbar^T of g is in place
    if (gn >= 0) load_part2(gn);

    // r^T = Hbar^T Q^T: racc[dt][qt] element i = feature 16 dt + 4 g4 + i of q.Hbar.
    f32x4_t racc[DT][2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int i = 0; i < 4; ++i) racc[dt][qt][i] = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const vec8 a = as_vec8<E>(lds_ld<uint4>(Ks, kofs[ks] + dt * 16 * 256));
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) racc[dt][qt] = E::mfma16(a, qf[qt][ks], racc[dt][qt]);
      }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const float f = psum[qt] * scale;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) oacc[dt][qt][i] = fmaf(racc[dt][qt][i], f, oacc[dt][qt][i]);
    }
    if (gn >= 0) wait_vmcnt<0>();  // this wave's part 2 of group gn landed
    barrier_lds_reads_done();      // every wave is done reading Hbar^T of g; part 2 of gn is in place
    if (gn >= 0) load_ht(gn);
    g = gn;
  }

  // O = A / (L + Gamma): one correctly rounded reciprocal per row, then products.
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float inv = 1.f / (quad16_sum(l_run[qt]) + quad16_sum(g_run[qt]));
    if (store_rows && qrow[qt] < row_limit) {
      uint16_t* orow = o + slice + (int64_t)qrow_st[qt] * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        uint2 w;
        w.x = E::pack2(oacc[dt][qt][0] * inv, oacc[dt][qt][1] * inv);
        w.y = E::pack2(oacc[dt][qt][2] * inv, oacc[dt][qt][3] * inv);
        *(uint2*)(orow + dt * 16 + 4 * g4) = w;
      }
    }
  }
}

size_t k4_pack_bytes(int D, int BT) {
  if (D == 128 && BT == 128) return K4DPack<128>::BYTES;
  if (D == 128 && BT == 64) return K4DPack<64>::BYTES;
  if (D == 64 && BT == 128) return K4Cfg<64, 128>::PK_BYTES;
  if (D == 64 && BT == 64) return K4Cfg<64, 64>::PK_BYTES;
  return 0;
}

hipError_t launch_pack_phase2(const float* kc, const float* vc, const float* hgroup, void* pack,
                              int bh, int T, int D, int BT, bool f16, hipStream_t stream) {
  const int NT = (T + BT - 1) / BT;
  const int NG = (NT + kGroup - 1) / kGroup;
  dim3 grid(NG, bh);
  auto out = (unsigned char*)pack;
  if (f16 && D != 128) return hipErrorInvalidValue;
  if (D == 128 && BT == 128) {
    if (f16)
      hipLaunchKernelGGL((k4_pack_xor<128, F16>), grid, dim3(256), 0, stream, kc, vc, hgroup, out, NT, NG);
    else
      hipLaunchKernelGGL((k4_pack_xor<128, Bf16>), grid, dim3(256), 0, stream, kc, vc, hgroup, out, NT, NG);
  } else if (D == 128 && BT == 64) {
    if (f16)
      hipLaunchKernelGGL((k4_pack_xor<64, F16>), grid, dim3(256), 0, stream, kc, vc, hgroup, out, NT, NG);
    else
      hipLaunchKernelGGL((k4_pack_xor<64, Bf16>), grid, dim3(256), 0, stream, kc, vc, hgroup, out, NT, NG);
  } else if (D == 64 && BT == 128)
    hipLaunchKernelGGL((k4_pack<64, 128>), grid, dim3(256), 0, stream, kc, vc, hgroup, out, NT, NG);
  else if (D == 64 && BT == 64)
    hipLaunchKernelGGL((k4_pack<64, 64>), grid, dim3(256), 0, stream, kc, vc, hgroup, out, NT, NG);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_sparse_attn(const void* q, const void* k, const void* v, const void* pack,
                              const int32_t* idx, const uint32_t* selmask, void* o, float scale,
                              int bh, int T, int text, int text_valid, int D, int BT, int NS,
                              int gamma_literal, const RowMap* rm, bool f16, hipStream_t stream) {
  if (text > 0 && D != 128) return hipErrorInvalidValue;  // the text segment is a D = 128 feature
  if (f16 && D != 128) return hipErrorInvalidValue;       // so are fp16 inputs
  if (text_valid < 0 || text_valid > text) return hipErrorInvalidValue;
  const int NT = (T + BT - 1) / BT;
  const int NG = (NT + kGroup - 1) / kGroup;
  const int NW = (NT + 31) / 32;
  const int xcd_chunk = (NT + 7) / 8;
  const int text_qtiles = (text_valid + BT - 1) / BT + (text - text_valid + BT - 1) / BT;
  const int n_text_wg = (bh * text_qtiles + 7) / 8 * 8;
  dim3 grid(n_text_wg + 8 * bh * xcd_chunk);
  dim3 grid_video(8 * bh * xcd_chunk);
  const float c = scale * kLog2e;
  auto a = (const uint16_t*)q;
  auto b = (const uint16_t*)k;
  auto cc = (const uint16_t*)v;
  auto pk = (const unsigned char*)pack;
  auto oo = (uint16_t*)o;
  // The D = 128 kernels, for either element type.
  auto dma = [&](auto kern, dim3 g, int chunk, int n_text, const RowMap& map) {
    hipLaunchKernelGGL(kern, g, dim3(256), 0, stream, a, b, cc, pk, selmask, oo, scale, c, T, NT, NG, NW, chunk,
                       gamma_literal, text, text_valid, n_text, bh, map);
  };
  static_assert(K4D<128>::THREADS == 256 && K4D<64, true>::THREADS == 256, "four-wave workgroups");
#define PASA_K4_LAUNCH(DD, BB)                                                                   \
  hipLaunchKernelGGL((k4_sparse_attn<DD, BB>), grid_video, dim3(K4Cfg<DD, BB>::THREADS), 0, stream, a, \
                     b, cc, pk, selmask, oo, scale, c, T, NT, NG, NW, xcd_chunk, gamma_literal)
  if (rm != nullptr) {  // token-major view of frame-major slices: D = 128, BT = 128 only
    if (D != 128 || BT != 128) return hipErrorInvalidValue;
    if (f16)
      dma(k4_sparse_attn_dma<128, false, true, false, F16>, grid, xcd_chunk, n_text_wg, *rm);
    else
      dma(k4_sparse_attn_dma<128, false, true, false, Bf16>, grid, xcd_chunk, n_text_wg, *rm);
  } else if (D == 128 && BT == 128) {
    if (f16)
      dma(k4_sparse_attn_dma<128, false, false, false, F16>, grid, xcd_chunk, n_text_wg, RowMap{});
    else
      dma(k4_sparse_attn_dma<128, false, false, false, Bf16>, grid, xcd_chunk, n_text_wg, RowMap{});
  } else if (D == 128 && BT == 64) {
    // Query blocks (and text tiles) in pairs: each XCD takes a contiguous run of a
    // slice's pairs.
    const int pair_chunk = ((NT + 1) / 2 + 7) / 8;
    const int n_text_pairs = (bh * ((text_qtiles + 1) / 2) + 7) / 8 * 8;
    const dim3 gp(n_text_pairs + 8 * bh * pair_chunk);
    if (f16)
      dma(k4_sparse_attn_dma<64, false, false, true, F16>, gp, pair_chunk, n_text_pairs, RowMap{});
    else
      dma(k4_sparse_attn_dma<64, false, false, true, Bf16>, gp, pair_chunk, n_text_pairs, RowMap{});
  }
  else if (D == 64 && BT == 128)
    PASA_K4_LAUNCH(64, 128);
  else if (D == 64 && BT == 64)
    PASA_K4_LAUNCH(64, 64);
  else
    return hipErrorInvalidValue;
#undef PASA_K4_LAUNCH
  return hipGetLastError();
}

hipError_t launch_dense_attn(const void* q, const void* k, const void* v, void* o, float scale, int bh,
                             int T, int text, int text_valid, bool f16, hipStream_t stream) {
  constexpr int BT = 128;
  if (T < 1 || text < 0 || text_valid < 0 || text_valid > text) return hipErrorInvalidValue;
  const int NT = (T + BT - 1) / BT;
  const int xcd_chunk = (NT + 7) / 8;
  const int text_qtiles = (text_valid + BT - 1) / BT + (text - text_valid + BT - 1) / BT;
  const int n_text_wg = (bh * text_qtiles + 7) / 8 * 8;
  dim3 grid(n_text_wg + 8 * bh * xcd_chunk);
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(K4D<BT>::THREADS), 0, stream, (const uint16_t*)q, (const uint16_t*)k,
                       (const uint16_t*)v, nullptr, nullptr, (uint16_t*)o, scale, scale * kLog2e, T, NT, 0, 0,
                       xcd_chunk, 1, text, text_valid, n_text_wg, bh, RowMap{});
  };
  if (f16)
    launch(k4_sparse_attn_dma<BT, true, false, false, F16>);
  else
    launch(k4_sparse_attn_dma<BT, true, false, false, Bf16>);
  return hipGetLastError();
}

}  // namespace pasa
