// K3: covariance-aware block scores and deterministic per-row top-k.
//
// Reference: svg/kernels/triton/group_pisa_attention.py:365-375
//   score = einsum(qc, kc * scale) + log(h_norm + 1e-6) [+ randn per key block]
//   indices = topk(score, NS).indices  (descending)
// Scores are fp32 here (the reference's einsum runs in the input dtype; parity
// is defined against fp32 math).  torch.topk leaves the order of equal scores
// unspecified; this kernel fixes it: (score desc, index asc), -0.0 == +0.0.
//
// Stage 1 (k3_scores): a 64x128-tile fp32 GEMM on the fp32 MFMA (persistent workgroups,
//   features double-buffered through LDS), with a fixed d-order, plus the per-key-block
//   log bias.
// Stage 2 (k3_topk): one wavefront per row finds the NS-th largest score by a bitwise
//   search over the orderable 32-bit score (ballot counts, narrowed to one register once
//   the bucket holding it is small), takes the ties at it by lowest index, emits the
//   selection bitmask (one bit per key block) from the ballots of the picks and, when the
//   caller asks for the index list, sorts the NS selected 64-bit keys
//   (orderable(score) << 32 | ~index) with a bitonic network.  K4 reads only the bitmask,
//   so the attention call skips the index list (the reference's indices never leave its
//   operator either).
#include "common.h"
#include "kernels.h"

namespace pasa {

constexpr int kScoreTJ = 128;  // key blocks per workgroup tile
constexpr int kScoreDC = 32;   // features per pipeline stage (one 128-byte row segment)

// Byte offset, inside an LDS stage block of 128-byte rows, of 16-byte chunk c (of 8) of
// tile row r: the chunk is stored at c ^ ((r >> 1) & 7), so the float4 reads of any 16
// consecutive rows at one logical chunk touch 16 distinct 16-byte bank groups.
__host__ __device__ __forceinline__ constexpr int score_chunk_byte(int r, int c) {
  return r * 128 + ((c ^ ((r >> 1) & 7)) << 4);
}

// Each workgroup computes 64 x 128 tiles of the score matrices (query blocks x key
// blocks), one after another (tile blockIdx.x, then + gridDim.x, ...; the grid is sized
// to three workgroups per CU), so a tile's stores drain while the next tile is
// multiplied.  Four waves each compute 32 query rows x 64 key columns as two 32 x 32
// sub-tiles on the fp32 MFMA (v_mfma_f32_32x32x2_f32).  The features are consumed in
// stages of 32, double-buffered in LDS (48 KB): the qc and kc rows of the next stage
// (the next tile's first stage after a tile's last) stream in by direct-to-LDS loads
// (rows past NT read as zero) while the current stage is multiplied.  The dot product
// over d is taken in a fixed order: within stage c, the half-wave hh of a lane supplies
// d = 32c + 16hh + s in step s, so one float4 read feeds four MFMAs.  kc * scale is
// rounded to fp32 before the product, as the reference computes it.
template <int D>
__global__ __launch_bounds__(256) void k3_scores(const float* __restrict__ qc,
                                                 const float* __restrict__ kc,
                                                 const float* __restrict__ hnorm,
                                                 const float* __restrict__ noise, float scale,
                                                 int use_cov_bias, float* __restrict__ scores, int NT,
                                                 int ntj, int tiles_per_slice, int ntiles) {
  constexpr int TI = 64;
  constexpr int NC = D / kScoreDC;              // stages per tile
  constexpr int A_BYTES = TI * 128;             // 64 query rows x 32 floats
  constexpr int B_BYTES = kScoreTJ * 128;       // 128 key rows x 32 floats
  constexpr int STAGE = A_BYTES + B_BYTES;      // 24 KB: 24 direct loads of 1 KB
  constexpr int LOADS = STAGE / 1024 / 4;       // per wave per stage
  static_assert(D % kScoreDC == 0 && STAGE % 4096 == 0, "stage split");
  __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * STAGE];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t slice_bytes = (uint32_t)NT * D * 4u;
  const uint32_t lds0 = lds_addr(lds);
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int ar = (wave >> 1) * 32 + l32;  // query row of the tile this lane supplies
  const int br0 = (wave & 1) * 64 + l32;  // key rows of its two sub-tiles: br0, br0 + 32

  // Direct load n of this wave fills 1 KB piece p = 4n + wave of a stage: pieces 0-7
  // hold query rows 8p .. 8p + 7, pieces 8-23 key rows 8(p - 8) .. ; lane L writes physical
  // chunk L & 7 of row 8p' + L/8, which holds logical chunk (L & 7) ^ ((row >> 1) & 7).
  uint32_t roff[LOADS];  // byte offset of the lane's chunk within its tile's row block
#pragma unroll
  for (int n = 0; n < LOADS; ++n) {
    const int p = 4 * n + wave;
    const int row = (p < TI / 8 ? p : p - TI / 8) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    roff[n] = (uint32_t)row * (uint32_t)(D * 4) + (uint32_t)(c * 16);
  }
  struct Tile {
    int bh, i0, j0;
  };
  auto tile_of = [&](int t) -> Tile {
    const int bh = t / tiles_per_slice;
    const int r = t - bh * tiles_per_slice;
    const int ti = r / ntj;
    return Tile{bh, ti * TI, (r - ti * ntj) * kScoreTJ};
  };
  auto load_stage = [&](const Tile& tl, int st, int buf) {
    const u32x4_t qd = make_rsrc_words(qc + (int64_t)tl.bh * NT * D, slice_bytes);
    const u32x4_t kd = make_rsrc_words(kc + (int64_t)tl.bh * NT * D, slice_bytes);
    const uint32_t qrow = (uint32_t)tl.i0 * (uint32_t)(D * 4) + (uint32_t)(st * kScoreDC * 4);
    const uint32_t krow = (uint32_t)tl.j0 * (uint32_t)(D * 4) + (uint32_t)(st * kScoreDC * 4);
    const uint32_t base = lds0 + buf * STAGE;
#pragma unroll
    for (int n = 0; n < LOADS; ++n) {
      const int p = 4 * n + wave;
      if (p < TI / 8)
        dma_load16_lds(qd, base + p * 1024, roff[n] + qrow, 0u);
      else
        dma_load16_lds(kd, base + p * 1024, roff[n] + krow, 0u);
    }
  };

  int t = blockIdx.x;
  if (t >= ntiles) return;
  Tile cur = tile_of(t);
  int buf = 0;
  load_stage(cur, 0, buf);
  while (true) {
    const int tn = t + (int)gridDim.x;
    const bool more = tn < ntiles;
    const Tile nxt = more ? tile_of(tn) : cur;
    f32x16_t acc0, acc1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      acc0[r] = 0.f;
      acc1[r] = 0.f;
    }
#pragma unroll
    for (int st = 0; st < NC; ++st) {
      // Prefetch the next stage (the next tile's first after this tile's last).
      const bool pre = st + 1 < NC || more;
      if (pre) {
        load_stage(st + 1 < NC ? cur : nxt, st + 1 < NC ? st + 1 : 0, buf ^ 1);
        wait_vmcnt<LOADS>();  // this wave's part of this stage landed (the next may be in flight)
      } else {
        wait_vmcnt<0>();
      }
      barrier_lds_reads_done();  // ... and every wave's
      const unsigned char* sa = lds + buf * STAGE;
      const unsigned char* sb = sa + A_BYTES;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const int c = hh * 4 + s4;  // logical chunk: features 16hh + 4s4 .. + 3 of the stage
        const float4 a = *reinterpret_cast<const float4*>(sa + score_chunk_byte(ar, c));
        float4 b0 = *reinterpret_cast<const float4*>(sb + score_chunk_byte(br0, c));
        float4 b1 = *reinterpret_cast<const float4*>(sb + score_chunk_byte(br0 + 32, c));
        b0 = make_float4(scale * b0.x, scale * b0.y, scale * b0.z, scale * b0.w);  // kc * scale first
        b1 = make_float4(scale * b1.x, scale * b1.y, scale * b1.z, scale * b1.w);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b0.x, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b1.x, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b0.y, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b1.y, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b0.z, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b1.z, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b0.w, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b1.w, acc1, 0, 0, 0);
      }
      barrier_lds_reads_done();  // every wave is done with this stage's buffer
      buf ^= 1;
    }
    // C: row (query block) 8(r>>2) + 4hh + (r&3) of a sub-tile, column (key block) l32.
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int gj = cur.j0 + br0 + 32 * s2;
      if (gj < NT) {
        float bias = 0.f;
        if (use_cov_bias) {
          bias = logf(hnorm[(int64_t)cur.bh * NT + gj] + 1e-6f);
          if (noise) bias = bias + noise[(int64_t)cur.bh * NT + gj];
        }
        const f32x16_t& acc = s2 ? acc1 : acc0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int gi = cur.i0 + (wave >> 1) * 32 + mfma32_row(r, hh);
          if (gi < NT) scores[((int64_t)cur.bh * NT + gi) * NT + gj] = acc[r] + bias;
        }
      }
    }
    if (!more) break;
    t = tn;
    cur = nxt;
  }
}

// Order-preserving map of fp32 scores to uint32 (-0.0 == +0.0).
__device__ __forceinline__ uint32_t score_ord(float s) {
  uint32_t bits = __float_as_uint(s);
  if ((bits & 0x7fffffffu) == 0) bits = 0;
  return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}

// The lanes for which c holds (as a wave-uniform mask).
__device__ __forceinline__ uint64_t ballot(bool c) { return __builtin_amdgcn_ballot_w64(c); }

// op(x) over the 64 lanes: DPP exchanges within rows of 16 (lane ^ 1, lane ^ 2, then the
// mirrors of 8 and 16 lanes), then one read per row.
template <class Op>
__device__ __forceinline__ uint32_t wave_reduce(uint32_t x, Op op) {
  x = op(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
  x = op(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xf, 0xf, false));   // quad_perm 2,3,0,1
  x = op(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xf, 0xf, false));  // row_half_mirror
  x = op(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x140, 0xf, 0xf, false));  // row_mirror
  return op(op((uint32_t)__builtin_amdgcn_readlane((int)x, 0), (uint32_t)__builtin_amdgcn_readlane((int)x, 16)),
            op((uint32_t)__builtin_amdgcn_readlane((int)x, 32), (uint32_t)__builtin_amdgcn_readlane((int)x, 48)));
}
__device__ __forceinline__ uint32_t wave_total(uint32_t x) {
  return wave_reduce(x, [](uint32_t a, uint32_t b) { return a + b; });
}

// Number of the S register slots' values, over the whole wavefront, that are >= t.  The
// first V slots are counted per lane in the VALU and summed across lanes once; the rest
// by a ballot and a scalar popcount each, so that both pipes share the work.
template <int S, int V>
__device__ __forceinline__ uint32_t count_ge(const uint32_t (&v)[S], uint32_t t) {
  uint32_t n = 0u;
  if constexpr (V > 0) {
    uint32_t c = 0u;
#pragma unroll
    for (int i = 0; i < V; ++i) c += v[i] >= t ? 1u : 0u;
    n = wave_total(c);
  }
#pragma unroll
  for (int i = V; i < S; ++i) n += (uint32_t)__popcll(ballot(v[i] >= t));
  return n;
}

// Lanes below this one whose bit is set in m.
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Blocks 64 i .. 64 i + 63 are mask words 2 i (lanes 0-31 of pbs[i]) and 2 i + 1; word w
// goes to lane w % 64 of mw[w / 64].  Each lane selects its words with compares (the
// compiler schedules these; an inline-asm v_writelane right after the VALU write of its
// register wrote a stale word 0 when nothing else separated them).
template <int KPL>
__device__ __forceinline__ void set_mask_words(const uint64_t (&pbs)[KPL], int lane, uint32_t (&mw)[2]) {
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int w0 = 2 * i;
    const uint32_t lo = (uint32_t)pbs[i];
    const uint32_t hi = (uint32_t)(pbs[i] >> 32);
    if (lane == (w0 & 63)) mw[w0 >> 6] = lo;
    if (lane == ((w0 + 1) & 63)) mw[(w0 + 1) >> 6] = hi;
  }
}

// The 64-bit value of lane ^ m.
__device__ __forceinline__ uint64_t key_xor(uint64_t k, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)k, m, 64);
  const uint32_t hi = __shfl_xor((uint32_t)(k >> 32), m, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Bitonic sort, descending, of the 64 R keys of a wavefront held in registers: element
// e = R * lane + s is key[s] of that lane.  Pairs closer than R are exchanged within a
// lane, the others across lanes (lane distance jj / R).  Keys are distinct except the
// zero padding.
template <int R>
__device__ __forceinline__ void wave_sort_desc(uint64_t (&key)[R], int lane) {
  constexpr int N = 64 * R;
#pragma unroll
  for (int kk = 2; kk <= N; kk <<= 1) {
#pragma unroll
    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
      if (jj < R) {
#pragma unroll
        for (int s = 0; s < R; ++s) {
          if (s & jj) continue;
          const bool desc = ((R * lane + s) & kk) == 0;
          const uint64_t a = key[s], b = key[s + jj];
          const bool swap = desc ? (a < b) : (a > b);
          key[s] = swap ? b : a;
          key[s + jj] = swap ? a : b;
        }
      } else {
#pragma unroll
        for (int s = 0; s < R; ++s) {
          const int e = R * lane + s;
          const uint64_t p = key_xor(key[s], jj / R);
          const bool keep_max = ((e & jj) == 0) == ((e & kk) == 0);
          key[s] = (keep_max == (key[s] > p)) ? key[s] : p;
        }
      }
    }
  }
}

// Bitonic sort, descending, of sel[0, NSP) in LDS (NSP a power of two).
__device__ __forceinline__ void lds_sort_desc(uint64_t* sel, int NSP, int lane) {
  for (int kk = 2; kk <= NSP; kk <<= 1) {
    for (int jj = kk >> 1; jj > 0; jj >>= 1) {
      for (int p = lane; p < (NSP >> 1); p += 64) {
        const int i = ((p & ~(jj - 1)) << 1) | (p & (jj - 1));
        const int l = i + jj;
        const uint64_t a = sel[i];
        const uint64_t b = sel[l];
        const bool desc = (i & kk) == 0;
        const bool swap = desc ? (a < b) : (a > b);
        sel[i] = swap ? b : a;
        sel[l] = swap ? a : b;
      }
      __syncthreads();
    }
  }
}

// Sorts the NS keys in sel[0, NS) (descending) and writes their indices to irow.
template <int R>
__device__ __forceinline__ void sort_and_store(const uint64_t* sel, int NS, int lane, int32_t* irow) {
  uint64_t key[R];
#pragma unroll
  for (int s = 0; s < R; ++s) key[s] = R * lane + s < NS ? sel[R * lane + s] : 0ull;
  wave_sort_desc<R>(key, lane);
#pragma unroll
  for (int s = 0; s < R; ++s)
    if (R * lane + s < NS) irow[R * lane + s] = (int)(0xffffffffu - (uint32_t)key[s]);
}

// The picks of a row: every score above T and, when RANK, of the scores equal to T the
// `need` with the lowest indices (without RANK every tie is taken).  With KEYS, the picked
// keys go to sel in index order (a lane that does not pick writes its own slot past NSP
// instead, so the store needs no branch); mw receives the selection mask, word w in lane
// w % 64 of mw[w / 64].
template <int KPL, bool RANK, bool KEYS>
__device__ __forceinline__ void pick_row(const uint32_t (&ok)[KPL], uint32_t T, uint32_t need, int NSP,
                                         int lane, uint64_t* sel, uint32_t (&mw)[2]) {
  uint32_t taken = 0u;  // ties at T taken so far (in index order)
  uint32_t base = 0u;   // picks so far (in index order)
  uint64_t pbs[KPL];    // ballots of the picks
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    bool pick;
    if constexpr (RANK) {
      const bool tie = ok[i] == T;
      const uint64_t tb = ballot(tie);
      pick = ok[i] > T || (tie && taken + lanes_below(tb) < need);
      taken += (uint32_t)__popcll(tb);
    } else {
      pick = ok[i] >= T;  // T >= 1, so a missing key (0) is never picked
    }
    const uint64_t pb = ballot(pick);
    if constexpr (KEYS) {
      const uint32_t pos = pick ? base + lanes_below(pb) : (uint32_t)(NSP + lane);
      sel[pos] = ((uint64_t)ok[i] << 32) | (uint64_t)(0xffffffffu - (uint32_t)(i * 64 + lane));
      base += (uint32_t)__popcll(pb);
    }
    pbs[i] = pb;
  }
  set_mask_words<KPL>(pbs, lane, mw);
}

// Slots counted in the VALU per search step (the rest by ballots).
template <int KPL>
constexpr int kValuSlots = KPL / 3;

// One wavefront per row.  The row's ordered scores stay in registers (KPL per lane,
// index j = 64 i + lane).  The NS-th largest ordered score T is found bit by bit from
// the top: the search keeps the bucket [prefix, prefix + 2^w) that holds T, with
// hi = #{scores >= prefix + 2^w} and lo = #{scores >= prefix}; a step halves the
// bucket by counting the scores >= its midpoint.  Once the bucket holds at most 64
// scores they are compacted into one register, and the remaining bits are searched over
// that register alone.  Every score above T is selected, and of the scores equal to T
// the lowest indices (ties go to the lowest index).  The selection bitmask is the ballot
// of the picks (two 32-block words per register); the NS picked keys
// (score << 32 | ~index) are packed into LDS in index order and sorted descending in
// registers (NS <= 256) or in LDS.  Dynamic LDS: (NSP + 64) * 8 bytes (NSP = pow2 >= NS).
// Without IDX only the bitmask is written (what K4 reads): no keys, no sort.
template <int KPL, bool IDX>
__global__ __launch_bounds__(64) void k3_topk(const float* __restrict__ scores, int NT, int NS, int NSP,
                                              int NW, int32_t* __restrict__ idx,
                                              uint32_t* __restrict__ selmask) {
  static_assert(KPL <= 64, "a row spans at most two 64-word mask registers");
  extern __shared__ uint64_t sel[];
  __shared__ uint32_t bucket[128];  // the compacted bucket, then one spill slot per lane
  const int row = blockIdx.x;
  const int bh = blockIdx.y;
  const int lane = threadIdx.x;
  const float* srow = scores + ((int64_t)bh * NT + row) * NT;

  // Missing keys (j >= NT) read as 0, below every ordered score (score_ord sets the
  // top bit of non-negative scores and maps negative ones to ~bits, which is > 0 for
  // every finite or infinite score; NaN scores do not occur).  The load index is
  // clamped so that the loads need no branch.
  uint32_t ok[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    const int j = i * 64 + lane;
    const uint32_t o = score_ord(srow[min(j, NT - 1)]);
    ok[i] = j < NT ? o : 0u;
  }

  // T = the largest t with #{j : ok_j >= t} >= NS.  Every midpoint tested is > 0, so
  // the missing keys are never counted.  The search starts from the bits that the row's
  // smallest and largest scores share: every score lies in that bucket.
  uint32_t mx = 0u, mn1 = 0xffffffffu;  // max ok, min (ok - 1) (a missing key gives 2^32 - 1)
#pragma unroll
  for (int i = 0; i < KPL; ++i) {
    mx = max(mx, ok[i]);
    mn1 = min(mn1, ok[i] - 1u);
  }
  mx = wave_reduce(mx, [](uint32_t a, uint32_t b) { return max(a, b); });
  const uint32_t mn = wave_reduce(mn1, [](uint32_t a, uint32_t b) { return min(a, b); }) + 1u;
  int w = mn == mx ? 0 : 32 - __builtin_clz(mn ^ mx);  // bits below the shared prefix
  uint32_t prefix = w == 32 ? 0u : mn & ~((1u << w) - 1u);
  uint32_t hi = 0u, lo = (uint32_t)NT;
  while (w > 0 && lo - hi > 64u) {
    --w;
    const uint32_t mid = prefix | (1u << w);
    const uint32_t n = count_ge<KPL, kValuSlots<KPL>>(ok, mid);
    if (n >= (uint32_t)NS) {
      prefix = mid;
      lo = n;
    } else {
      hi = n;
    }
  }
  if (w > 0) {
    // The lo - hi <= 64 scores in [prefix, prefix + 2^w): into one register.  A score
    // below prefix wraps to ok - prefix >= 2^32 - prefix >= 2^w (prefix + 2^w <= 2^32).
    // Lanes whose score is outside write their own spill slot, so the store needs no
    // branch.
    const uint32_t span = w == 32 ? 0xffffffffu : (1u << w) - 1u;
    uint32_t base = 0u;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const bool in = (ok[i] - prefix <= span) & (ok[i] != 0u);
      const uint64_t m = ballot(in);
      const uint32_t r = base + lanes_below(m);
      bucket[in ? r : 64u + lane] = ok[i];
      base += (uint32_t)__popcll(m);
    }
    __syncthreads();
    uint32_t c[1] = {(uint32_t)lane < lo - hi ? bucket[lane] : 0u};
    const uint32_t above = hi;  // scores above the compacted bucket
    while (w > 0) {
      --w;
      const uint32_t mid = prefix | (1u << w);
      const uint32_t n = above + count_ge<1, 0>(c, mid);
      if (n >= (uint32_t)NS) {
        prefix = mid;
        lo = n;
      } else {
        hi = n;
      }
    }
  }
  // prefix = T; hi = #{scores > T}, lo = #{scores >= T}.  Every score above T is
  // selected and, of the lo - hi scores equal to T, the need = NS - hi with the lowest
  // indices (all of them when lo - hi == need, the usual case).
  const uint32_t need = (uint32_t)NS - hi;
  uint32_t mw[2] = {0u, 0u};
  if (lo - hi == need)
    pick_row<KPL, false, IDX>(ok, prefix, need, NSP, lane, sel, mw);
  else
    pick_row<KPL, true, IDX>(ok, prefix, need, NSP, lane, sel, mw);
  uint32_t* mrow = selmask + ((int64_t)bh * NT + row) * NW;
  if (lane < NW) mrow[lane] = mw[0];
  if (64 + lane < NW) mrow[64 + lane] = mw[1];
  if constexpr (!IDX) return;
  __syncthreads();

  int32_t* irow = idx + ((int64_t)bh * NT + row) * NS;
  if (NS <= 64) {
    sort_and_store<1>(sel, NS, lane, irow);
  } else if (NS <= 128) {
    sort_and_store<2>(sel, NS, lane, irow);
  } else if (NS <= 256) {
    sort_and_store<4>(sel, NS, lane, irow);
  } else {
    for (int i = NS + lane; i < NSP; i += 64) sel[i] = 0ull;
    __syncthreads();
    lds_sort_desc(sel, NSP, lane);
    for (int i = lane; i < NS; i += 64) irow[i] = (int)(0xffffffffu - (uint32_t)(sel[i] & 0xffffffffull));
  }
}

hipError_t launch_scores(const float* qc, const float* kc, const float* hnorm, const float* noise,
                         float scale, int use_cov_bias, float* scores, int bh, int NT, int D,
                         hipStream_t stream) {
  const int nti = (NT + 63) / 64;
  const int ntj = (NT + kScoreTJ - 1) / kScoreTJ;
  const int ntiles = bh * nti * ntj;
  // Three workgroups per CU of the MI355X (256 CUs); each loops over its tiles, so any
  // grid size is correct.
  constexpr int kResident = 3 * 256;
  const int grid = ntiles < kResident ? ntiles : kResident;
  if (D == 128)
    hipLaunchKernelGGL((k3_scores<128>), dim3(grid), dim3(256), 0, stream, qc, kc, hnorm, noise, scale, use_cov_bias,
                       scores, NT, ntj, nti * ntj, ntiles);
  else if (D == 64)
    hipLaunchKernelGGL((k3_scores<64>), dim3(grid), dim3(256), 0, stream, qc, kc, hnorm, noise, scale, use_cov_bias,
                       scores, NT, ntj, nti * ntj, ntiles);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// Rows longer than k3_topk holds in registers (NT > 4096): one workgroup of 256 threads per
// row, the row read from memory (L2) in index order.  The NS-th largest ordered score T is
// found by a radix select, 8 bits per pass from the top, with a 256-bin histogram in LDS of
// the scores in the current bucket (integer counts: the order of the LDS atomic adds does
// not matter).  Every score above T is selected and, of those equal to T, the lowest
// indices, ranked by a workgroup prefix count of the ties in index order.  With IDX the
// picked keys (score << 32 | ~index) are packed into LDS in index order and sorted
// descending (bitonic, NSP = pow2 >= NS <= 8192: 64 KB of dynamic LDS).
template <bool IDX>
__global__ __launch_bounds__(256) void k3_topk_large(const float* __restrict__ scores, int NT, int NS, int NSP,
                                                     int NW, int32_t* __restrict__ idx,
                                                     uint32_t* __restrict__ selmask) {
  extern __shared__ uint64_t sel[];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wcount[4];
  __shared__ uint32_t s_bin, s_above;
  const int row = blockIdx.x;
  const int bh = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const float* srow = scores + ((int64_t)bh * NT + row) * NT;
  uint32_t prefix = 0u, fixed = 0u, above = 0u;  // bucket bits so far; #scores above the bucket
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[tid] = 0u;
    __syncthreads();
    for (int j = tid; j < NT; j += 256) {
      const uint32_t o = score_ord(srow[j]);
      if ((o & fixed) == prefix) atomicAdd(&hist[(o >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t cum = above;
      int b = 255;
      for (; b > 0; --b) {
        if (cum + hist[b] >= (uint32_t)NS) break;
        cum += hist[b];
      }
      s_bin = (uint32_t)b;
      s_above = cum;
    }
    __syncthreads();
    prefix |= s_bin << shift;
    fixed |= 255u << shift;
    above = s_above;
  }
  // prefix = T; above = #{scores > T}; the NS - above lowest-index scores equal to T are taken.
  const uint32_t need = (uint32_t)NS - above;
  uint32_t* mrow = selmask + ((int64_t)bh * NT + row) * NW;
  uint32_t ties = 0u, picks = 0u;  // ties and picks in earlier chunks
  for (int j0 = 0; j0 < NT; j0 += 256) {
    const int j = j0 + tid;
    const uint32_t o = j < NT ? score_ord(srow[j]) : 0u;
    const bool tie = j < NT && o == prefix;
    const uint64_t tb = ballot(tie);
    if (lane == 0) wcount[wave] = (uint32_t)__popcll(tb);
    __syncthreads();
    uint32_t below = 0u, total = 0u;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      below += w < wave ? wcount[w] : 0u;
      total += wcount[w];
    }
    const bool pick = j < NT && (o > prefix || (tie && ties + below + lanes_below(tb) < need));
    ties += total;
    const uint64_t pb = ballot(pick);
    if (lane == 0) {
      const int w0 = (j0 + 64 * wave) >> 5;
      if (w0 < NW) mrow[w0] = (uint32_t)pb;
      if (w0 + 1 < NW) mrow[w0 + 1] = (uint32_t)(pb >> 32);
    }
    __syncthreads();  // wcount is rewritten below / in the next chunk
    if constexpr (IDX) {
      if (lane == 0) wcount[wave] = (uint32_t)__popcll(pb);
      __syncthreads();
      uint32_t pbelow = 0u, ptotal = 0u;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        pbelow += w < wave ? wcount[w] : 0u;
        ptotal += wcount[w];
      }
      if (pick) sel[picks + pbelow + lanes_below(pb)] = ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - (uint32_t)j);
      picks += ptotal;
      __syncthreads();
    }
  }
  if constexpr (IDX) {
    for (int i = NS + tid; i < NSP; i += 256) sel[i] = 0ull;
    __syncthreads();
    for (int kk = 2; kk <= NSP; kk <<= 1) {
      for (int jj = kk >> 1; jj > 0; jj >>= 1) {
        for (int p = tid; p < (NSP >> 1); p += 256) {
          const int i = ((p & ~(jj - 1)) << 1) | (p & (jj - 1));
          const int l = i + jj;
          const uint64_t a = sel[i];
          const uint64_t b = sel[l];
          const bool desc = (i & kk) == 0;
          const bool swap = desc ? (a < b) : (a > b);
          sel[i] = swap ? b : a;
          sel[l] = swap ? a : b;
        }
        __syncthreads();
      }
    }
    int32_t* irow = idx + ((int64_t)bh * NT + row) * NS;
    for (int i = tid; i < NS; i += 256) irow[i] = (int)(0xffffffffu - (uint32_t)(sel[i] & 0xffffffffull));
  }
}

hipError_t launch_topk(const float* scores, int bh, int NT, int NS, int32_t* idx,
                       uint32_t* selmask, hipStream_t stream) {
  int NSP = 1;
  while (NSP < NS) NSP <<= 1;
  if (NSP < 2) NSP = 2;
  const int NW = (NT + 31) / 32;
  dim3 grid(NT, bh);
  if (NT > 4096) {
    if (idx && NSP > kMaxLargeSortKeys) return hipErrorInvalidValue;
    if (idx)
      hipLaunchKernelGGL((k3_topk_large<true>), grid, dim3(256), (size_t)NSP * sizeof(uint64_t), stream, scores, NT,
                         NS, NSP, NW, idx, selmask);
    else
      hipLaunchKernelGGL((k3_topk_large<false>), grid, dim3(256), 0, stream, scores, NT, NS, NSP, NW, idx, selmask);
    return hipGetLastError();
  }
  const size_t lds = idx ? (size_t)(NSP + 64) * sizeof(uint64_t) : 0;
#define PASA_TOPK(K)                                                                                         \
  case K:                                                                                                    \
    if (idx)                                                                                                 \
      hipLaunchKernelGGL((k3_topk<K, true>), grid, dim3(64), lds, stream, scores, NT, NS, NSP, NW, idx, selmask); \
    else                                                                                                     \
      hipLaunchKernelGGL((k3_topk<K, false>), grid, dim3(64), lds, stream, scores, NT, NS, NSP, NW, idx, selmask); \
    break;
  // Registers per lane: ceil(NT / 64) rounded up to a multiple of 4.
  switch (4 * ((NT + 255) / 256)) {
    PASA_TOPK(4) PASA_TOPK(8) PASA_TOPK(12) PASA_TOPK(16) PASA_TOPK(20) PASA_TOPK(24) PASA_TOPK(28)
    PASA_TOPK(32) PASA_TOPK(36) PASA_TOPK(40) PASA_TOPK(44) PASA_TOPK(48) PASA_TOPK(52) PASA_TOPK(56)
    PASA_TOPK(60) PASA_TOPK(64)
    default:
      return hipErrorInvalidValue;
  }
#undef PASA_TOPK
  return hipGetLastError();
}

}  // namespace pasa
