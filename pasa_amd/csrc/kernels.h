// Internal launcher declarations (host side).  Shapes are validated by capi.hip
// before any of these is called.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "common.h"

namespace pasa {

constexpr int kMaxSelectBlocks = 1 << 16;  // NT limit of the selection (k3_topk: NT <= 4096 in
                                            // registers; k3_topk_large beyond)
constexpr int kMaxLargeSortKeys = 8192;    // index list of k3_topk_large: NS <= 8192 (LDS sort)

hipError_t launch_permute(const void* s0, const void* s1, const void* s2, void* d0, void* d1,
                          void* d2, int ntens, int bh, int S, int F, int P, int ctx, int row_bytes,
                          const int32_t* head_is_temporal, int inverse, hipStream_t stream);

// T: rows of the blocked segment; Tslice: rows per slice (T plus any text rows).
// rm: nullptr, or the token-major view of frame-major slices (D = 128, BT = 128).
// split > 1: each group's blocks go to `split` workgroups, whose raw partial sums
// (partials: [bh, NG, split, D, D] fp32) a second kernel reduces in order into hgroup.
// rm: frame-major q, k, v (token-major view); tm_copies[3] then receive that view of q, k, v.
hipError_t launch_block_stats(const void* q, const void* k, const void* v, float* qc, float* kc,
                              float* vc, float* hnorm, float* hgroup, int bh, int T, int Tslice, int D,
                              int BT, int G, const RowMap* rm, void* const* tm_copies, float* partials, int split,
                              bool f16, hipStream_t stream);
int block_stats_split(int bh, int T, int D, int BT, int G);  // the split the launcher is given by the C ABI

hipError_t launch_scores(const float* qc, const float* kc, const float* hnorm, const float* noise,
                         float scale, int use_cov_bias, float* scores, int bh, int NT, int D,
                         hipStream_t stream);

hipError_t launch_topk(const float* scores, int bh, int NT, int NS, int32_t* idx,
                       uint32_t* selmask, hipStream_t stream);

size_t k4_pack_bytes(int D, int BT);  // per (slice, group) phase-2 pack image

// f16: the pack (and, below, q, k, v, o) hold fp16 instead of bf16 (D = 128 only).
hipError_t launch_pack_phase2(const float* kc, const float* vc, const float* hgroup, void* pack,
                              int bh, int T, int D, int BT, bool f16, hipStream_t stream);

// T: rows of the blocked (video) segment; text: rows of the text segment that
// follows it in each slice (slices are T + text rows apart), the first text_valid of
// them the prompt and the rest padding.
hipError_t launch_sparse_attn(const void* q, const void* k, const void* v, const void* pack,
                              const int32_t* idx, const uint32_t* selmask, void* o, float scale,
                              int bh, int T, int text, int text_valid, int D, int BT, int NS,
                              int gamma_literal, const RowMap* rm, bool f16, hipStream_t stream);

// Dense softmax attention with K4's phase-1 machinery (every key block exact, no
// selection, no correction), D = 128.  T video rows, then `text` rows of which the
// first text_valid are the prompt: rows attend within [0, T + text_valid) or within
// the padding [T + text_valid, T + text).
hipError_t launch_dense_attn(const void* q, const void* k, const void* v, void* o, float scale, int bh,
                             int T, int text, int text_valid, bool f16, hipStream_t stream);

// ---- any-shape path (any_shape.hip) ----------------------------------------------
// fp32, bf16 or fp16 q, k, v (dtype: kAnyBf16 / kAnyF16 / kAnyF32, the pasa_dtype_t
// values); head dim 1 .. 128; any block size and group size.  Outputs as the tuned
// kernels' (fp32 statistics; o in the input type).
constexpr int kAnyBf16 = 0;
constexpr int kAnyF16 = 1;
constexpr int kAnyF32 = 2;
hipError_t launch_block_stats_any(const void* q, const void* k, const void* v, float* qc, float* kc, float* vc,
                                  float* hnorm, float* hgroup, int bh, int T, int Tslice, int D, int BT, int G,
                                  int dtype, hipStream_t stream);
hipError_t launch_scores_any(const float* qc, const float* kc, const float* hnorm, const float* noise, float scale,
                             int use_cov_bias, float* scores, int bh, int NT, int D, hipStream_t stream);
// all: dense (every key block exact, no correction; kc, vc, hgroup, selmask unused).
hipError_t launch_sparse_attn_any(const void* q, const void* k, const void* v, const float* kc, const float* vc,
                                  const float* hgroup, const uint32_t* selmask, void* o, float scale, int bh, int T,
                                  int text, int text_valid, int D, int BT, int G, int gamma_literal, int all,
                                  int dtype, hipStream_t stream);
int64_t sparse_attn_any_tiles(int T, int text, int text_valid, int BT);  // grid.x of launch_sparse_attn_any

// ---- K5: processor prologue (RMSNorm + rotary embedding + head-major layout) ----
constexpr int kNormHead = 1;       // RMSNorm over each head's D channels, weight [D]
constexpr int kNormRow = 2;        // RMSNorm over the token's H*D channels, weight [H*D]
constexpr int kRopeCosSinF32 = 1;  // cos, sin: fp32 [rope_rows, D]
constexpr int kRopeComplexF64 = 2; // cos = real, sin = imaginary part: fp64 [rope_rows, D/2]

struct PrologueTensor {
  const uint16_t* in;      // bf16; nullptr: tensor skipped
  uint16_t* out;           // bf16
  const uint16_t* weight;  // bf16 RMSNorm weight; nullptr: no norm for this tensor
};

struct PrologueParams {
  PrologueTensor t[3];      // q, k (normalised and rotated), v (layout only)
  const void* cos;
  const void* sin;
  int64_t B, S, H;          // batch, rows per (b, h) slice read, heads
  int64_t OS, row0;         // output rows per slice and first output row
  int64_t rope_rows;        // rows [0, rope_rows) are rotated
  int D;
  int in_bshd, out_bshd;    // 1: [B, S, H, D]; 0: [B, H, S, D]
  int norm;                 // 0, kNormHead or kNormRow
  int round_twice;          // 1: diffusers RMSNorm rounding; 0: one rounding
  int rope;                 // 0, kRopeCosSinF32 or kRopeComplexF64
  float eps;
};

int prologue_max_chunks();  // H * D / 8 limit
hipError_t launch_prologue(const PrologueParams& p, hipStream_t stream);

// ---- K6: DiT block row operations (modulate.hip) ------------------------------------
struct RowOpParams {
  const void* x;              // [M, N] input, bf16 or fp32 (x_f32)
  const void* r;              // stage A residual [M, N] (bf16 or fp32: r_f32), or null (no stage A)
  const float* gate;          // stage A gate, fp32 rows of N per batch, or null (plain add)
  void* h;                    // stage A output [M, N] (bf16 or fp32: h_f32), or null
  const void* w;              // stage B affine weight [N] (bf16 or fp32: wb_f32), or null
  const void* b;              // stage B affine bias [N], or null
  const float* scale;         // stage B modulation, fp32 rows of N per batch, or null
  const float* shift;         // with scale
  void* y;                    // stage B output [M, N] (bf16 or fp32: y_f32), or null (no stage B)
  int64_t M;
  int64_t rows_per_batch;     // rows sharing one gate/scale/shift row
  int64_t param_stride;       // elements between the gate/scale/shift rows of successive batches
  int N;                      // multiple of 8, <= row_ops_max_cols()
  int x_f32, r_f32, h_f32, wb_f32, y_f32;
  int ln;                     // LayerNorm in stage B
  float eps;
};

int row_ops_max_cols();
hipError_t launch_row_ops(const RowOpParams& p, hipStream_t stream);

}  // namespace pasa
