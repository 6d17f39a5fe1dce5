/*
 * pasa.h — C ABI of the MI355X (gfx950) PISA-PG sparse-attention hot path.
 *
 * Every entry point is extern "C", takes plain device pointers, sizes and a
 * hipStream_t passed as void*, and returns an int status (0 = OK, negative =
 * error, see pasa_status_t).  The library never allocates device memory: the
 * caller passes every buffer, including workspace (pasa_sparse_attn_noalloc alone
 * uses a static device array instead, sized at load).  All shape / dtype / size
 * checks run on the host before any HIP call, so every error path is reachable
 * without a GPU.  No entry point synchronises; work is enqueued on `stream`.
 * No atomics on global memory: identical inputs give bitwise-identical outputs.
 *
 * Tensor layout: q, k, v, o are [B, H, T, D] contiguous, passed as BH = B*H
 * slices of [T, D].  Reference interface cited per entry point; paths are
 * relative to the reference tree (ZHANGWENTAI/PASA).
 *
 * Shapes.  The tuned gfx950 kernels take bf16 q, k, v (fp16 at head_dim 128), head_dim
 * 64 or 128, block_size 64 or 128 and (attention) group_size 32.  pasa_block_stats,
 * pasa_select, pasa_sparse_attn, pasa_sparse_attn_noalloc and pasa_dense_attn also take
 * every other shape the reference does (group_pisa_attention.py:307-398: any float dtype,
 * any group size, any power-of-two block size): fp32, bf16 or fp16 inputs, head_dim
 * 1 .. 128, block_size a power of two in [16, 256], group_size 1 .. 2^20, on the
 * any-shape kernels (the same mathematics in plain VALU arithmetic, for completeness
 * rather than speed).  The pack / packed / placed entry points take the tuned shapes only.
 *
 * Text segment (text_len > 0; head_dim 128 on the tuned kernels): the last text_len rows of each
 * slice are text tokens (HunyuanVideo appends its text last).  Blocks, statistics,
 * selection and the first-order correction cover the first T - text_len rows; every
 * video query block also attends to all text keys exactly, and text query rows
 * attend densely to all T keys.  text_len = 0 is the reference's behaviour (PISA
 * over all rows as ordinary tokens; group_pisa_attention.py:317, 330-333 document
 * prompt_token_length but do not use it).
 * Text padding (pasa_sparse_attn*'s text_valid, 0 <= text_valid <= text_len): only
 * the first text_valid text rows are the prompt, the rest padding.  As in the
 * reference's dense HunyuanVideo path (cu_seqlens [0, valid, T],
 * svg/models/hyvideo/attention.py:314-322), the sequence splits into two segments
 * that attend only within themselves: video rows and prompt rows see the video
 * rows and the prompt keys, padding rows see the padding keys.  text_valid =
 * text_len means no padding.
 */
#ifndef PASA_H_
#define PASA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PASA_ABI_VERSION 11

typedef enum {
  PASA_OK = 0,
  PASA_ERR_NULL_POINTER = -1,   /* a required pointer is NULL                     */
  PASA_ERR_BAD_SHAPE = -2,      /* a size is <= 0, or sizes are inconsistent      */
  PASA_ERR_HEAD_DIM = -3,       /* head_dim not taken by this entry point         */
  PASA_ERR_BLOCK_SIZE = -4,     /* block_size not taken by this entry point       */
  PASA_ERR_NUM_SELECTED = -5,   /* ns outside [1, NT]                             */
  PASA_ERR_OVERFLOW = -6,       /* an element count overflows the index type     */
  PASA_ERR_DTYPE = -7,          /* dtype not supported by this entry point        */
  PASA_ERR_WORKSPACE = -8,      /* workspace NULL or smaller than required        */
  PASA_ERR_BAD_ARG = -9,        /* scale / density not finite, scale <= 0, ...    */
  PASA_ERR_TEXT_SEGMENT = -10,  /* text segment does not fit the sequence         */
  PASA_ERR_LAUNCH = -11,        /* a kernel launch failed (hipGetLastError)       */
  PASA_ERR_GROUP_SIZE = -12,    /* group_size not taken by this entry point       */
  PASA_ERR_TOO_MANY_BLOCKS = -13 /* NT above 65536, or an index list > 8192 at NT > 4096 */
} pasa_status_t;

typedef enum {
  PASA_DTYPE_BF16 = 0,
  PASA_DTYPE_F16 = 1,
  PASA_DTYPE_F32 = 2
} pasa_dtype_t;

/* ---- library / error API ------------------------------------------------ */

/* ABI version of the loaded library (PASA_ABI_VERSION). */
int pasa_abi_version(void);

/* Static text for a status code. */
const char* pasa_status_string(int status);

/* Thread-local text of the last error raised on the calling thread ("" if none). */
const char* pasa_last_error(void);

/* NS = min(max(1, int(density * NT)), NT), the reference's top-k count computed
 * in double precision with truncation toward zero.
 * Replaces: svg/kernels/triton/group_pisa_attention.py:373.
 * Returns NS (>= 1) or a negative status for a non-finite density / NT <= 0. */
int64_t pasa_num_selected(double density, int64_t num_blocks);

/* ---- K1: frame-major <-> token-major layout permutation -------------------
 * Forward (inverse = 0), frame-major -> token-major, for sequence row r < S - ctx:
 *     dst[p*F + f] = src[f*P + p]      (F = num_frame, P = frame_size)
 * Inverse (inverse = 1), token-major -> frame-major:
 *     dst[f*P + p] = src[p*F + f]
 * The last `context_length` rows are copied unchanged.  S = ctx + F*P.
 * Up to three tensors (Q, K, V) are permuted in one launch; unused src/dst
 * pointers must be NULL.  head_is_temporal: optional int32 [BH]; a slice whose
 * flag is 0 is copied unchanged (the reference's "spatial" heads); NULL = all
 * slices permuted.  dtype selects the element size (2 or 4 bytes); head_dim *
 * element size must be a multiple of 16 bytes.  src and dst must not overlap.
 * Replaces: svg/models/hyvideo/placement.py:6-31 (closed forms),
 *   hunyuan_sparse_head_placement :124-153 (kernel :34-121, forward, 3 tensors),
 *   hunyuan_hidden_states_placement :360-387 (kernel :285-357, inverse, 1 tensor). */
int pasa_permute(const void* src0, const void* src1, const void* src2,
                 void* dst0, void* dst1, void* dst2, int n_tensors,
                 int64_t bh, int64_t num_frame, int64_t frame_size,
                 int64_t context_length, int64_t head_dim, int dtype,
                 const int32_t* head_is_temporal, int inverse, void* stream);

/* ---- K2: block statistics + per-group first-order moment ------------------
 * For every slice and key block j of the first Tv = T - text_len rows
 * (NT = ceil(Tv / block_size), n_j its length):
 *   qc[j] = mean_t q_t,  kc[j] = mean_t k_t,  vc[j] = sum_t v_t     (fp32 [BH,NT,D])
 *   hnorm[j] = || sum_t (k_t - kc[j]) v_t^T ||_F                        (fp32 [BH,NT])
 *   hgroup[g] = (1/G) * sum_{j in group g, j < NT} H_j                 (fp32 [BH,NG,D,D])
 * with NG = ceil(NT / G).  H_j is never materialised in memory.
 * dtype: PASA_DTYPE_BF16, PASA_DTYPE_F16 or PASA_DTYPE_F32 (q, k, v; the statistics
 * are fp32 either way); shapes as described at the top.
 * Replaces: fused_chunk_reduce group_pisa_attention.py:268-288 (kernel :66-129,
 *   sqrt at :287) and compute_h_group :291-301. */
int pasa_block_stats(const void* q, const void* k, const void* v,
                     float* qc, float* kc, float* vc, float* hnorm, float* hgroup,
                     int64_t bh, int64_t seq_len, int64_t text_len, int64_t head_dim,
                     int64_t block_size, int64_t group_size, int dtype, void* stream);

/* pasa_block_stats with a workspace that lets small grids split each group's blocks
 * over several workgroups (when BH * NG is small next to the CU count): their partial
 * sums land in the workspace and a second kernel adds them in a fixed order, so the
 * result is deterministic (and differs from the unsplit one only in the order of the
 * group sum).  workspace == NULL: the unsplit kernel; else workspace_bytes must be >=
 * pasa_block_stats_workspace_bytes(...) (0 when no split would be used) and the
 * workspace 16-byte aligned.
 * Replaces: the same reference functions as pasa_block_stats. */
int pasa_block_stats_ws(const void* q, const void* k, const void* v,
                        float* qc, float* kc, float* vc, float* hnorm, float* hgroup,
                        int64_t bh, int64_t seq_len, int64_t text_len, int64_t head_dim,
                        int64_t block_size, int64_t group_size, int dtype,
                        void* workspace, size_t workspace_bytes, void* stream);

size_t pasa_block_stats_workspace_bytes(int64_t bh, int64_t seq_len, int64_t text_len,
                                        int64_t head_dim, int64_t block_size, int64_t group_size);

/* ---- K3: block scores + deterministic top-k -------------------------------
 * scores[I][j] = sum_d qc[I][d] * (scale * kc[j][d])
 *              + (use_cov_bias ? log(hnorm[j] + 1e-6) + (noise ? noise[j] : 0) : 0)
 * idx[I][0..NS) = the NS largest scores of row I, ordered by (score desc, index asc);
 * ties are broken by lowest index; -0.0 and +0.0 compare equal.  idx may be NULL: then
 * only selmask is written (all pasa_sparse_attn reads), and the sort is skipped.
 * selmask[I][w] bit b set  <=>  key block 32*w + b is among the NS selected   (uint32 [BH,NT,ceil(NT/32)])
 * NS = pasa_num_selected(density, NT).  noise: optional fp32 [BH, NT] (one draw per
 * key block, shared by all query blocks; used only with use_cov_bias).  scores_out:
 * optional fp32 [BH, NT, NT] output; when NULL the workspace holds the scores.
 * workspace: device buffer of at least pasa_select_workspace_bytes(bh, NT) bytes
 * (may be NULL when scores_out is given).  head_dim 1 .. 128; NT <= 65536 (rows of more
 * than 4096 blocks take a radix select over the row in memory, whose index list, when
 * asked for, holds at most 8192 blocks).
 * Replaces: group_pisa_attention.py:365-375. */
int pasa_select(const float* qc, const float* kc, const float* hnorm, const float* noise,
                double scale, double density, int use_cov_bias,
                int32_t* idx, uint32_t* selmask, float* scores_out,
                void* workspace, size_t workspace_bytes,
                int64_t bh, int64_t num_blocks, int64_t head_dim, void* stream);

size_t pasa_select_workspace_bytes(int64_t bh, int64_t num_blocks);

/* Top-k of given fp32 scores [BH, NT, NT] with the rule above: the bit-exact
 * parity entry of K3 (same kernel as pasa_select's second stage).
 * Replaces: torch.topk at group_pisa_attention.py:374-375. */
int pasa_select_from_scores(const float* scores, int64_t ns, int32_t* idx, uint32_t* selmask,
                            int64_t bh, int64_t num_blocks, void* stream);

/* ---- K4: block-sparse attention with per-group first-order correction -----
 * For query block I: exact online-softmax attention over the key blocks selected
 * in selmask[I], then for each group g of 32 key blocks the zero-order (kc, vc)
 * plus first-order (hgroup) contribution of the blocks of g not selected, merged
 * into the same running max; o = A / (L + Gamma).  The kernel reads the selection
 * from selmask only (idx, the matching index list as pasa_select writes it, is not
 * read and may be NULL): the exact blocks are visited in ascending block order,
 * which equals the reference's top-k order up to floating-point rounding.
 * gamma_literal = 1 reproduces the reference exactly: Gamma (the zero-order
 * denominator, sum p_j * n_j) is not rescaled when the running max rises;
 * gamma_literal = 0 rescales it with A and L.
 * scale: the natural-log softmax scale s (> 0); scores use s*log2(e) in base 2
 * and the first-order term uses s.
 * dtype: PASA_DTYPE_BF16, PASA_DTYPE_F16 or PASA_DTYPE_F32 (q, k, v, o; kc, vc and
 * hgroup are rounded to that type where the reference stores them in it, and P is
 * rounded to it before P.V, as the reference casts it to v's dtype; fp32 calls round
 * nothing); shapes as described at the top.
 * workspace: >= pasa_sparse_attn_workspace_bytes(...) bytes (packed phase-2
 * operands, written by this call; 0 bytes and NULL allowed for shapes outside the
 * tuned ones, whose kernel reads kc, vc and hgroup directly).
 * Replaces: pisa_pg_fwd_kernel group_pisa_attention.py:135-262, launched at :380-396. */
int pasa_sparse_attn(const void* q, const void* k, const void* v,
                     const float* kc, const float* vc, const float* hgroup,
                     const int32_t* idx, const uint32_t* selmask, void* o,
                     double scale, int64_t bh, int64_t seq_len, int64_t text_len,
                     int64_t text_valid, int64_t head_dim,
                     int64_t block_size, int64_t group_size, int64_t ns,
                     int gamma_literal, int dtype,
                     void* workspace, size_t workspace_bytes, void* stream);

size_t pasa_sparse_attn_workspace_bytes(int64_t bh, int64_t seq_len, int64_t text_len,
                                        int64_t head_dim, int64_t block_size, int64_t group_size);

/* The two halves of pasa_sparse_attn, for callers that reuse the packed phase-2
 * operands or time the attention kernel alone.
 * pasa_pack_phase2 writes, per (slice, group of 32 key blocks), kbar, the value
 * sums (transposed) and Hbar (transposed) in `dtype` (bf16, or fp16 at head_dim 128;
 * it must be the dtype of the attention call that reads the pack) into `pack`
 * (pasa_sparse_attn_workspace_bytes(...) bytes).
 * Replaces: the stores of kc/vc in the input dtype (group_pisa_attention.py:118-119)
 * and the cast of h_group at its use (:251). */
int pasa_pack_phase2(const float* kc, const float* vc, const float* hgroup, void* pack,
                     size_t pack_bytes, int64_t bh, int64_t seq_len, int64_t text_len,
                     int64_t head_dim, int64_t block_size, int64_t group_size, int dtype,
                     void* stream);

/* K4 proper on operands packed by pasa_pack_phase2 (same arguments and semantics
 * as pasa_sparse_attn otherwise).
 * Replaces: pisa_pg_fwd_kernel group_pisa_attention.py:135-262. */
int pasa_sparse_attn_packed(const void* q, const void* k, const void* v, const void* pack,
                            size_t pack_bytes, const int32_t* idx, const uint32_t* selmask,
                            void* o, double scale, int64_t bh, int64_t seq_len, int64_t text_len,
                            int64_t text_valid, int64_t head_dim, int64_t block_size,
                            int64_t group_size, int64_t ns, int gamma_literal, int dtype, void* stream);

/* pasa_sparse_attn without a workspace argument: the packed phase-2 operands live in
 * a static device array of PASA_NOALLOC_SCRATCH_BYTES bytes that the library holds on
 * every GPU it runs on until the process ends, so the call allocates nothing and
 * needs no caller buffer beyond its inputs and outputs.  Its size limits the shape:
 * pasa_sparse_attn_workspace_bytes(...) <= PASA_NOALLOC_SCRATCH_BYTES must hold.  That
 * is bh * ceil(ceil((seq_len - text_len) / block_size) / 32) slice-groups of 53,248 bytes
 * each at head_dim 128 (1,260 slice-groups fit: the Wan2.1-14B 720p shape at block size
 * 128 needs 760, HunyuanVideo 720p at block size 128 720, Wan2.1-1.3B at block size 64
 * 192) and of 20,480 bytes each at head_dim 64 (3,276 fit); a larger shape returns
 * PASA_ERR_WORKSPACE before any launch.  Calls on one GPU share its array,
 * so calls that overlap on one GPU race; calls in stream order do not.  The first
 * call on a device looks the array's address up (hipGetSymbolAddress) and caches it.
 * Arguments and results otherwise as pasa_sparse_attn (same kernels, bitwise-equal
 * output).
 * No counterpart in the reference: this entry is for callers that cannot allocate
 * device memory, such as code under HIP graph capture and tight serving loops. */
#define PASA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int pasa_sparse_attn_noalloc(const void* q, const void* k, const void* v,
                             const float* kc, const float* vc, const float* hgroup,
                             const int32_t* idx, const uint32_t* selmask, void* o,
                             double scale, int64_t bh, int64_t seq_len, int64_t text_len,
                             int64_t text_valid, int64_t head_dim,
                             int64_t block_size, int64_t group_size, int64_t ns,
                             int gamma_literal, int dtype, void* stream);

/* ---- Token-major view of frame-major tensors -------------------------------- */

/* The HunyuanVideo placement (pasa_permute's forward map) as a view: for a head
 * whose flag is set, logical row p*F + f of the first F*P rows of a slice (token p
 * of frame f, token-major) is stored at row f*P + p (frame-major); the rows after
 * them (the text tail) and every row of a head whose flag is 0 are in place. */
typedef struct {
  int64_t num_frame;               /* F */
  int64_t frame_size;              /* P, tokens per frame; F*P = seq_len - text_len <= 2^24 */
  const int32_t* head_is_temporal; /* device int32 [heads]; NULL: every head permuted      */
  int64_t heads;                   /* slice s is head s % heads                            */
} pasa_placement_t;

/* The placement folded into K2 and K4.  pasa_block_stats_placed reads frame-major
 * q, k, v once: it computes the statistics of their token-major view and writes that
 * view to k_tm, v_tm and, unless it is NULL, q_tm (device [BH, seq_len, head_dim] in q's
 * dtype, text rows copied in place) in the same pass.  pasa_sparse_attn_packed_placed takes
 * the frame-major q itself (each query row is read once, through the placement map) and
 * the token-major copies k_tm, v_tm as k, v, and stores o frame-major.  Together they equal pasa_permute ->
 * pasa_block_stats -> ... -> pasa_sparse_attn_packed -> inverse pasa_permute bit for
 * bit, without the permutation's separate read of q, k, v and its second pass over o.
 * The copies are written while q, k, v are read: a copy that overlaps q, k, v or another
 * copy (an in-place permutation) returns PASA_ERR_BAD_ARG.
 * head_dim 128, block_size 128; arguments otherwise as for the unplaced entry points
 * (pasa_block_stats_placed's workspace as pasa_block_stats_ws's: with the same
 * workspace the group moments equal the unplaced call's bit for bit).
 * Replaces: hunyuan_sparse_head_placement / hunyuan_hidden_states_placement around the
 * attention call (svg/models/hyvideo/placement.py:124-153, :360-387;
 * svg/models/hyvideo/attention.py:412-446). */
int pasa_block_stats_placed(const void* q, const void* k, const void* v,
                            void* q_tm, void* k_tm, void* v_tm,
                            float* qc, float* kc, float* vc, float* hnorm, float* hgroup,
                            int64_t bh, int64_t seq_len, int64_t text_len, int64_t head_dim,
                            int64_t block_size, int64_t group_size,
                            const pasa_placement_t* placement, int dtype,
                            void* workspace, size_t workspace_bytes, void* stream);
int pasa_sparse_attn_packed_placed(const void* q, const void* k, const void* v, const void* pack,
                                   size_t pack_bytes, const int32_t* idx, const uint32_t* selmask,
                                   void* o, double scale, int64_t bh, int64_t seq_len,
                                   int64_t text_len, int64_t text_valid, int64_t head_dim,
                                   int64_t block_size, int64_t group_size, int64_t ns,
                                   int gamma_literal, const pasa_placement_t* placement,
                                   int dtype, void* stream);

/* Dense softmax attention, o = softmax(scale * q k^T) v, on K4's exact-tile path
 * (every key block exact; no statistics, selection or correction).  With a text
 * segment (text_len > 0) the attention is block-diagonal over [0, seq_len -
 * text_len + text_valid) and the padding rows after it, the cu_seqlens semantics
 * of the dense HunyuanVideo path.  bf16 or fp16 at head_dim 128 on the tuned kernel;
 * fp32, bf16 or fp16 at head_dim 1 .. 128 otherwise; no workspace.
 * Replaces: the dense warm-up branch of the processors, flash_attention /
 * F.scaled_dot_product_attention (svg/models/wan/attention.py:299-301, :378-379;
 * svg/models/hyvideo/attention.py:450-476, :671-672). */
int pasa_dense_attn(const void* q, const void* k, const void* v, void* o, double scale,
                    int64_t bh, int64_t seq_len, int64_t text_len, int64_t text_valid,
                    int64_t head_dim, int dtype, void* stream);

/* ---- Processor prologue (K5) ------------------------------------------------ */

typedef enum {
  PASA_LAYOUT_BHSD = 0,  /* [B, H, S, D]: head-major, what the attention entry points read */
  PASA_LAYOUT_BSHD = 1   /* [B, S, H*D]: token-major, what the projections produce        */
} pasa_layout_t;

typedef enum {
  PASA_NORM_NONE = 0,
  PASA_NORM_HEAD = 1,    /* RMSNorm over each head's D channels; weight [D]      */
  PASA_NORM_ROW = 2      /* RMSNorm over the token's H*D channels; weight [H*D]  */
} pasa_norm_t;

typedef enum {
  PASA_NORM_ROUND_ONCE = 0,  /* y = bf16((x*rstd)*w), rstd = 1/sqrt(mean(x^2)+eps)          */
  PASA_NORM_ROUND_TWICE = 1  /* y = bf16(bf16(x*rsqrt(mean(x^2)+eps))*w): diffusers RMSNorm */
} pasa_norm_rounding_t;

typedef enum {
  PASA_ROPE_NONE = 0,
  PASA_ROPE_COSSIN_F32 = 1,  /* cos, sin fp32 [rope_rows, D]; pairs (x[2i], x[2i+1]):
                                o[2i] = x[2i]cos[2i] - x[2i+1]sin[2i],
                                o[2i+1] = x[2i+1]cos[2i+1] + x[2i]sin[2i+1], fp32 steps */
  PASA_ROPE_COMPLEX_F64 = 2  /* cos = Re, sin = Im, fp64 [rope_rows, D/2]; (x[2i] + i x[2i+1])
                                times the coefficient in fp64, cast fp64 -> fp32 -> bf16     */
} pasa_rope_t;

/* Q/K RMSNorm and rotary embedding, fused with the head split, in one pass.
 * xq, xk, xv: bf16 inputs in in_layout with `seq_len` rows per (b, h) (any may be
 * NULL: that tensor is skipped; its output must then be NULL too).  q, k, v: bf16
 * outputs in out_layout with out_seq_len rows per (b, h); input row s lands at
 * output row out_row0 + s (so two calls can fill the video and text parts of one
 * joint sequence).  wq, wk: bf16 RMSNorm weights ([D] for PASA_NORM_HEAD, [H*D]
 * for PASA_NORM_ROW); a NULL weight leaves that tensor unnormalised.  V is only
 * moved.  Rows s < rope_rows of Q and K are rotated after the norm; rows past it
 * (trailing text tokens) are not.  Each step rounds to bf16 where the step-by-step
 * reference does, so the result equals the unfused pipeline up to the order of
 * the sum of squares.  Input and output may be the same buffer when in_layout ==
 * out_layout, out_seq_len == seq_len and out_row0 == 0 (in place); other
 * overlaps are not allowed.  head_dim 64 or 128; heads*head_dim <= 8192.
 * Replaces: triton_rmsnorm_forward (svg/kernels/triton/rmsnorm.py:8-101) and the
 * head split + rotary steps of the Wan processor (svg/models/wan/attention.py:31-57,
 * :114-150, :182-188); the absent _kernels.rms_norm_forward and
 * _kernels.apply_qk_rope_inplace_cossin_{txtlast,complex} (call sites
 * svg/models/hyvideo/attention.py:162-190, svg/models/wan/attention.py:36-39), with
 * the PyTorch fallbacks at hyvideo/attention.py:196-230 as their observable
 * behaviour. */
int pasa_qkv_prologue(const void* xq, const void* xk, const void* xv,
                      void* q, void* k, void* v,
                      const void* wq, const void* wk,
                      int64_t batch, int64_t seq_len, int64_t heads, int64_t head_dim,
                      int in_layout, int out_layout, int64_t out_seq_len, int64_t out_row0,
                      int norm, int norm_rounding, double eps,
                      const void* rope_cos, const void* rope_sin, int rope, int64_t rope_rows,
                      int dtype, void* stream);

/* ---- DiT block row operations (K6) ------------------------------------------ */

/* Per token row of `cols` elements (rows = batches * rows_per_batch), in one pass:
 *   stage A, when residual != NULL:
 *     h = residual + x * gate   (gate == NULL: h = residual + x), rounded to h_dtype;
 *     written to h_out when h_out != NULL (h_out may equal residual: in place).
 *   stage B, when y != NULL, on h (stage A) or on x:
 *     layernorm != 0:  v = (v - mean) * rstd, mean = sum(v)/cols,
 *                      rstd = 1/sqrt(sum((v - mean)^2)/cols + eps)
 *     weight != NULL:  v = v * weight;   bias != NULL: v = v + bias
 *     scale != NULL:   v = v * (1 + scale) + shift
 *     written to y as y_dtype.
 * Every product and sum is one fp32 operation rounded to nearest, as in the
 * reference's PyTorch fallback; the two row sums are taken per lane in column-chunk
 * order and then across the 64 lanes of a wave (a fixed order: equal inputs give
 * equal outputs).  x_dtype, residual_dtype, h_dtype, y_dtype, wb_dtype: bf16 or
 * fp32; gate, scale, shift: fp32, one row of `cols` per batch, successive rows
 * `param_stride` elements apart (0: one row for every batch).  cols: a multiple of
 * 8, at most 8192; every pointer 16-byte aligned, param_stride a multiple of 4.
 * Buffers among x, residual, h_out and y either do not overlap or are the same
 * pointer with the same dtype.
 * Replaces: triton_layernorm_forward (svg/kernels/triton/layernorm.py:9-63,
 * :110-161, :200-206), triton_modulate_shift_forward (modulate.py:12-78) and
 * triton_modulate_gate_residual_forward (modulate.py:85-164), as called by the Wan
 * block (svg/models/wan/custom_models.py:23-115), where one call does a gated
 * residual and the following LayerNorm and modulation together. */
int pasa_row_ops(const void* x, int x_dtype,
                 const void* residual, int residual_dtype, const float* gate, void* h_out, int h_dtype,
                 int layernorm, const void* weight, const void* bias, int wb_dtype,
                 const float* scale, const float* shift,
                 void* y, int y_dtype,
                 int64_t rows, int64_t cols, int64_t rows_per_batch, int64_t param_stride,
                 double eps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PASA_H_ */
