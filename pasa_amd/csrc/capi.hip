// C ABI of the PISA-PG hot path (declared in include/pasa.h).
//
// Every entry point validates all arguments on the host before touching the
// HIP runtime, records a thread-local error message and returns a negative
// pasa_status_t on failure; kernel launch failures are reported from
// hipGetLastError as PASA_ERR_LAUNCH.  Nothing here allocates or synchronises.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "../../include/pasa.h"
#include "kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return PASA_OK;
}

int launch_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(PASA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

constexpr int64_t kMaxGridY = 65535;
constexpr int64_t kMaxI32 = 2147483647;

int check_head_dim(int64_t d) {
  if (d != 64 && d != 128) return fail(PASA_ERR_HEAD_DIM, "head_dim %lld not in {64, 128}", (long long)d);
  return PASA_OK;
}

int check_block(int64_t b) {
  if (b != 64 && b != 128) return fail(PASA_ERR_BLOCK_SIZE, "block_size %lld not in {64, 128}", (long long)b);
  return PASA_OK;
}

int check_bh_seq(int64_t bh, int64_t seq_len, int64_t head_dim) {
  if (bh <= 0 || seq_len <= 0) return fail(PASA_ERR_BAD_SHAPE, "bh=%lld and seq_len=%lld must be > 0", (long long)bh, (long long)seq_len);
  if (bh > kMaxGridY) return fail(PASA_ERR_OVERFLOW, "bh=%lld exceeds %lld", (long long)bh, (long long)kMaxGridY);
  if (seq_len > kMaxI32 / 2) return fail(PASA_ERR_OVERFLOW, "seq_len=%lld too large", (long long)seq_len);
  if (head_dim > 0 && bh > INT64_MAX / seq_len / head_dim / 4) return fail(PASA_ERR_OVERFLOW, "bh*seq_len*head_dim overflows");
  return PASA_OK;
}

// The kernels address one (batch, head) slice through a 32-bit buffer offset;
// one padded block past the end must still be addressable.
int check_slice_bytes(int64_t seq_len, int64_t head_dim, int64_t elem_bytes) {
  if ((seq_len + 128) * head_dim * elem_bytes > (int64_t)UINT32_MAX)
    return fail(PASA_ERR_OVERFLOW, "seq_len*head_dim*%lld bytes exceeds the 4 GiB slice limit", (long long)elem_bytes);
  return PASA_OK;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// The text segment is the last text_len rows of each slice; at least one blocked
// row must remain.  Only the D = 128 kernels implement it.
int check_text(int64_t seq_len, int64_t text_len, int64_t head_dim) {
  if (text_len < 0 || text_len >= seq_len)
    return fail(PASA_ERR_TEXT_SEGMENT, "text_len=%lld must be in [0, seq_len=%lld)", (long long)text_len, (long long)seq_len);
  if (text_len > 0 && head_dim != 128)
    return fail(PASA_ERR_TEXT_SEGMENT, "a text segment needs head_dim 128 (got %lld)", (long long)head_dim);
  return PASA_OK;
}

}  // namespace

extern "C" {

int pasa_abi_version(void) { return PASA_ABI_VERSION; }

const char* pasa_status_string(int status) {
  switch (status) {
    case PASA_OK: return "ok";
    case PASA_ERR_NULL_POINTER: return "null pointer";
    case PASA_ERR_BAD_SHAPE: return "bad shape";
    case PASA_ERR_HEAD_DIM: return "unsupported head_dim";
    case PASA_ERR_BLOCK_SIZE: return "unsupported block_size";
    case PASA_ERR_NUM_SELECTED: return "number of selected blocks out of range";
    case PASA_ERR_OVERFLOW: return "size overflow";
    case PASA_ERR_DTYPE: return "unsupported dtype";
    case PASA_ERR_WORKSPACE: return "workspace missing or too small";
    case PASA_ERR_BAD_ARG: return "bad argument";
    case PASA_ERR_TEXT_SEGMENT: return "text segment does not fit";
    case PASA_ERR_LAUNCH: return "kernel launch failed";
    case PASA_ERR_GROUP_SIZE: return "unsupported group_size";
    case PASA_ERR_TOO_MANY_BLOCKS: return "too many key blocks for the select kernel";
    default: return "unknown status";
  }
}

const char* pasa_last_error(void) { return g_err; }

int64_t pasa_num_selected(double density, int64_t num_blocks) {
  if (num_blocks <= 0) return fail(PASA_ERR_BAD_SHAPE, "num_blocks must be > 0");
  if (!std::isfinite(density)) return fail(PASA_ERR_BAD_ARG, "density must be finite");
  const double prod = density * (double)num_blocks;
  if (!std::isfinite(prod) || std::fabs(prod) > 9.0e18) return fail(PASA_ERR_BAD_ARG, "density * NT overflows");
  int64_t ns = (int64_t)prod;  // truncation toward zero, as Python's int()
  if (ns < 1) ns = 1;
  if (ns > num_blocks) ns = num_blocks;
  ok();
  return ns;
}

int pasa_permute(const void* src0, const void* src1, const void* src2, void* dst0, void* dst1,
                 void* dst2, int n_tensors, int64_t bh, int64_t num_frame, int64_t frame_size,
                 int64_t context_length, int64_t head_dim, int dtype,
                 const int32_t* head_is_temporal, int inverse, void* stream) {
  if (n_tensors < 1 || n_tensors > 3) return fail(PASA_ERR_BAD_ARG, "n_tensors=%d not in [1, 3]", n_tensors);
  const void* srcs[3] = {src0, src1, src2};
  void* dsts[3] = {dst0, dst1, dst2};
  for (int i = 0; i < n_tensors; ++i)
    if (!srcs[i] || !dsts[i]) return fail(PASA_ERR_NULL_POINTER, "tensor %d: src/dst is NULL", i);
  int esize;
  if (dtype == PASA_DTYPE_BF16 || dtype == PASA_DTYPE_F16) esize = 2;
  else if (dtype == PASA_DTYPE_F32) esize = 4;
  else return fail(PASA_ERR_DTYPE, "dtype %d unknown", dtype);
  if (head_dim <= 0) return fail(PASA_ERR_BAD_SHAPE, "head_dim must be > 0");
  const int64_t row_bytes = head_dim * esize;
  if (row_bytes % 16 != 0 || row_bytes > 4096)
    return fail(PASA_ERR_HEAD_DIM, "head_dim*element size = %lld bytes must be a multiple of 16 and <= 4096", (long long)row_bytes);
  if (num_frame <= 0 || frame_size <= 0 || context_length < 0)
    return fail(PASA_ERR_BAD_SHAPE, "num_frame and frame_size must be > 0, context_length >= 0");
  if (num_frame > kMaxI32 / frame_size) return fail(PASA_ERR_OVERFLOW, "num_frame*frame_size overflows");
  const int64_t S = context_length + num_frame * frame_size;
  if (S > kMaxI32) return fail(PASA_ERR_OVERFLOW, "sequence length %lld too large", (long long)S);
  int rc = check_bh_seq(bh, S, head_dim);
  if (rc) return rc;
  if (inverse != 0 && inverse != 1) return fail(PASA_ERR_BAD_ARG, "inverse must be 0 or 1");
  const uintptr_t bytes = (uintptr_t)(bh * S * row_bytes);
  for (int i = 0; i < n_tensors; ++i)
    for (int jx = 0; jx < n_tensors; ++jx) {
      const uintptr_t a = (uintptr_t)srcs[i], b = (uintptr_t)dsts[jx];
      if (a < b + bytes && b < a + bytes) return fail(PASA_ERR_BAD_ARG, "src %d overlaps dst %d (in-place permutation is not supported)", i, jx);
    }
  return launch_status(pasa::launch_permute(src0, src1, src2, dst0, dst1, dst2, n_tensors, (int)bh, (int)S,
                                            (int)num_frame, (int)frame_size, (int)context_length,
                                            (int)row_bytes, head_is_temporal, inverse, (hipStream_t)stream),
                       "pasa_permute");
}

// The attention path's 16-bit tensors: bf16, or fp16 at head_dim 128 (the D = 64 kernels
// are bf16 only).
static int check_attn_dtype(int dtype, int64_t head_dim, const char* what) {
  if (dtype == PASA_DTYPE_BF16) return PASA_OK;
  if (dtype == PASA_DTYPE_F16) {
    if (head_dim == 128) return PASA_OK;
    return fail(PASA_ERR_DTYPE, "%s: fp16 inputs need head_dim 128 (got %lld)", what, (long long)head_dim);
  }
  return fail(PASA_ERR_DTYPE, "%s: dtype %d is not bf16 or fp16", what, dtype);
}

// The tuned kernels' shapes: bf16 (fp16 at head_dim 128) q, k, v, head_dim 64 or 128, block
// size 64 or 128.  Every other shape the entry points accept (fp32 inputs, head dims 1 ..
// 128, block sizes 16 .. 256) runs on the any-shape kernels (any_shape.hip).
static bool tuned_shape(int dtype, int64_t head_dim, int64_t block_size) {
  return (head_dim == 64 || head_dim == 128) && (block_size == 64 || block_size == 128) &&
         (dtype == PASA_DTYPE_BF16 || (dtype == PASA_DTYPE_F16 && head_dim == 128));
}

// ... and the tuned attention kernels also need group size 32, and a text segment only at
// head_dim 128.
static bool tuned_attn_shape(int dtype, int64_t head_dim, int64_t block_size, int64_t group_size,
                             int64_t text_len) {
  return tuned_shape(dtype, head_dim, block_size) && group_size == 32 && (text_len == 0 || head_dim == 128);
}

static int check_any_dtype(int dtype, const char* what) {
  if (dtype == PASA_DTYPE_BF16 || dtype == PASA_DTYPE_F16 || dtype == PASA_DTYPE_F32) return PASA_OK;
  return fail(PASA_ERR_DTYPE, "%s: dtype %d is not bf16, fp16 or fp32", what, dtype);
}

// The any-shape kernels: head_dim 1 .. 128, block size a power of two in [16, 256] (the
// reference's Triton kernels need a power of two, and tl.dot at least 16), group size
// 1 .. 2^20, a text segment that leaves at least one blocked row.
static int check_any_shape(int64_t bh, int64_t seq_len, int64_t text_len, int64_t head_dim, int64_t block_size,
                           int64_t group_size, const char* what) {
  if (head_dim < 1 || head_dim > 128)
    return fail(PASA_ERR_HEAD_DIM, "%s: head_dim %lld not in [1, 128]", what, (long long)head_dim);
  if (block_size < 16 || block_size > 256 || (block_size & (block_size - 1)))
    return fail(PASA_ERR_BLOCK_SIZE, "%s: block_size %lld is not a power of two in [16, 256]", what,
                (long long)block_size);
  if (group_size <= 0 || group_size > 1 << 20)
    return fail(PASA_ERR_GROUP_SIZE, "%s: group_size %lld must be in [1, 2^20]", what, (long long)group_size);
  int rc;
  if ((rc = check_bh_seq(bh, seq_len, head_dim))) return rc;
  if (text_len < 0 || text_len >= seq_len)
    return fail(PASA_ERR_TEXT_SEGMENT, "%s: text_len=%lld must be in [0, seq_len=%lld)", what, (long long)text_len,
                (long long)seq_len);
  return PASA_OK;
}

static int block_stats_impl(const void* q, const void* k, const void* v, float* qc, float* kc, float* vc,
                            float* hnorm, float* hgroup, int64_t bh, int64_t seq_len, int64_t text_len,
                            int64_t head_dim, int64_t block_size, int64_t group_size, int dtype,
                            const pasa::RowMap* rm, void* const* tm_copies, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (!q || !k || !v || !qc || !kc || !vc || !hnorm || !hgroup) return fail(PASA_ERR_NULL_POINTER, "pasa_block_stats: NULL pointer");
  int rc;
  // The tuned statistics kernels take a text segment at head_dim 128 only.
  if (rm == nullptr && (!tuned_shape(dtype, head_dim, block_size) || (text_len != 0 && head_dim != 128))) {
    if ((rc = check_any_dtype(dtype, "pasa_block_stats"))) return rc;
    if ((rc = check_any_shape(bh, seq_len, text_len, head_dim, block_size, group_size, "pasa_block_stats")))
      return rc;
    const int64_t ng = cdiv(cdiv(seq_len - text_len, block_size), group_size);
    if (ng > 65535 * 1024LL) return fail(PASA_ERR_OVERFLOW, "pasa_block_stats: too many groups");
    return launch_status(pasa::launch_block_stats_any(q, k, v, qc, kc, vc, hnorm, hgroup, (int)bh,
                                                      (int)(seq_len - text_len), (int)seq_len, (int)head_dim,
                                                      (int)block_size, (int)group_size, dtype, (hipStream_t)stream),
                         "pasa_block_stats");
  }
  if ((rc = check_head_dim(head_dim))) return rc;
  if ((rc = check_attn_dtype(dtype, head_dim, "pasa_block_stats"))) return rc;
  if ((rc = check_block(block_size))) return rc;
  if ((rc = check_bh_seq(bh, seq_len, head_dim))) return rc;
  if ((rc = check_slice_bytes(seq_len, head_dim, 2))) return rc;
  if ((rc = check_text(seq_len, text_len, head_dim))) return rc;
  if (group_size <= 0 || group_size > 1 << 20) return fail(PASA_ERR_GROUP_SIZE, "group_size %lld must be in [1, 2^20]", (long long)group_size);
  int split = 1;
  if (workspace != nullptr) {
    split = pasa::block_stats_split((int)bh, (int)(seq_len - text_len), (int)head_dim, (int)block_size,
                                    (int)group_size);
    const size_t need = pasa_block_stats_workspace_bytes(bh, seq_len, text_len, head_dim, block_size, group_size);
    if (workspace_bytes < need)
      return fail(PASA_ERR_WORKSPACE, "pasa_block_stats_ws: workspace %zu bytes < %zu", workspace_bytes, need);
    if (((uintptr_t)workspace | (uintptr_t)hgroup) & 15u)
      return fail(PASA_ERR_BAD_ARG, "pasa_block_stats_ws: workspace and hgroup must be 16-byte aligned");
  }
  return launch_status(pasa::launch_block_stats(q, k, v, qc, kc, vc, hnorm, hgroup, (int)bh,
                                                (int)(seq_len - text_len), (int)seq_len, (int)head_dim,
                                                (int)block_size, (int)group_size, rm, tm_copies,
                                                (float*)workspace, split, dtype == PASA_DTYPE_F16,
                                                (hipStream_t)stream),
                       "pasa_block_stats");
}

size_t pasa_block_stats_workspace_bytes(int64_t bh, int64_t seq_len, int64_t text_len, int64_t head_dim,
                                        int64_t block_size, int64_t group_size) {
  if (bh <= 0 || bh > kMaxGridY || seq_len <= 0 || seq_len > kMaxI32 / 2 || text_len < 0 || text_len >= seq_len ||
      (head_dim != 64 && head_dim != 128) || (block_size != 64 && block_size != 128) || group_size <= 0 ||
      group_size > 1 << 20)
    return 0;
  const int split = pasa::block_stats_split((int)bh, (int)(seq_len - text_len), (int)head_dim, (int)block_size,
                                            (int)group_size);
  if (split == 1) return 0;
  const int64_t ng = cdiv(cdiv(seq_len - text_len, block_size), group_size);
  return (size_t)bh * (size_t)ng * (size_t)split * (size_t)(head_dim * head_dim) * sizeof(float);
}

int pasa_block_stats(const void* q, const void* k, const void* v, float* qc, float* kc, float* vc,
                     float* hnorm, float* hgroup, int64_t bh, int64_t seq_len, int64_t text_len,
                     int64_t head_dim, int64_t block_size, int64_t group_size, int dtype, void* stream) {
  return block_stats_impl(q, k, v, qc, kc, vc, hnorm, hgroup, bh, seq_len, text_len, head_dim, block_size,
                          group_size, dtype, nullptr, nullptr, nullptr, 0, stream);
}

int pasa_block_stats_ws(const void* q, const void* k, const void* v, float* qc, float* kc, float* vc,
                        float* hnorm, float* hgroup, int64_t bh, int64_t seq_len, int64_t text_len,
                        int64_t head_dim, int64_t block_size, int64_t group_size, int dtype, void* workspace,
                        size_t workspace_bytes, void* stream) {
  return block_stats_impl(q, k, v, qc, kc, vc, hnorm, hgroup, bh, seq_len, text_len, head_dim, block_size,
                          group_size, dtype, nullptr, nullptr, workspace, workspace_bytes, stream);
}

// The placement's row map, after checking it fits the slices it will address.
static int check_placement(const pasa_placement_t* pl, int64_t bh, int64_t seq_len, int64_t text_len,
                           int64_t head_dim, int64_t block_size, pasa::RowMap* rm) {
  if (!pl) return fail(PASA_ERR_NULL_POINTER, "placement is NULL");
  if (head_dim != 128) return fail(PASA_ERR_HEAD_DIM, "the placed kernels need head_dim 128 (got %lld)", (long long)head_dim);
  if (block_size != 128) return fail(PASA_ERR_BLOCK_SIZE, "the placed kernels need block_size 128 (got %lld)", (long long)block_size);
  if (pl->num_frame < 1 || pl->frame_size < 1 || pl->num_frame > (1 << 24) || pl->frame_size > (1 << 24) ||
      pl->num_frame * pl->frame_size != seq_len - text_len)
    return fail(PASA_ERR_BAD_SHAPE, "num_frame*frame_size=%lld*%lld must equal seq_len - text_len = %lld",
                (long long)pl->num_frame, (long long)pl->frame_size, (long long)(seq_len - text_len));
  if (pl->num_frame * pl->frame_size > (1 << 24))
    return fail(PASA_ERR_OVERFLOW, "num_frame*frame_size exceeds 2^24 rows");
  if (pl->heads < 1 || bh % pl->heads != 0)
    return fail(PASA_ERR_BAD_SHAPE, "heads=%lld must divide bh=%lld", (long long)pl->heads, (long long)bh);
  *rm = pasa::RowMap{(int)pl->num_frame, (int)pl->frame_size, 1.0f / (float)pl->num_frame, pl->head_is_temporal,
                     (int)pl->heads};
  return PASA_OK;
}

int pasa_block_stats_placed(const void* q, const void* k, const void* v, void* q_tm, void* k_tm, void* v_tm,
                            float* qc, float* kc, float* vc, float* hnorm, float* hgroup, int64_t bh,
                            int64_t seq_len, int64_t text_len, int64_t head_dim, int64_t block_size,
                            int64_t group_size, const pasa_placement_t* placement, int dtype, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (!k_tm || !v_tm) return fail(PASA_ERR_NULL_POINTER, "pasa_block_stats_placed: NULL pointer");
  pasa::RowMap rm;
  int rc;
  if ((rc = check_placement(placement, bh, seq_len, text_len, head_dim, block_size, &rm))) return rc;
  void* const copies[3] = {q_tm, k_tm, v_tm};
  // The copies are written while q, k, v are still being read (and each other's rows are
  // distinct), so none may overlap an input or another copy.
  if (bh > 0 && seq_len > 0 && bh <= kMaxGridY && seq_len <= kMaxI32 / 2) {
    const uintptr_t bytes = (uintptr_t)(bh * seq_len * head_dim * 2);
    const void* const inputs[3] = {q, k, v};
    const char* const names[3] = {"q", "k", "v"};
    for (int i = 0; i < 3; ++i) {
      if (!copies[i]) continue;
      const uintptr_t a = (uintptr_t)copies[i];
      for (int j = 0; j < 3; ++j) {
        const uintptr_t b = (uintptr_t)inputs[j];
        if (b && a < b + bytes && b < a + bytes)
          return fail(PASA_ERR_BAD_ARG, "pasa_block_stats_placed: %s_tm overlaps %s", names[i], names[j]);
        const uintptr_t c = (uintptr_t)copies[j];
        if (j != i && c && a < c + bytes && c < a + bytes)
          return fail(PASA_ERR_BAD_ARG, "pasa_block_stats_placed: %s_tm overlaps %s_tm", names[i], names[j]);
      }
    }
  }
  return block_stats_impl(q, k, v, qc, kc, vc, hnorm, hgroup, bh, seq_len, text_len, head_dim, block_size,
                          group_size, dtype, &rm, copies, workspace, workspace_bytes, stream);
}

size_t pasa_select_workspace_bytes(int64_t bh, int64_t num_blocks) {
  if (bh <= 0 || num_blocks <= 0) return 0;
  return (size_t)bh * (size_t)num_blocks * (size_t)num_blocks * sizeof(float);
}

static int check_select_shape(int64_t bh, int64_t nt) {
  if (bh <= 0 || nt <= 0) return fail(PASA_ERR_BAD_SHAPE, "bh=%lld and num_blocks=%lld must be > 0", (long long)bh, (long long)nt);
  if (bh > kMaxGridY) return fail(PASA_ERR_OVERFLOW, "bh=%lld exceeds %lld", (long long)bh, (long long)kMaxGridY);
  if (nt > pasa::kMaxSelectBlocks) return fail(PASA_ERR_TOO_MANY_BLOCKS, "num_blocks=%lld exceeds %d", (long long)nt, pasa::kMaxSelectBlocks);
  return PASA_OK;
}

// Rows of more than 4096 blocks sort their index list in LDS: at most 8192 indices.
static int check_index_list(const int32_t* idx, int64_t nt, int64_t ns) {
  if (idx != nullptr && nt > 4096 && ns > pasa::kMaxLargeSortKeys)
    return fail(PASA_ERR_TOO_MANY_BLOCKS, "an index list of %lld blocks (of %lld) exceeds %d; pass idx = NULL "
                "for the selection bitmask alone", (long long)ns, (long long)nt, pasa::kMaxLargeSortKeys);
  return PASA_OK;
}

int pasa_select(const float* qc, const float* kc, const float* hnorm, const float* noise,
                double scale, double density, int use_cov_bias, int32_t* idx, uint32_t* selmask,
                float* scores_out, void* workspace, size_t workspace_bytes, int64_t bh,
                int64_t num_blocks, int64_t head_dim, void* stream) {
  if (!qc || !kc || !selmask) return fail(PASA_ERR_NULL_POINTER, "pasa_select: NULL pointer");
  if (use_cov_bias && !hnorm) return fail(PASA_ERR_NULL_POINTER, "pasa_select: hnorm is NULL with use_cov_bias");
  int rc;
  if ((rc = check_select_shape(bh, num_blocks))) return rc;
  if (head_dim < 1 || head_dim > 128)
    return fail(PASA_ERR_HEAD_DIM, "pasa_select: head_dim %lld not in [1, 128]", (long long)head_dim);
  if (!std::isfinite(scale)) return fail(PASA_ERR_BAD_ARG, "scale must be finite");
  const int64_t ns = pasa_num_selected(density, num_blocks);
  if (ns < 0) return (int)ns;
  if ((rc = check_index_list(idx, num_blocks, ns))) return rc;
  float* scores = scores_out;
  if (!scores) {
    if (!workspace) return fail(PASA_ERR_WORKSPACE, "pasa_select: need scores_out or a workspace");
    if (workspace_bytes < pasa_select_workspace_bytes(bh, num_blocks))
      return fail(PASA_ERR_WORKSPACE, "pasa_select: workspace %zu < %zu bytes", workspace_bytes, pasa_select_workspace_bytes(bh, num_blocks));
    scores = (float*)workspace;
  }
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 64 || head_dim == 128)
    rc = launch_status(pasa::launch_scores(qc, kc, hnorm, noise, (float)scale, use_cov_bias, scores, (int)bh,
                                           (int)num_blocks, (int)head_dim, s),
                       "pasa_select(scores)");
  else
    rc = launch_status(pasa::launch_scores_any(qc, kc, hnorm, noise, (float)scale, use_cov_bias, scores, (int)bh,
                                               (int)num_blocks, (int)head_dim, s),
                       "pasa_select(scores)");
  if (rc) return rc;
  return launch_status(pasa::launch_topk(scores, (int)bh, (int)num_blocks, (int)ns, idx, selmask, s),
                       "pasa_select(topk)");
}

int pasa_select_from_scores(const float* scores, int64_t ns, int32_t* idx, uint32_t* selmask,
                            int64_t bh, int64_t num_blocks, void* stream) {
  if (!scores || !selmask) return fail(PASA_ERR_NULL_POINTER, "pasa_select_from_scores: NULL pointer");
  int rc;
  if ((rc = check_select_shape(bh, num_blocks))) return rc;
  if (ns < 1 || ns > num_blocks) return fail(PASA_ERR_NUM_SELECTED, "ns=%lld not in [1, %lld]", (long long)ns, (long long)num_blocks);
  if ((rc = check_index_list(idx, num_blocks, ns))) return rc;
  return launch_status(pasa::launch_topk(scores, (int)bh, (int)num_blocks, (int)ns, idx, selmask, (hipStream_t)stream),
                       "pasa_select_from_scores");
}

size_t pasa_sparse_attn_workspace_bytes(int64_t bh, int64_t seq_len, int64_t text_len, int64_t head_dim,
                                        int64_t block_size, int64_t group_size) {
  if (bh <= 0 || seq_len <= 0 || text_len < 0 || text_len >= seq_len || (head_dim != 64 && head_dim != 128) ||
      (block_size != 64 && block_size != 128) || group_size != 32)
    return 0;
  const int64_t nt = cdiv(seq_len - text_len, block_size);
  const int64_t ng = cdiv(nt, group_size);
  return (size_t)bh * (size_t)ng * pasa::k4_pack_bytes((int)head_dim, (int)block_size);
}

static int check_attn_shape(int64_t bh, int64_t seq_len, int64_t text_len, int64_t head_dim,
                            int64_t block_size, int64_t group_size) {
  int rc;
  if ((rc = check_head_dim(head_dim))) return rc;
  if ((rc = check_block(block_size))) return rc;
  if ((rc = check_bh_seq(bh, seq_len, head_dim))) return rc;
  if ((rc = check_slice_bytes(seq_len, head_dim, 2))) return rc;
  if ((rc = check_text(seq_len, text_len, head_dim))) return rc;
  if (group_size != 32) return fail(PASA_ERR_GROUP_SIZE, "group_size %lld != 32", (long long)group_size);
  // text query tiles: at most one more than cdiv(text_len, block_size) (prompt and padding split)
  const int64_t grid = 8 * bh * cdiv(cdiv(seq_len - text_len, block_size), 8) +
                       8 * cdiv(bh * (cdiv(text_len, block_size) + 1), 8);
  if (grid > kMaxI32) return fail(PASA_ERR_OVERFLOW, "grid too large");
  return PASA_OK;
}

static int check_pack(const void* pack, size_t pack_bytes, int64_t bh, int64_t seq_len, int64_t text_len,
                      int64_t head_dim, int64_t block_size, int64_t group_size) {
  const size_t need = pasa_sparse_attn_workspace_bytes(bh, seq_len, text_len, head_dim, block_size, group_size);
  if (!pack || pack_bytes < need)
    return fail(PASA_ERR_WORKSPACE, "phase-2 pack buffer %zu < %zu bytes", pack ? pack_bytes : (size_t)0, need);
  return PASA_OK;
}

int pasa_pack_phase2(const float* kc, const float* vc, const float* hgroup, void* pack, size_t pack_bytes,
                     int64_t bh, int64_t seq_len, int64_t text_len, int64_t head_dim, int64_t block_size,
                     int64_t group_size, int dtype, void* stream) {
  if (!kc || !vc || !hgroup) return fail(PASA_ERR_NULL_POINTER, "pasa_pack_phase2: NULL pointer");
  int rc;
  if ((rc = check_attn_shape(bh, seq_len, text_len, head_dim, block_size, group_size))) return rc;
  if ((rc = check_attn_dtype(dtype, head_dim, "pasa_pack_phase2"))) return rc;
  if ((rc = check_pack(pack, pack_bytes, bh, seq_len, text_len, head_dim, block_size, group_size))) return rc;
  return launch_status(pasa::launch_pack_phase2(kc, vc, hgroup, pack, (int)bh, (int)(seq_len - text_len),
                                                (int)head_dim, (int)block_size, dtype == PASA_DTYPE_F16,
                                                (hipStream_t)stream),
                       "pasa_pack_phase2");
}

// idx is not read (the kernels visit the blocks of selmask), so it may be NULL.
// tuned: NULL for the packed entry points (the tuned shapes only); else receives whether
// the call runs on the tuned kernels or on the any-shape ones.
static int check_attn_args(const void* q, const void* k, const void* v, const int32_t* idx,
                           const uint32_t* selmask, const void* o, double scale, int64_t bh,
                           int64_t seq_len, int64_t text_len, int64_t text_valid, int64_t head_dim,
                           int64_t block_size, int64_t group_size, int64_t ns, int gamma_literal, int dtype,
                           bool* tuned = nullptr) {
  (void)idx;
  if (!q || !k || !v || !selmask || !o) return fail(PASA_ERR_NULL_POINTER, "pasa_sparse_attn: NULL pointer");
  int rc;
  if (tuned != nullptr && !tuned_attn_shape(dtype, head_dim, block_size, group_size, text_len)) {
    *tuned = false;
    if ((rc = check_any_dtype(dtype, "pasa_sparse_attn"))) return rc;
    if ((rc = check_any_shape(bh, seq_len, text_len, head_dim, block_size, group_size, "pasa_sparse_attn")))
      return rc;
    if (pasa::sparse_attn_any_tiles((int)(seq_len - text_len), (int)text_len, (int)text_len,
                                    (int)block_size) + 2 > kMaxI32)
      return fail(PASA_ERR_OVERFLOW, "grid too large");
  } else {
    if (tuned != nullptr) *tuned = true;
    if ((rc = check_attn_shape(bh, seq_len, text_len, head_dim, block_size, group_size))) return rc;
    if ((rc = check_attn_dtype(dtype, head_dim, "pasa_sparse_attn"))) return rc;
  }
  if (text_valid < 0 || text_valid > text_len)
    return fail(PASA_ERR_TEXT_SEGMENT, "text_valid=%lld must be in [0, text_len=%lld]", (long long)text_valid,
                (long long)text_len);
  const int64_t nt = cdiv(seq_len - text_len, block_size);
  if (ns < 1 || ns > nt) return fail(PASA_ERR_NUM_SELECTED, "ns=%lld not in [1, %lld]", (long long)ns, (long long)nt);
  if (nt > INT64_MAX / bh / ns) return fail(PASA_ERR_OVERFLOW, "bh*NT*ns overflows");
  if (!std::isfinite(scale) || !(scale > 0.0)) return fail(PASA_ERR_BAD_ARG, "scale must be finite and > 0");
  if (gamma_literal != 0 && gamma_literal != 1) return fail(PASA_ERR_BAD_ARG, "gamma_literal must be 0 or 1");
  return PASA_OK;
}

static int sparse_attn_packed_impl(const void* q, const void* k, const void* v, const void* pack,
                                   size_t pack_bytes, const int32_t* idx, const uint32_t* selmask, void* o,
                                   double scale, int64_t bh, int64_t seq_len, int64_t text_len, int64_t text_valid,
                                   int64_t head_dim, int64_t block_size, int64_t group_size, int64_t ns,
                                   int gamma_literal, int dtype, const pasa::RowMap* rm, void* stream) {
  int rc;
  if ((rc = check_attn_args(q, k, v, idx, selmask, o, scale, bh, seq_len, text_len, text_valid, head_dim,
                            block_size, group_size, ns, gamma_literal, dtype)))
    return rc;
  if ((rc = check_pack(pack, pack_bytes, bh, seq_len, text_len, head_dim, block_size, group_size))) return rc;
  return launch_status(pasa::launch_sparse_attn(q, k, v, pack, idx, selmask, o, (float)scale, (int)bh,
                                                (int)(seq_len - text_len), (int)text_len, (int)text_valid,
                                                (int)head_dim, (int)block_size, (int)ns, gamma_literal, rm,
                                                dtype == PASA_DTYPE_F16, (hipStream_t)stream),
                       "pasa_sparse_attn");
}

int pasa_sparse_attn_packed(const void* q, const void* k, const void* v, const void* pack, size_t pack_bytes,
                            const int32_t* idx, const uint32_t* selmask, void* o, double scale, int64_t bh,
                            int64_t seq_len, int64_t text_len, int64_t text_valid, int64_t head_dim,
                            int64_t block_size, int64_t group_size, int64_t ns, int gamma_literal, int dtype,
                            void* stream) {
  return sparse_attn_packed_impl(q, k, v, pack, pack_bytes, idx, selmask, o, scale, bh, seq_len, text_len,
                                 text_valid, head_dim, block_size, group_size, ns, gamma_literal, dtype, nullptr,
                                 stream);
}

int pasa_sparse_attn_packed_placed(const void* q, const void* k, const void* v, const void* pack,
                                   size_t pack_bytes, const int32_t* idx, const uint32_t* selmask, void* o,
                                   double scale, int64_t bh, int64_t seq_len, int64_t text_len, int64_t text_valid,
                                   int64_t head_dim, int64_t block_size, int64_t group_size, int64_t ns,
                                   int gamma_literal, const pasa_placement_t* placement, int dtype, void* stream) {
  pasa::RowMap rm;
  int rc;
  if ((rc = check_placement(placement, bh, seq_len, text_len, head_dim, block_size, &rm))) return rc;
  return sparse_attn_packed_impl(q, k, v, pack, pack_bytes, idx, selmask, o, scale, bh, seq_len, text_len,
                                 text_valid, head_dim, block_size, group_size, ns, gamma_literal, dtype, &rm, stream);
}

int pasa_sparse_attn(const void* q, const void* k, const void* v, const float* kc, const float* vc,
                     const float* hgroup, const int32_t* idx, const uint32_t* selmask, void* o,
                     double scale, int64_t bh, int64_t seq_len, int64_t text_len, int64_t text_valid,
                     int64_t head_dim, int64_t block_size, int64_t group_size, int64_t ns, int gamma_literal,
                     int dtype, void* workspace, size_t workspace_bytes, void* stream) {
  if (!kc || !vc || !hgroup) return fail(PASA_ERR_NULL_POINTER, "pasa_sparse_attn: NULL pointer");
  int rc;
  bool tuned = true;
  if ((rc = check_attn_args(q, k, v, idx, selmask, o, scale, bh, seq_len, text_len, text_valid, head_dim,
                            block_size, group_size, ns, gamma_literal, dtype, &tuned)))
    return rc;
  if (!tuned)  // the any-shape kernel reads kc, vc, hgroup directly: no workspace
    return launch_status(pasa::launch_sparse_attn_any(q, k, v, kc, vc, hgroup, selmask, o, (float)scale, (int)bh,
                                                      (int)(seq_len - text_len), (int)text_len, (int)text_valid,
                                                      (int)head_dim, (int)block_size, (int)group_size,
                                                      gamma_literal, 0, dtype, (hipStream_t)stream),
                         "pasa_sparse_attn");
  if ((rc = check_pack(workspace, workspace_bytes, bh, seq_len, text_len, head_dim, block_size, group_size)))
    return rc;
  if ((rc = pasa_pack_phase2(kc, vc, hgroup, workspace, workspace_bytes, bh, seq_len, text_len, head_dim,
                             block_size, group_size, dtype, stream)))
    return rc;
  return pasa_sparse_attn_packed(q, k, v, workspace, workspace_bytes, idx, selmask, o, scale, bh, seq_len,
                                 text_len, text_valid, head_dim, block_size, group_size, ns, gamma_literal,
                                 dtype, stream);
}

}  // extern "C"

// ---- the allocation-free attention entry ------------------------------------
//
// pasa_sparse_attn_noalloc keeps its phase-2 pack in `scratch`, one static device
// array per GPU that lives until the process ends.  In host code `scratch` names a
// host-side stand-in, not device memory, so kernels receive the address that
// hipGetSymbolAddress returns for the device the call runs on, looked up once per
// device (with that device current) and cached.  Every call on one device reuses
// that device's array: calls that overlap on one device race.  The pack kernel
// writes every byte K4 reads, so nothing has to be cleared between calls.
namespace {

constexpr size_t kScratchBytes = PASA_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device `stream` belongs to (the current device
// for the null stream).
int scratch_address(void* stream, void** out) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice((hipStream_t)stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return fail(PASA_ERR_LAUNCH, "pasa_sparse_attn_noalloc: device of the stream: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(PASA_ERR_BAD_ARG, "pasa_sparse_attn_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    if ((e = hipGetDevice(&cur)) != hipSuccess)
      return fail(PASA_ERR_LAUNCH, "pasa_sparse_attn_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return fail(PASA_ERR_LAUNCH, "pasa_sparse_attn_noalloc: hipSetDevice(%d): %s", dev, hipGetErrorString(e));
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess && e2 != hipSuccess) e = e2;
    }
    if (e != hipSuccess || p == nullptr)
      return fail(PASA_ERR_LAUNCH, "pasa_sparse_attn_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PASA_OK;
}

}  // namespace

extern "C" {

int pasa_sparse_attn_noalloc(const void* q, const void* k, const void* v, const float* kc, const float* vc,
                             const float* hgroup, const int32_t* idx, const uint32_t* selmask, void* o,
                             double scale, int64_t bh, int64_t seq_len, int64_t text_len, int64_t text_valid,
                             int64_t head_dim, int64_t block_size, int64_t group_size, int64_t ns,
                             int gamma_literal, int dtype, void* stream) {
  if (!kc || !vc || !hgroup) return fail(PASA_ERR_NULL_POINTER, "pasa_sparse_attn_noalloc: NULL pointer");
  int rc;
  bool tuned = true;
  if ((rc = check_attn_args(q, k, v, idx, selmask, o, scale, bh, seq_len, text_len, text_valid, head_dim,
                            block_size, group_size, ns, gamma_literal, dtype, &tuned)))
    return rc;
  if (!tuned)  // the any-shape kernel needs no scratch
    return launch_status(pasa::launch_sparse_attn_any(q, k, v, kc, vc, hgroup, selmask, o, (float)scale, (int)bh,
                                                      (int)(seq_len - text_len), (int)text_len, (int)text_valid,
                                                      (int)head_dim, (int)block_size, (int)group_size,
                                                      gamma_literal, 0, dtype, (hipStream_t)stream),
                         "pasa_sparse_attn_noalloc");
  const size_t need = pasa_sparse_attn_workspace_bytes(bh, seq_len, text_len, head_dim, block_size, group_size);
  if (need > kScratchBytes)
    return fail(PASA_ERR_WORKSPACE,
                "pasa_sparse_attn_noalloc: the phase-2 pack needs %zu bytes, more than the %zu-byte static scratch "
                "(call pasa_sparse_attn with a workspace instead)", need, kScratchBytes);
  void* pack = nullptr;
  if ((rc = scratch_address(stream, &pack))) return rc;
  if ((rc = pasa_pack_phase2(kc, vc, hgroup, pack, kScratchBytes, bh, seq_len, text_len, head_dim, block_size,
                             group_size, dtype, stream)))
    return rc;
  return pasa_sparse_attn_packed(q, k, v, pack, kScratchBytes, idx, selmask, o, scale, bh, seq_len, text_len,
                                 text_valid, head_dim, block_size, group_size, ns, gamma_literal, dtype, stream);
}

int pasa_dense_attn(const void* q, const void* k, const void* v, void* o, double scale, int64_t bh,
                    int64_t seq_len, int64_t text_len, int64_t text_valid, int64_t head_dim, int dtype,
                    void* stream) {
  if (!q || !k || !v || !o) return fail(PASA_ERR_NULL_POINTER, "pasa_dense_attn: NULL pointer");
  int rc;
  if (!(head_dim == 128 && (dtype == PASA_DTYPE_BF16 || dtype == PASA_DTYPE_F16))) {
    // fp32 inputs or head dims other than 128: the any-shape kernel with every block exact
    if ((rc = check_any_dtype(dtype, "pasa_dense_attn"))) return rc;
    if ((rc = check_any_shape(bh, seq_len, text_len, head_dim, 64, 1, "pasa_dense_attn"))) return rc;
    if (text_valid < 0 || text_valid > text_len)
      return fail(PASA_ERR_TEXT_SEGMENT, "text_valid=%lld must be in [0, text_len=%lld]", (long long)text_valid,
                  (long long)text_len);
    if (!std::isfinite(scale) || !(scale > 0.0)) return fail(PASA_ERR_BAD_ARG, "scale must be finite and > 0");
    if (pasa::sparse_attn_any_tiles((int)(seq_len - text_len), (int)text_len, (int)text_valid, 64) > kMaxI32)
      return fail(PASA_ERR_OVERFLOW, "grid too large");
    return launch_status(pasa::launch_sparse_attn_any(q, k, v, nullptr, nullptr, nullptr, nullptr, o, (float)scale,
                                                      (int)bh, (int)(seq_len - text_len), (int)text_len,
                                                      (int)text_valid, (int)head_dim, 64, 1, 1, 1, dtype,
                                                      (hipStream_t)stream),
                         "pasa_dense_attn");
  }
  if ((rc = check_attn_dtype(dtype, head_dim, "pasa_dense_attn"))) return rc;
  if ((rc = check_bh_seq(bh, seq_len, head_dim))) return rc;
  if ((rc = check_slice_bytes(seq_len, head_dim, 2))) return rc;
  if ((rc = check_text(seq_len, text_len, head_dim))) return rc;
  if (text_valid < 0 || text_valid > text_len)
    return fail(PASA_ERR_TEXT_SEGMENT, "text_valid=%lld must be in [0, text_len=%lld]", (long long)text_valid,
                (long long)text_len);
  if (!std::isfinite(scale) || !(scale > 0.0)) return fail(PASA_ERR_BAD_ARG, "scale must be finite and > 0");
  const int64_t grid = 8 * bh * cdiv(cdiv(seq_len - text_len, 128), 8) + 8 * cdiv(bh * (cdiv(text_len, 128) + 1), 8);
  if (grid > kMaxI32) return fail(PASA_ERR_OVERFLOW, "grid too large");
  return launch_status(pasa::launch_dense_attn(q, k, v, o, (float)scale, (int)bh, (int)(seq_len - text_len),
                                               (int)text_len, (int)text_valid, dtype == PASA_DTYPE_F16,
                                               (hipStream_t)stream),
                       "pasa_dense_attn");
}

int pasa_qkv_prologue(const void* xq, const void* xk, const void* xv, void* q, void* k, void* v,
                      const void* wq, const void* wk, int64_t batch, int64_t seq_len, int64_t heads,
                      int64_t head_dim, int in_layout, int out_layout, int64_t out_seq_len, int64_t out_row0,
                      int norm, int norm_rounding, double eps, const void* rope_cos, const void* rope_sin,
                      int rope, int64_t rope_rows, int dtype, void* stream) {
  const void* ins[3] = {xq, xk, xv};
  void* outs[3] = {q, k, v};
  bool any = false;
  for (int t = 0; t < 3; ++t) {
    if ((ins[t] == nullptr) != (outs[t] == nullptr))
      return fail(PASA_ERR_NULL_POINTER, "pasa_qkv_prologue: tensor %d has only one of input/output", t);
    any = any || ins[t] != nullptr;
  }
  if (!any) return fail(PASA_ERR_NULL_POINTER, "pasa_qkv_prologue: no tensor given");
  if (dtype != PASA_DTYPE_BF16) return fail(PASA_ERR_DTYPE, "pasa_qkv_prologue: only bf16 is supported");
  int rc;
  if ((rc = check_head_dim(head_dim))) return rc;
  if (batch <= 0 || seq_len <= 0 || heads <= 0 || out_seq_len <= 0)
    return fail(PASA_ERR_BAD_SHAPE, "batch, seq_len, heads and out_seq_len must be > 0");
  if (batch > 65535) return fail(PASA_ERR_BAD_SHAPE, "batch %lld > 65535", (long long)batch);
  if (heads * (head_dim / 8) > pasa::prologue_max_chunks())
    return fail(PASA_ERR_BAD_SHAPE, "heads*head_dim=%lld exceeds %d", (long long)(heads * head_dim),
                pasa::prologue_max_chunks() * 8);
  if (out_row0 < 0 || out_row0 > out_seq_len - seq_len)
    return fail(PASA_ERR_BAD_SHAPE, "rows [%lld, %lld) do not fit out_seq_len=%lld", (long long)out_row0,
                (long long)(out_row0 + seq_len), (long long)out_seq_len);
  if (seq_len > INT64_MAX / batch / heads / head_dim || out_seq_len > INT64_MAX / batch / heads / head_dim ||
      cdiv(cdiv(seq_len, 4), 8) * 24 > kMaxI32)
    return fail(PASA_ERR_OVERFLOW, "pasa_qkv_prologue: sizes overflow");
  if ((in_layout != PASA_LAYOUT_BHSD && in_layout != PASA_LAYOUT_BSHD) ||
      (out_layout != PASA_LAYOUT_BHSD && out_layout != PASA_LAYOUT_BSHD))
    return fail(PASA_ERR_BAD_ARG, "unknown layout");
  if (norm != PASA_NORM_NONE && norm != PASA_NORM_HEAD && norm != PASA_NORM_ROW)
    return fail(PASA_ERR_BAD_ARG, "unknown norm %d", norm);
  if (norm_rounding != PASA_NORM_ROUND_ONCE && norm_rounding != PASA_NORM_ROUND_TWICE)
    return fail(PASA_ERR_BAD_ARG, "unknown norm_rounding %d", norm_rounding);
  if (!std::isfinite(eps) || eps < 0.0) return fail(PASA_ERR_BAD_ARG, "eps must be finite and >= 0");
  if (norm != PASA_NORM_NONE && !wq && !wk)
    return fail(PASA_ERR_NULL_POINTER, "a norm needs at least one of wq, wk");
  if (rope != PASA_ROPE_NONE && rope != PASA_ROPE_COSSIN_F32 && rope != PASA_ROPE_COMPLEX_F64)
    return fail(PASA_ERR_BAD_ARG, "unknown rope %d", rope);
  if (rope != PASA_ROPE_NONE && (!rope_cos || !rope_sin))
    return fail(PASA_ERR_NULL_POINTER, "rope tables are NULL");
  if (rope != PASA_ROPE_NONE && (rope_rows < 0 || rope_rows > seq_len))
    return fail(PASA_ERR_BAD_SHAPE, "rope_rows=%lld not in [0, seq_len=%lld]", (long long)rope_rows,
                (long long)seq_len);
  for (int t = 0; t < 3; ++t)
    if (ins[t] && ins[t] == outs[t] && (in_layout != out_layout || out_seq_len != seq_len || out_row0 != 0))
      return fail(PASA_ERR_BAD_ARG, "in place (tensor %d) needs equal layouts, out_seq_len == seq_len and "
                  "out_row0 == 0", t);
  pasa::PrologueParams p{};
  const void* ws[3] = {wq, wk, nullptr};
  for (int t = 0; t < 3; ++t)
    p.t[t] = pasa::PrologueTensor{(const uint16_t*)ins[t], (uint16_t*)outs[t],
                                  norm != PASA_NORM_NONE ? (const uint16_t*)ws[t] : nullptr};
  p.cos = rope_cos;
  p.sin = rope_sin;
  p.B = batch;
  p.S = seq_len;
  p.H = heads;
  p.OS = out_seq_len;
  p.row0 = out_row0;
  p.rope_rows = rope != PASA_ROPE_NONE ? rope_rows : 0;
  p.D = (int)head_dim;
  p.in_bshd = in_layout == PASA_LAYOUT_BSHD;
  p.out_bshd = out_layout == PASA_LAYOUT_BSHD;
  p.norm = norm == PASA_NORM_HEAD ? pasa::kNormHead : (norm == PASA_NORM_ROW ? pasa::kNormRow : 0);
  p.round_twice = norm_rounding == PASA_NORM_ROUND_TWICE;
  p.rope = rope == PASA_ROPE_COSSIN_F32 ? pasa::kRopeCosSinF32 : (rope == PASA_ROPE_COMPLEX_F64 ? pasa::kRopeComplexF64 : 0);
  p.eps = (float)eps;
  return launch_status(pasa::launch_prologue(p, (hipStream_t)stream), "pasa_qkv_prologue");
}

int pasa_row_ops(const void* x, int x_dtype, const void* residual, int residual_dtype, const float* gate,
                 void* h_out, int h_dtype,
                 int layernorm, const void* weight, const void* bias, int wb_dtype, const float* scale,
                 const float* shift, void* y, int y_dtype, int64_t rows, int64_t cols, int64_t rows_per_batch,
                 int64_t param_stride, double eps, void* stream) {
  if (!x) return fail(PASA_ERR_NULL_POINTER, "pasa_row_ops: x is NULL");
  if (!residual && (gate || h_out))
    return fail(PASA_ERR_NULL_POINTER, "pasa_row_ops: gate / h_out need a residual");
  if (!residual && !y) return fail(PASA_ERR_NULL_POINTER, "pasa_row_ops: nothing to compute (residual and y NULL)");
  if (residual && !h_out && !y) return fail(PASA_ERR_NULL_POINTER, "pasa_row_ops: residual given but no output");
  if (!y && (layernorm || weight || bias || scale || shift))
    return fail(PASA_ERR_NULL_POINTER, "pasa_row_ops: stage B arguments given but y is NULL");
  if ((scale == nullptr) != (shift == nullptr))
    return fail(PASA_ERR_NULL_POINTER, "pasa_row_ops: scale and shift go together");
  auto fdt = [](int d) { return d == PASA_DTYPE_BF16 || d == PASA_DTYPE_F32; };
  if (!fdt(x_dtype) || !fdt(residual_dtype) || !fdt(h_dtype) || !fdt(y_dtype) || !fdt(wb_dtype))
    return fail(PASA_ERR_DTYPE, "pasa_row_ops: dtypes must be bf16 or fp32");
  if (rows <= 0 || cols <= 0 || rows_per_batch <= 0 || rows % rows_per_batch != 0)
    return fail(PASA_ERR_BAD_SHAPE, "pasa_row_ops: rows=%lld, cols=%lld, rows_per_batch=%lld", (long long)rows,
                (long long)cols, (long long)rows_per_batch);
  if (cols % 8 != 0 || cols > pasa::row_ops_max_cols())
    return fail(PASA_ERR_BAD_SHAPE, "pasa_row_ops: cols=%lld must be a multiple of 8 and <= %d", (long long)cols,
                pasa::row_ops_max_cols());
  if (param_stride < 0 || param_stride % 4 != 0 || (param_stride > 0 && param_stride < cols))
    return fail(PASA_ERR_BAD_SHAPE, "pasa_row_ops: param_stride=%lld must be 0 or a multiple of 4 >= cols",
                (long long)param_stride);
  if (rows > INT64_MAX / cols / 4 || cdiv(rows, 4) > kMaxI32 ||
      (param_stride > 0 && rows / rows_per_batch > INT64_MAX / param_stride / 4))
    return fail(PASA_ERR_OVERFLOW, "pasa_row_ops: sizes overflow");
  if (layernorm && (!std::isfinite(eps) || eps < 0.0))
    return fail(PASA_ERR_BAD_ARG, "pasa_row_ops: eps must be finite and >= 0");
  const void* ptrs[] = {x, residual, gate, h_out, weight, bias, scale, shift, y};
  for (const void* q : ptrs)
    if (q && ((uintptr_t)q & 15u))
      return fail(PASA_ERR_BAD_ARG, "pasa_row_ops: pointers must be 16-byte aligned");
  // Row buffers: overlapping ones must be the same pointer with the same dtype.
  struct Buf { const void* p; int dt; };
  const Buf bufs[4] = {{x, x_dtype}, {residual, residual_dtype}, {h_out, h_dtype}, {y, y_dtype}};
  for (int i = 0; i < 4; ++i)
    for (int j = i + 1; j < 4; ++j) {
      if (!bufs[i].p || !bufs[j].p) continue;
      const uintptr_t a = (uintptr_t)bufs[i].p, b = (uintptr_t)bufs[j].p;
      const uintptr_t na = (uintptr_t)(rows * cols * (bufs[i].dt == PASA_DTYPE_F32 ? 4 : 2));
      const uintptr_t nb = (uintptr_t)(rows * cols * (bufs[j].dt == PASA_DTYPE_F32 ? 4 : 2));
      const bool overlap = a < b + nb && b < a + na;
      if (overlap && (a != b || bufs[i].dt != bufs[j].dt))
        return fail(PASA_ERR_BAD_ARG, "pasa_row_ops: row buffers %d and %d overlap without being the same "
                    "buffer of the same dtype", i, j);
    }
  pasa::RowOpParams p{};
  p.x = x;
  p.r = residual;
  p.gate = gate;
  p.h = h_out;
  p.w = weight;
  p.b = bias;
  p.scale = scale;
  p.shift = shift;
  p.y = y;
  p.M = rows;
  p.rows_per_batch = rows_per_batch;
  p.param_stride = param_stride;
  p.N = (int)cols;
  p.x_f32 = x_dtype == PASA_DTYPE_F32;
  p.r_f32 = residual_dtype == PASA_DTYPE_F32;
  p.h_f32 = h_dtype == PASA_DTYPE_F32;
  p.wb_f32 = wb_dtype == PASA_DTYPE_F32;
  p.y_f32 = y_dtype == PASA_DTYPE_F32;
  p.ln = layernorm != 0;
  p.eps = (float)eps;
  return launch_status(pasa::launch_row_ops(p, (hipStream_t)stream), "pasa_row_ops");
}

}  // extern "C"
