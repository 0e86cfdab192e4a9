// Host-side helpers shared by the launchers of the C ABI.
#pragma once

#include "../../include/sparsewave_amd.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <initializer_list>

namespace sw {

// Record a formatted message for sw_last_error() and return `code`.
int fail(int code, const char *fmt, ...);
void clear_error();

inline int hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess)
    return fail(SW_ERR_HIP, "%s failed: %s", what, hipGetErrorString(e));
  return SW_OK;
}

// After a kernel launch: report a launch-configuration error if any.
inline int launch_check(const char *kernel) {
  return hip_check(hipGetLastError(), kernel);
}

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// True when every byte offset into a dense operand of n rows of w floats
// fits 32 bits, so that kernels may address it as a wave-uniform base plus a
// 32-bit lane offset.
inline bool narrow_offsets(int64_t n, int64_t w) {
  return n >= 0 && w >= 0 && (w == 0 || n <= (int64_t)(UINT32_MAX / 4) / w);
}

// Grid limits.  The dispatch packet holds each dimension's work-item count
// in 32 bits, and a launch whose x dimension passes 2^32 - 1 work-items is
// cut short without an error (a thread-per-position SpMM over 2^31 - 2^16
// nonzeros at K = 4, 8.6e9 work-items, left its last rows unwritten).
// grid_dim therefore folds a 1-D launch of `blocks` workgroups of `threads`
// work-items into (x, y) when x alone cannot hold it; its kernels read their
// workgroup as swd::block_id() (y * gridDim.x + x), and the up to y - 1
// surplus workgroups of the last row return from their kernels' own index
// checks.  Below 2^32 work-items the grid stays 1-D, as before.
constexpr int64_t kMaxGridX = 2147483647;
constexpr int64_t kMaxGridY = 65535;

// Workgroups of `threads` work-items that one grid row (x) holds.
inline int64_t grid_row(int64_t threads) {
  const int64_t t = threads > 0 ? threads : 1;
  const int64_t n = (int64_t)UINT32_MAX / t;
  return n < kMaxGridX ? n : kMaxGridX;
}

inline dim3 grid_dim(int64_t blocks, int64_t threads) {
  const int64_t row = grid_row(threads);
  if (blocks <= row)
    return dim3((unsigned)blocks);
  const int64_t gy = ceil_div(blocks, row);
  return dim3((unsigned)ceil_div(blocks, gy), (unsigned)gy);
}

// A launch of `grid` workgroups of `threads` that grid_dim can fold.
inline int check_grid(int64_t grid, int64_t threads, const char *what) {
  if (grid > grid_row(threads) * kMaxGridY)
    return fail(SW_ERR_INVALID_SHAPE, "%s needs %lld workgroups, more than "
                "one launch allows", what, (long long)grid);
  return SW_OK;
}

// A launch whose kernel indexes its workgroups by blockIdx.x alone (a 1-D
// grid that is never folded, or the x dimension of a 2-D one).
inline int check_flat_grid(int64_t grid, int64_t threads, const char *what) {
  if (grid > grid_row(threads))
    return fail(SW_ERR_INVALID_SHAPE, "%s needs %lld workgroups of %lld "
                "work-items, more than one grid dimension holds", what,
                (long long)grid, (long long)threads);
  return SW_OK;
}

// Validate options, or use defaults when `opts` is NULL.
inline int resolve_options(const sw_options *opts, sw_options *out) {
  if (opts) {
    *out = *opts;
  } else {
    sw_options_init(out);
  }
  return sw_validate_options(out);
}

inline bool streq(const char *a, const char *b) { return std::strcmp(a, b) == 0; }

// Every value buffer must be aligned to its element (2 bytes for bf16, 4 for
// fp32) on every path, whatever the options: a kernel may take any buffer as
// a whole element, so an odd bf16 address is rejected before any launch.
inline int check_value_alignment(size_t elem,
                                 std::initializer_list<const void *> ptrs) {
  for (const void *p : ptrs)
    if (p && (reinterpret_cast<uintptr_t>(p) & (elem - 1)) != 0)
      return fail(SW_ERR_INVALID_ARGUMENT,
                  "a value buffer is not aligned to its %zu-byte element",
                  elem);
  return SW_OK;
}

// The SpMM position mappings add partial sums into the output across
// workgroups, which a bf16 output cannot hold.  Checked before the first
// launch of every entry point that ends in a bf16 SpMM (the SpMM itself and
// the attention chain), so a rejected call leaves every buffer untouched.
inline int check_bf16_spmm_mapping(const sw_options &o) {
  if (streq(o.spmm_mapping, "thread-per-position") ||
      streq(o.spmm_mapping, "wave-per-position"))
    return fail(SW_ERR_INVALID_OPTION,
                "spmm-mapping=%s adds partial sums into the output across "
                "workgroups, which a bf16 output cannot hold; bf16 takes "
                "thread-per-output, wave-per-row-tile, wave-per-row-balanced "
                "or row-tile-mfma",
                o.spmm_mapping);
  return SW_OK;
}

// Largest nnz a CSR operand may have.  Row loops step a position index past
// the row's end by less than one step (at most 16 positions for each of up
// to 1024 threads), so with nnz below INT32_MAX - 2^16 every position a
// kernel computes in int32 stays in range.
constexpr int64_t kMaxCsrNnz = (int64_t)INT32_MAX - 65536;

// CSR shape checks mirroring verifyCSRStorage
// (lib/Dialect/SparseWave/IR/SparseWaveOps.cpp:62-109): rows >= 0,
// nnz within the i32 index range, and non-null arrays where data exists.
inline int check_csr(const int32_t *ro, const int32_t *col, const void *val,
                     int64_t rows, int64_t nnz, bool need_col) {
  if (rows < 0 || nnz < 0)
    return fail(SW_ERR_INVALID_SHAPE,
                "expected non-negative rows and nnz, but got %lld and %lld",
                (long long)rows, (long long)nnz);
  if (rows > INT32_MAX - 1 || nnz > kMaxCsrNnz)
    return fail(SW_ERR_INVALID_SHAPE,
                "i32 CSR indices cannot address %lld rows / %lld nonzeros "
                "(at most %lld nonzeros)",
                (long long)rows, (long long)nnz, (long long)kMaxCsrNnz);
  if (!ro)
    return fail(SW_ERR_INVALID_ARGUMENT, "row offsets pointer is null");
  if (nnz > 0 && ((need_col && !col) || !val))
    return fail(SW_ERR_INVALID_ARGUMENT,
                "column index or value pointer is null");
  return SW_OK;
}

} // namespace sw
