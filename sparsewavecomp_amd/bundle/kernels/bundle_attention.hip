// The six fixed-shape kernels of a sparse-attention lrrt bundle (gfx950).
//
// One kernel per compilation, selected by SW_ATTENTION_ROLE, with the stable
// entry-point names and argument lists of the reference bundle
// (tools/sparsewave-bundle/sparsewave_bundle_ir.py:25-81) and its math
// (examples/pytorch/integration/SparseAttentionToSparseWave.cpp:270-312):
//   1 sparse_attention_scores    (rowOffsets, columnIndices, maskValues,
//                                 query, transposedKey, scores)
//                                 scores = mask * beta + (q . k) * alpha
//   2 sparse_attention_row_max   (rowOffsets, scores, rowMaximum)
//   3 sparse_attention_exp       (rowOffsets, rowMaximum, scores)
//   4 sparse_attention_row_sum   (rowOffsets, scores, rowSum)
//   5 sparse_attention_normalize (rowOffsets, rowSum, scores)
//   6 sparse_attention_output    (rowOffsets, columnIndices, scores, value,
//                                 output)
// Baked shapes: SW_ROWS (query rows), SW_KEY_ROWS, SW_HEAD_DIM,
// SW_VALUE_COLS; SW_ALPHA / SW_BETA scale the scores.  Kernels 1-5 launch one
// work-item per row, kernel 6 one per output element (n = rows * value
// columns), both with the linear grid ceil_div(n, 64) * 64.  A work-item
// keeps kDeep of its row's entries (the scores kernel: four positions of
// sixteen terms) in flight per step.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#ifndef SW_ATTENTION_ROLE
#error "SW_ATTENTION_ROLE must be defined"
#endif

#define SW_KERNEL extern "C" __global__ __launch_bounds__(64) void

__device__ __forceinline__ int work_item() {
  return blockIdx.x * 64 + __builtin_amdgcn_workitem_id_x();
}

// Entries a work-item keeps in flight on its row (a row handled by one
// work-item is a chain of memory trips; values are still combined in
// position order).
constexpr int kDeep = 16;

// arith.maximumf: NaN if either operand is NaN, and +0 above -0 -- the
// IEEE 754-2019 maximum, one v_maximum_f32
__device__ __forceinline__ float maximumf(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}

#if SW_ATTENTION_ROLE == 1
// Row r's scores by one work-item: four positions of sixteen terms in
// flight, every dot added term by term in order.
__device__ __forceinline__ void scores_row(
    const int32_t *__restrict__ rowOffsets,
    const int32_t *__restrict__ columnIndices,
    const float *__restrict__ maskValues, const float *__restrict__ query,
    const float *__restrict__ transposedKey, float *__restrict__ scores,
    int r) {
  const float *q = query + (int64_t)r * SW_HEAD_DIM;
  constexpr int NP = 4;
  const int32_t e = rowOffsets[r + 1];
  for (int32_t p = rowOffsets[r]; p < e; p += NP) {
    int64_t c[NP];
    float dot[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      c[j] = columnIndices[p + j < e ? p + j : e - 1];
      dot[j] = 0.0f;
    }
    int i = 0;
    for (; i + kDeep <= SW_HEAD_DIM; i += kDeep) {
      float qv[kDeep], kv[NP][kDeep];
#pragma unroll
      for (int u = 0; u < kDeep; ++u)
        qv[u] = q[i + u];
#pragma unroll
      for (int j = 0; j < NP; ++j)
#pragma unroll
        for (int u = 0; u < kDeep; ++u)
          kv[j][u] = transposedKey[(int64_t)(i + u) * SW_KEY_ROWS + c[j]];
#pragma unroll
      for (int j = 0; j < NP; ++j)
#pragma unroll
        for (int u = 0; u < kDeep; ++u)
          dot[j] = __builtin_fmaf(qv[u], kv[j][u], dot[j]);
    }
    for (; i < SW_HEAD_DIM; ++i) {
#pragma unroll
      for (int j = 0; j < NP; ++j)
        dot[j] = __builtin_fmaf(
            q[i], transposedKey[(int64_t)i * SW_KEY_ROWS + c[j]], dot[j]);
    }
#pragma unroll
    for (int j = 0; j < NP; ++j)
      if (p + j < e)
        scores[p + j] =
            maskValues[p + j] * (float)SW_BETA + dot[j] * (float)SW_ALPHA;
  }
}

#if (SW_HEAD_DIM == 64 || SW_HEAD_DIM == 128) && \
    4LL * SW_HEAD_DIM * SW_KEY_ROWS <= 0xFFFFFFFFLL
// The workgroup's 64 rows (one wave: the launch is one work-item per row, 64
// per workgroup) as one matrix-core tile when they share the column prefix
// structure of block masks (the library's code, csrc/sw_sddmm_tile64.h,
// whose lane offsets into the transposed key fit 32 bits);
// otherwise each row by its own work-item.
#include "../../csrc/sw_sddmm_tile64.h"

SW_KERNEL sparse_attention_scores(const int32_t *__restrict__ rowOffsets,
                                  const int32_t *__restrict__ columnIndices,
                                  const float *__restrict__ maskValues,
                                  const float *__restrict__ query,
                                  const float *__restrict__ transposedKey,
                                  float *__restrict__ scores) {
  __shared__ int32_t lcol[sw_tile64::kTileCols];
  if (sw_tile64::sddmm_tile64<float, SW_HEAD_DIM / 64, true>(
          rowOffsets, columnIndices, maskValues, query, transposedKey, scores,
          SW_ROWS, SW_KEY_ROWS, (int64_t)blockIdx.x * 64, lcol,
          [](float mask, float dot) {
            return mask * (float)SW_BETA + dot * (float)SW_ALPHA;
          }))
    return;
  const int r = work_item();
  if (r < SW_ROWS)
    scores_row(rowOffsets, columnIndices, maskValues, query, transposedKey,
               scores, r);
}
#else
SW_KERNEL sparse_attention_scores(const int32_t *__restrict__ rowOffsets,
                                  const int32_t *__restrict__ columnIndices,
                                  const float *__restrict__ maskValues,
                                  const float *__restrict__ query,
                                  const float *__restrict__ transposedKey,
                                  float *__restrict__ scores) {
  const int r = work_item();
  if (r < SW_ROWS)
    scores_row(rowOffsets, columnIndices, maskValues, query, transposedKey,
               scores, r);
}
#endif
#elif SW_ATTENTION_ROLE >= 2 && SW_ATTENTION_ROLE <= 5
// The row kernels: one work-item per row, kRowDeep of its entries in flight
// per step; the row's last partial step loads kRowDeep entries too, from
// positions clamped to its last entry, and selects the ones in the row (no
// entry-by-entry tail, each entry of which would be a memory round trip).
constexpr int kRowDeep = 32;

#if SW_ATTENTION_ROLE == 2 || SW_ATTENTION_ROLE == 4
// row maximum (identity -inf, the NaN-propagating maximum) or row sum
// (identity 0, entries added in position order)
#if SW_ATTENTION_ROLE == 2
#define SW_ROW_REDUCE_NAME sparse_attention_row_max
#define SW_ROW_REDUCE_OUT rowMaximum
#else
#define SW_ROW_REDUCE_NAME sparse_attention_row_sum
#define SW_ROW_REDUCE_OUT rowSum
#endif
SW_KERNEL SW_ROW_REDUCE_NAME(const int32_t *__restrict__ rowOffsets,
                             const float *__restrict__ scores,
                             float *__restrict__ SW_ROW_REDUCE_OUT) {
  constexpr bool kMax = SW_ATTENTION_ROLE == 2;
  const int r = work_item();
  if (r >= SW_ROWS)
    return;
  float a = kMax ? -INFINITY : 0.0f;
  const int32_t e = rowOffsets[r + 1];
  int32_t p = rowOffsets[r];
  for (; p + kRowDeep <= e; p += kRowDeep) {
    float v[kRowDeep];
#pragma unroll
    for (int u = 0; u < kRowDeep; ++u)
      v[u] = scores[p + u];
#pragma unroll
    for (int u = 0; u < kRowDeep; ++u)
      a = kMax ? maximumf(a, v[u]) : a + v[u];
  }
  if (p < e) {
    float v[kRowDeep];
#pragma unroll
    for (int u = 0; u < kRowDeep; ++u)
      v[u] = scores[p + u < e ? p + u : e - 1];
#pragma unroll
    for (int u = 0; u < kRowDeep; ++u)
      if (kMax)
        a = p + u < e ? maximumf(a, v[u]) : a;
      else
        a = p + u < e ? a + v[u] : a;
  }
  SW_ROW_REDUCE_OUT[r] = a;
}
#else
// exp(s - row maximum) or s / row sum, in place
#if SW_ATTENTION_ROLE == 3
#define SW_ROW_MAP_NAME sparse_attention_exp
#define SW_ROW_MAP_IN rowMaximum
#else
#define SW_ROW_MAP_NAME sparse_attention_normalize
#define SW_ROW_MAP_IN rowSum
#endif
SW_KERNEL SW_ROW_MAP_NAME(const int32_t *__restrict__ rowOffsets,
                          const float *__restrict__ SW_ROW_MAP_IN,
                          float *scores) {
  constexpr bool kExp = SW_ATTENTION_ROLE == 3;
  const int r = work_item();
  if (r >= SW_ROWS)
    return;
  const float m = SW_ROW_MAP_IN[r];
  const int32_t e = rowOffsets[r + 1];
  int32_t p = rowOffsets[r];
  for (; p + kRowDeep <= e; p += kRowDeep) {
    float v[kRowDeep];
#pragma unroll
    for (int u = 0; u < kRowDeep; ++u)
      v[u] = scores[p + u];
#pragma unroll
    for (int u = 0; u < kRowDeep; ++u)
      scores[p + u] = kExp ? expf(v[u] - m) : v[u] / m;
  }
  if (p < e) {
    float v[kRowDeep];
#pragma unroll
    for (int u = 0; u < kRowDeep; ++u)
      v[u] = scores[p + u < e ? p + u : e - 1];
#pragma unroll
    for (int u = 0; u < kRowDeep; ++u)
      if (p + u < e)
        scores[p + u] = kExp ? expf(v[u] - m) : v[u] / m;
  }
}
#endif
#elif SW_ATTENTION_ROLE == 6
#if SW_VALUE_COLS % 64 == 0
// One wave per 64 output columns of one row (the launch is one work-item
// per output element): the row's column indices and probabilities are the
// same in every lane, so they come through scalar loads, kOutDeep entries
// at a time, and each lane gathers its V column; products are added in
// position order, as one work-item per element does.
constexpr int kOutDeep = 32;

SW_KERNEL sparse_attention_output(const int32_t *__restrict__ rowOffsets,
                                  const int32_t *__restrict__ columnIndices,
                                  const float *__restrict__ scores,
                                  const float *__restrict__ value,
                                  float *__restrict__ output) {
  const int e0 = blockIdx.x * 64; // the wave's first output element
  const int r = e0 / SW_VALUE_COLS;
  const int c = e0 - r * SW_VALUE_COLS + (int)__builtin_amdgcn_workitem_id_x();
  if (r >= SW_ROWS)
    return;
  const int32_t pe = rowOffsets[r + 1];
  int32_t p = rowOffsets[r];
  float acc = 0.0f;
  for (; p + kOutDeep <= pe; p += kOutDeep) {
    int32_t cc[kOutDeep];
    float sv[kOutDeep], vv[kOutDeep];
#pragma unroll
    for (int u = 0; u < kOutDeep; ++u) {
      cc[u] = columnIndices[p + u];
      sv[u] = scores[p + u];
    }
#pragma unroll
    for (int u = 0; u < kOutDeep; ++u)
      vv[u] = value[(int64_t)cc[u] * SW_VALUE_COLS + c];
#pragma unroll
    for (int u = 0; u < kOutDeep; ++u)
      acc = __builtin_fmaf(sv[u], vv[u], acc);
  }
  // the row's last partial step: positions clamped to its last entry, the
  // products past it skipped (selected, not multiplied by zero: V may hold
  // inf)
  if (p < pe) {
    int32_t cc[kOutDeep];
    float sv[kOutDeep], vv[kOutDeep];
#pragma unroll
    for (int u = 0; u < kOutDeep; ++u) {
      const int32_t q = p + u < pe ? p + u : pe - 1;
      cc[u] = columnIndices[q];
      sv[u] = scores[q];
    }
#pragma unroll
    for (int u = 0; u < kOutDeep; ++u)
      vv[u] = value[(int64_t)cc[u] * SW_VALUE_COLS + c];
#pragma unroll
    for (int u = 0; u < kOutDeep; ++u)
      acc = p + u < pe ? __builtin_fmaf(sv[u], vv[u], acc) : acc;
  }
  output[(int64_t)r * SW_VALUE_COLS + c] = acc;
}
#else
SW_KERNEL sparse_attention_output(const int32_t *__restrict__ rowOffsets,
                                  const int32_t *__restrict__ columnIndices,
                                  const float *__restrict__ scores,
                                  const float *__restrict__ value,
                                  float *__restrict__ output) {
  const int e = work_item();
  if (e >= SW_ROWS * SW_VALUE_COLS)
    return;
  const int r = e / SW_VALUE_COLS, c = e - r * SW_VALUE_COLS;
  float acc = 0.0f;
  const int32_t pe = rowOffsets[r + 1];
  int32_t p = rowOffsets[r];
  for (; p + kDeep <= pe; p += kDeep) {
    float sv[kDeep], vv[kDeep];
    int32_t cc[kDeep];
#pragma unroll
    for (int u = 0; u < kDeep; ++u) {
      sv[u] = scores[p + u];
      cc[u] = columnIndices[p + u];
    }
#pragma unroll
    for (int u = 0; u < kDeep; ++u)
      vv[u] = value[(int64_t)cc[u] * SW_VALUE_COLS + c];
#pragma unroll
    for (int u = 0; u < kDeep; ++u)
      acc = __builtin_fmaf(sv[u], vv[u], acc);
  }
  for (; p < pe; ++p)
    acc = __builtin_fmaf(scores[p],
                         value[(int64_t)columnIndices[p] * SW_VALUE_COLS + c],
                         acc);
  output[e] = acc;
}
#endif
#else
#error "unknown SW_ATTENTION_ROLE"
#endif
