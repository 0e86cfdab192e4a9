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

__device__ __forceinline__ float maximumf(float a, float b) {
  if (a != a || b != b)
    return __builtin_nanf("");
  if (a == b)
    return __float_as_int(a) < 0 ? b : a;
  return a > b ? a : b;
}

#if SW_ATTENTION_ROLE == 1
SW_KERNEL sparse_attention_scores(const int32_t *__restrict__ rowOffsets,
                                  const int32_t *__restrict__ columnIndices,
                                  const float *__restrict__ maskValues,
                                  const float *__restrict__ query,
                                  const float *__restrict__ transposedKey,
                                  float *__restrict__ scores) {
  const int r = work_item();
  if (r >= SW_ROWS)
    return;
  const float *q = query + (int64_t)r * SW_HEAD_DIM;
  // four positions per step, sixteen terms of each dot in flight; every dot
  // is still added term by term in order
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
#elif SW_ATTENTION_ROLE == 2
SW_KERNEL sparse_attention_row_max(const int32_t *__restrict__ rowOffsets,
                                   const float *__restrict__ scores,
                                   float *__restrict__ rowMaximum) {
  const int r = work_item();
  if (r >= SW_ROWS)
    return;
  float m = -INFINITY;
  const int32_t e = rowOffsets[r + 1];
  int32_t p = rowOffsets[r];
  for (; p + kDeep <= e; p += kDeep) {
    float v[kDeep];
#pragma unroll
    for (int u = 0; u < kDeep; ++u)
      v[u] = scores[p + u];
#pragma unroll
    for (int u = 0; u < kDeep; ++u)
      m = maximumf(m, v[u]);
  }
  for (; p < e; ++p)
    m = maximumf(m, scores[p]);
  rowMaximum[r] = m;
}
#elif SW_ATTENTION_ROLE == 3
SW_KERNEL sparse_attention_exp(const int32_t *__restrict__ rowOffsets,
                               const float *__restrict__ rowMaximum,
                               float *scores) {
  const int r = work_item();
  if (r >= SW_ROWS)
    return;
  const float m = rowMaximum[r];
  const int32_t e = rowOffsets[r + 1];
  int32_t p = rowOffsets[r];
  for (; p + kDeep <= e; p += kDeep) {
    float v[kDeep];
#pragma unroll
    for (int u = 0; u < kDeep; ++u)
      v[u] = scores[p + u];
#pragma unroll
    for (int u = 0; u < kDeep; ++u)
      scores[p + u] = expf(v[u] - m);
  }
  for (; p < e; ++p)
    scores[p] = expf(scores[p] - m);
}
#elif SW_ATTENTION_ROLE == 4
SW_KERNEL sparse_attention_row_sum(const int32_t *__restrict__ rowOffsets,
                                   const float *__restrict__ scores,
                                   float *__restrict__ rowSum) {
  const int r = work_item();
  if (r >= SW_ROWS)
    return;
  float s = 0.0f;
  const int32_t e = rowOffsets[r + 1];
  int32_t p = rowOffsets[r];
  for (; p + kDeep <= e; p += kDeep) {
    float v[kDeep];
#pragma unroll
    for (int u = 0; u < kDeep; ++u)
      v[u] = scores[p + u];
#pragma unroll
    for (int u = 0; u < kDeep; ++u)
      s += v[u];
  }
  for (; p < e; ++p)
    s += scores[p];
  rowSum[r] = s;
}
#elif SW_ATTENTION_ROLE == 5
SW_KERNEL sparse_attention_normalize(const int32_t *__restrict__ rowOffsets,
                                     const float *__restrict__ rowSum,
                                     float *scores) {
  const int r = work_item();
  if (r >= SW_ROWS)
    return;
  const float s = rowSum[r];
  const int32_t e = rowOffsets[r + 1];
  int32_t p = rowOffsets[r];
  for (; p + kDeep <= e; p += kDeep) {
    float v[kDeep];
#pragma unroll
    for (int u = 0; u < kDeep; ++u)
      v[u] = scores[p + u];
#pragma unroll
    for (int u = 0; u < kDeep; ++u)
      scores[p + u] = v[u] / s;
  }
  for (; p < e; ++p)
    scores[p] = scores[p] / s;
}
#elif SW_ATTENTION_ROLE == 6
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
#else
#error "unknown SW_ATTENTION_ROLE"
#endif
