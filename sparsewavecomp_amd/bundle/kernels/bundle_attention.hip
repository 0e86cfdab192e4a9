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

#if SW_HEAD_DIM % 64 == 0
// The 64 rows of a workgroup (one wave: the launch is one work-item per
// row, 64 per workgroup) as a tile on the fp32 matrix cores, when every
// row's column list is a prefix of the tile's last row's -- true for block
// masks, causal diagonal blocks included, whose blocks line up with the
// 64-row tiles.  Then the tile's scores are the dense products of its Q rows
// with the K^T columns of the last row's entries, 16 entries (a chunk) at a
// time: S^T = K_chunk Q^T with v_mfma_f32_16x16x4_f32, the gathered K^T
// columns as the A operand and four 16-row Q tiles as B operands, so that
// lane (i, g) holds row 16 R + i's scores at entries t0 + 4g .. t0 + 4g + 3.
// The check reads every column index of the tile once (coalesced, 8 rows
// per batch); a tile that fails it, or whose last row has more than
// kTileCols entries, computes each row by its own work-item.
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kKB = SW_HEAD_DIM / 64;
constexpr int kTileCols = 512;
constexpr int kCheckRows = 8; // rows whose columns one check batch loads

SW_KERNEL sparse_attention_scores(const int32_t *__restrict__ rowOffsets,
                                  const int32_t *__restrict__ columnIndices,
                                  const float *__restrict__ maskValues,
                                  const float *__restrict__ query,
                                  const float *__restrict__ transposedKey,
                                  float *__restrict__ scores) {
  __shared__ int32_t lcol[kTileCols]; // the last row's columns
  const int l = (int)__builtin_amdgcn_workitem_id_x();
  const int i = l & 15, g = l >> 4;
  const int r0 = blockIdx.x * 64;
  const int nt = SW_ROWS - r0 < 64 ? SW_ROWS - r0 : 64; // >= 1
  const int rr = r0 + (l < nt ? l : nt - 1);
  const int32_t rb = rowOffsets[rr];
  const int32_t rlen = l < nt ? rowOffsets[rr + 1] - rb : 0;
  const int32_t bl = __builtin_amdgcn_readlane(rb, nt - 1);
  const int32_t len_last = __builtin_amdgcn_readlane(rlen, nt - 1);
  bool ok = len_last <= kTileCols; // wave-uniform
  if (ok && len_last == 0) {
    // an empty last row: the tile is a prefix tile only when every row is
    // empty (and bl may then be the arrays' end, so nothing is loaded)
    ok = __builtin_amdgcn_ballot_w64(rlen > 0) == 0;
  } else if (ok) {
    // entries past the last row's end repeat its final column, so that a
    // chunk's lanes read valid columns without a check
    const int span = (len_last + 15) & ~15;
    for (int t = l; t < span; t += 64)
      lcol[t] = columnIndices[bl + (t < len_last ? t : len_last - 1)];
    __syncthreads();
    // every load unconditional, from a clamped valid position (a row's
    // last entry, or the last row's first for an empty row), so that no
    // branch splits a batch; the compare then selects the entries in range
    bool mine = rlen <= len_last;
    for (int i0 = 0; i0 < nt; i0 += kCheckRows) {
      int32_t x[kCheckRows][kTileCols / 64];
#pragma unroll
      for (int j = 0; j < kCheckRows; ++j) {
        const int row = i0 + j < nt ? i0 + j : nt - 1;
        const int32_t b = __builtin_amdgcn_readlane(rb, row);
        const int32_t n = __builtin_amdgcn_readlane(rlen, row);
#pragma unroll
        for (int u = 0; u < kTileCols / 64; ++u) {
          const int t = l + 64 * u;
          x[j][u] = columnIndices[n > 0 ? b + (t < n ? t : n - 1) : bl];
        }
      }
#pragma unroll
      for (int j = 0; j < kCheckRows; ++j) {
        const int row = i0 + j < nt ? i0 + j : nt - 1;
        const int32_t n = __builtin_amdgcn_readlane(rlen, row);
#pragma unroll
        for (int u = 0; u < kTileCols / 64; ++u) {
          const int t = l + 64 * u;
          mine &= !(t < n && t < len_last) || x[j][u] == lcol[t];
        }
      }
    }
    ok = __builtin_amdgcn_ballot_w64(!mine) == 0;
  }
  if (!ok) {
    if (r0 + l < SW_ROWS)
      scores_row(rowOffsets, columnIndices, maskValues, query, transposedKey,
                 scores, r0 + l);
    return;
  }
  // every row is a prefix of an empty last row: no entries, and lcol holds
  // no column to gather from
  if (len_last == 0)
    return;
  // row 16 R + i's first position and length, each 16-row tile's longest
  // row, and its Q rows (B operand of step st: elements 64 kb + 16 g + st)
  int32_t rbR[4], lenR[4], maxR[4];
  float qb[4][16 * kKB];
#pragma unroll
  for (int R = 0; R < 4; ++R) {
    const int src = 16 * R + i;
    rbR[R] = __builtin_amdgcn_ds_bpermute(src << 2, rb);
    lenR[R] = __builtin_amdgcn_ds_bpermute(src << 2, rlen);
    int m = lenR[R];
#pragma unroll
    for (int o = 1; o < 16; o <<= 1)
      m = max(m, __builtin_amdgcn_ds_bpermute((l ^ o) << 2, m));
    maxR[R] = __builtin_amdgcn_readlane(m, 16 * R);
    const int qr = r0 + src < SW_ROWS ? r0 + src : SW_ROWS - 1;
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        v4f v;
        __builtin_memcpy(&v,
                         query + (int64_t)qr * SW_HEAD_DIM + 64 * kb +
                             16 * g + 4 * u,
                         sizeof v);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          qb[R][16 * kb + 4 * u + e] = v[e];
      }
  }
  // one chunk's K^T gathers (A operand of step st: K^T[64 kb + 16 g + st]
  // at the column of entry t0 + i) and the mask values of the entries its
  // lanes store, each from a clamped valid position (selected afterwards),
  // so that no branch splits the loads
  auto load = [&](int t0, float (&a)[16 * kKB], float (&mv)[4][4])
      __attribute__((always_inline)) {
    const int64_t c = lcol[t0 + i];
#pragma unroll
    for (int kb = 0; kb < kKB; ++kb)
#pragma unroll
      for (int st = 0; st < 16; ++st)
        a[16 * kb + st] =
            transposedKey[(int64_t)(64 * kb + 16 * g + st) * SW_KEY_ROWS + c];
#pragma unroll
    for (int R = 0; R < 4; ++R)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int t = t0 + 4 * g + v;
        const int32_t p = lenR[R] > 0
                              ? rbR[R] + (t < lenR[R] ? t : lenR[R] - 1)
                              : bl;
        mv[R][v] = maskValues[p];
      }
  };
  // a chunk's products and its scores' stores (one 16-byte store when the
  // lane's four entries are all in its row)
  auto compute = [&](int t0, const float (&a)[16 * kKB],
                     const float (&mv)[4][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int R = 0; R < 4; ++R) {
      if (t0 >= maxR[R]) // wave-uniform
        continue;
      // two independent chains of products (even and odd steps)
      v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 16 * kKB; st += 2) {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[st], qb[R][st], acc0,
                                                    0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[st + 1], qb[R][st + 1],
                                                    acc1, 0, 0, 0);
      }
      const v4f acc = acc0 + acc1;
      v4f sc;
#pragma unroll
      for (int v = 0; v < 4; ++v)
        sc[v] = mv[R][v] * (float)SW_BETA + acc[v] * (float)SW_ALPHA;
      const int t = t0 + 4 * g;
      float *dst = scores + rbR[R] + t;
      if (t + 3 < lenR[R]) {
        __builtin_memcpy(dst, &sc, sizeof sc);
      } else {
#pragma unroll
        for (int v = 0; v < 3; ++v)
          if (t + v < lenR[R])
            dst[v] = sc[v];
      }
    }
  };
  // chunks in pairs, each buffer named (a runtime buffer index would put
  // the arrays behind indexed register moves): the next chunk's loads fly
  // over a chunk's products
  float a0[16 * kKB], a1[16 * kKB], m0[4][4], m1[4][4];
  load(0, a0, m0);
  for (int t0 = 0; t0 < len_last; t0 += 32) {
    if (t0 + 16 < len_last)
      load(t0 + 16, a1, m1);
    compute(t0, a0, m0);
    if (t0 + 16 >= len_last)
      break;
    if (t0 + 32 < len_last)
      load(t0 + 32, a0, m0);
    compute(t0 + 16, a1, m1);
  }
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
