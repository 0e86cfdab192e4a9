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
  if (sw_tile64::sddmm_tile64<float, SW_HEAD_DIM / 64, true, false>(
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
// exp(s - row maximum) or s / row sum, in place.  The exponential is the
// hardware base-2 exponential of (s - max) log2 e and the division one
// correctly rounded reciprocal of the row sum per row times each entry, as
// in the library's fused attention kernels: within the chain's probability
// bound (2^-24 |x log2 e| ln 2 relative for the product, 1.5 ulp for the
// reciprocal and multiply), against expf's 13 vector instructions and the
// IEEE division's 11 per entry, which left each of the launch's 128 waves
// (one per CU) issue-bound (configuration 5: exponentials 20.2 -> 13.2 us,
// division 16.3 -> 11.9 us).
#include "../../csrc/sw_device.h"
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
  // the row maximum, or the reciprocal of the row sum
  const float m = kExp ? SW_ROW_MAP_IN[r] : 1.0f / SW_ROW_MAP_IN[r];
  auto map = [m](float v) __attribute__((always_inline)) {
    return kExp ? swd::exp_by_exp2(v - m) : v * m;
  };
  const int32_t e = rowOffsets[r + 1];
  int32_t p = rowOffsets[r];
  for (; p + kRowDeep <= e; p += kRowDeep) {
    float v[kRowDeep];
#pragma unroll
    for (int u = 0; u < kRowDeep; ++u)
      v[u] = scores[p + u];
#pragma unroll
    for (int u = 0; u < kRowDeep; ++u)
      scores[p + u] = map(v[u]);
  }
  if (p < e) {
    float v[kRowDeep];
#pragma unroll
    for (int u = 0; u < kRowDeep; ++u)
      v[u] = scores[p + u < e ? p + u : e - 1];
#pragma unroll
    for (int u = 0; u < kRowDeep; ++u)
      if (p + u < e)
        scores[p + u] = map(v[u]);
  }
}
#endif
#elif SW_ATTENTION_ROLE == 6
#if SW_VALUE_COLS % 64 == 0
#include "../../csrc/sw_device.h"

// Row r's 64 output columns c0 .. c0 + 63 by one wave (lane l: column
// c0 + l): the row's column indices and probabilities are the same in
// every lane, so they come through scalar loads, kOutDeep entries at a
// time, and each lane gathers its V column; products are added in position
// order, as one work-item per element does.
constexpr int kOutDeep = 32;

__device__ __forceinline__ void output_row(
    const int32_t *__restrict__ rowOffsets,
    const int32_t *__restrict__ columnIndices,
    const float *__restrict__ scores, const float *__restrict__ value,
    float *__restrict__ output, int r, int c) {
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

// Rows r0 .. r0 + 15 (those below SW_ROWS), output columns nb .. nb + 63, by
// one wave on the matrix cores, when every row's columns are a prefix of
// the tile's last row's (block masks) and the last row holds 4 to
// kOutTileCols entries: C = P V over the last row's entries, 16 at a time
// (four v_mfma_f32_16x16x4_f32 steps per 16-column output tile), lane
// (i, g) supplying P[row i][t0 + 4g + st] (zero past row i's end) and lane
// (j, g) V[c_{t0+4g+st}][nb + 4j + n] for the four output tiles n, whose
// columns interleave (tile n's column j is output column nb + 4j + n) so
// that one 16-byte load of a V row feeds all four.  Each V row a chunk
// reads serves the tile's 16 rows (one wave per row and 64 columns read it
// once per row: 724 MB of V rows from L2 on configuration 5).  Returns
// false (nothing stored) for other tiles; every output stored is checked
// and a tile with an inf or NaN output returns false too, as an inf or NaN
// V row that a shorter row leaves out reaches that row as 0 * inf.
constexpr int kOutTileCols = 512;
constexpr int kOutSub = 2; // 16-entry chunks per load step (three in flight)

__device__ __forceinline__ bool output_tile16(
    const int32_t *__restrict__ rowOffsets,
    const int32_t *__restrict__ columnIndices,
    const float *__restrict__ scores, const float *__restrict__ value,
    float *__restrict__ output, int r0, int nb, int32_t *lcol) {
  using swd::at_bytes;
  using swd::v4f;
  typedef int v4i __attribute__((ext_vector_type(4)));
  const int l = __lane_id(), i = l & 15, g = l >> 4;
  const int nt = SW_ROWS - r0 < 16 ? SW_ROWS - r0 : 16;
  // lanes 0 .. nt hold rowOffsets[r0 .. r0 + nt] (one trip)
  const int32_t my_ro = rowOffsets[r0 + (l < nt ? l : nt)];
  const int32_t bl = __builtin_amdgcn_readlane(my_ro, nt - 1);
  const int32_t te = __builtin_amdgcn_readlane(my_ro, nt);
  const int32_t len_last = te - bl;
  if (len_last < 4 || len_last > kOutTileCols ||
      (int64_t)te > (int64_t)(UINT32_MAX / 4))
    return false;
  // row i's first position and length (lanes of rows past nt: length 0)
  const int ic = i < nt ? i : nt - 1;
  const int32_t ra = __builtin_amdgcn_ds_bpermute(ic << 2, my_ro);
  const int32_t la =
      i < nt ? __builtin_amdgcn_ds_bpermute((ic + 1) << 2, my_ro) - ra : 0;
  // the last row's columns in LDS, slots past its end repeating its final
  // column; then every row but the last against them: lane l compares
  // entries 4l .. 4l + 3 and 256 + 4l .. + 3, read as element-aligned
  // 16-byte windows from min(b + t, te - 4) (a window holding a compared
  // entry never moves: such a row ends at or before bl <= te - 4)
  {
    int32_t y[kOutTileCols / 64];
#pragma unroll
    for (int u = 0; u < kOutTileCols / 64; ++u) {
      const int t = l + 64 * u;
      y[u] = *at_bytes(columnIndices,
                       4u * (uint32_t)(bl + (t < len_last ? t : len_last - 1)));
    }
    v4i x[15][2];
#pragma unroll
    for (int j = 0; j < 15; ++j) {
      const int row = j < nt - 1 ? j : nt - 1;
      const int32_t b = __builtin_amdgcn_readlane(my_ro, row);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int32_t w = std::min(b + 4 * l + 256 * u, te - 4);
        __builtin_memcpy(&x[j][u], at_bytes(columnIndices, 4u * (uint32_t)w),
                         sizeof(v4i));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kOutTileCols / 64; ++u)
      lcol[l + 64 * u] = y[u];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    bool mine = true;
#pragma unroll
    for (int j = 0; j < 15; ++j) {
      const int row = j < nt - 1 ? j : nt - 1;
      const int32_t b = __builtin_amdgcn_readlane(my_ro, row);
      const int32_t n = __builtin_amdgcn_readlane(my_ro, row + 1) - b;
      mine &= n <= len_last;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int t = 4 * l + 256 * u;
        v4i ref;
        __builtin_memcpy(&ref, lcol + t, sizeof ref);
#pragma unroll
        for (int m = 0; m < 4; ++m)
          mine &= !(t + m < n) || x[j][u][m] == ref[m];
      }
    }
    if (__builtin_amdgcn_ballot_w64(!mine) != 0)
      return false;
  }
  // one step's operands (kOutSub 16-entry chunks): P for entries
  // t0 + 16h + 4g .. + 3 of row i (positions clamped into the row, or the
  // last row's first for an empty row; zero past the row), and the V rows
  // of those entries' columns
  auto load = [&](int t0, float (&a)[kOutSub][4], v4f (&bv)[kOutSub][4])
      __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < kOutSub; ++h)
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int t = t0 + 16 * h + 4 * g + st;
        const int32_t q = la > 0 ? ra + (t < la ? t : la - 1) : bl;
        a[h][st] = *at_bytes(scores, 4u * (uint32_t)q);
        const uint32_t c = lcol[t];
        bv[h][st] = *reinterpret_cast<const v4f *>(
            value + (int64_t)c * SW_VALUE_COLS + nb + 4 * i);
      }
  };
  v4f acc[4];
#pragma unroll
  for (int n = 0; n < 4; ++n)
    acc[n] = v4f{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int t0, const float (&a)[kOutSub][4],
                     const v4f (&bv)[kOutSub][4])
      __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < kOutSub; ++h)
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const float pa = t0 + 16 * h + 4 * g + st < la ? a[h][st] : 0.0f;
#pragma unroll
        for (int n = 0; n < 4; ++n)
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, bv[h][st][n],
                                                        acc[n], 0, 0, 0);
      }
  };
  // three steps in flight, every step's loads unconditional (steps past
  // the last re-read the last), each buffer named.  The loop body has no
  // exit between its three steps, so that it is one block and a scheduling
  // barrier after each step's loads keeps them where they are issued (the
  // scheduler sank the P loads to their products, and an exit between the
  // steps let the compiler move a step's loads past the next step's
  // products): up to two steps past the last are computed, with P zero (a
  // step's entries past the last row hold P = 0; an inf or NaN in the V row
  // they repeat makes the tile take the row-by-row path).
  constexpr int kStep = 16 * kOutSub;
  const int nch = (len_last + kStep - 1) / kStep; // steps
  auto t_of = [&](int k) __attribute__((always_inline)) {
    return kStep * (k < nch ? k : nch - 1);
  };
  float a0[kOutSub][4], a1[kOutSub][4], a2[kOutSub][4];
  v4f b0[kOutSub][4], b1[kOutSub][4], b2[kOutSub][4];
  load(t_of(0), a0, b0);
  load(t_of(1), a1, b1);
  for (int k = 0; k < nch; k += 3) {
    load(t_of(k + 2), a2, b2);
    __builtin_amdgcn_sched_barrier(0);
    compute(kStep * k, a0, b0);
    load(t_of(k + 3), a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    compute(kStep * (k + 1), a1, b1);
    load(t_of(k + 4), a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    compute(kStep * (k + 2), a2, b2);
  }
  // lane (j, g) holds C[4g + v][4j + n] in acc[n][v]
  bool nonfinite = false;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const v4f o = {acc[0][v], acc[1][v], acc[2][v], acc[3][v]};
    nonfinite |= !(__builtin_isfinite(o.x) && __builtin_isfinite(o.y) &&
                   __builtin_isfinite(o.z) && __builtin_isfinite(o.w));
    const int rr = 4 * g + v;
    if (rr < nt)
      *reinterpret_cast<v4f *>(output + (int64_t)(r0 + rr) * SW_VALUE_COLS +
                               nb + 4 * i) = o;
  }
  return __builtin_amdgcn_ballot_w64(nonfinite) == 0;
}

// The launch has one work-item per output element, 64 per workgroup: the
// first (SW_ROWS / 16) (SW_VALUE_COLS / 64) one-wave workgroups each take a
// 16-row tile of 64 output columns (XCD-spread, as workgroups are dealt to
// the XCDs in turn) and the rest return; a tile that is not a prefix tile
// is computed row by row by its wave.
SW_KERNEL sparse_attention_output(const int32_t *__restrict__ rowOffsets,
                                  const int32_t *__restrict__ columnIndices,
                                  const float *__restrict__ scores,
                                  const float *__restrict__ value,
                                  float *__restrict__ output) {
  constexpr int kBlocks = SW_VALUE_COLS / 64;
  constexpr int kTiles = (SW_ROWS + 15) / 16 * kBlocks;
  const int wv = blockIdx.x;
  if (wv >= kTiles)
    return;
  __shared__ int32_t lcol[kOutTileCols];
  const int r0 = wv / kBlocks * 16, nb = wv % kBlocks * 64;
  if (output_tile16(rowOffsets, columnIndices, scores, value, output, r0, nb,
                    lcol))
    return;
  const int nt = SW_ROWS - r0 < 16 ? SW_ROWS - r0 : 16;
  for (int r = r0; r < r0 + nt; ++r)
    output_row(rowOffsets, columnIndices, scores, value, output, r,
               nb + (int)__builtin_amdgcn_workitem_id_x());
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
