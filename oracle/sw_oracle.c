/*
 * CPU oracle for the SparseWave sparse hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path (the HIP library,
 * the Python host mirror, the bundle tool) may link, load or call this file.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * it, and only as the checker or as the timed CPU baseline.
 *
 * Every function is a scalar, single-threaded restatement of the reference's
 * algorithm, in the reference's loop order, with an fp32 accumulator that
 * starts at zero and separate multiply and add (build with
 * -ffp-contract=off so the compiler does not fuse them).  Citations are
 * path:line into sott0n/SparseWaveComp.
 *
 * Parity pins (what checks each function; see tests/test_oracle.py):
 *   round_bf16 / bf16_to_f32: torch's float32 -> bfloat16 conversion on
 *       random, tie, subnormal, overflow and non-finite patterns, and hand
 *       cases (1 + 2^-8 -> 1, 1 + 3 * 2^-8 -> 1 + 2^-6).
 *   sparse_attention_bf16: a dense torch restatement of the six ops with
 *       torch's bf16 rounding between them, the golden attention vector
 *       within bf16 accuracy, and a mutation (one rounding left out) that
 *       the dense check catches.
 *   spmv / spmm / bsr / sddmm / row_reduce / rowwise_map / attention:
 *       golden vectors held by the reference's runtime tests, scipy.sparse
 *       and dense numpy closed forms on random inputs, mutation tests.
 *   row_at_position: numpy.searchsorted(side="right") - 1 on random CSR with
 *       empty rows, brute force on tiny inputs.
 *   position_space: coverage/disjointness/size invariants, brute force.
 *   spmv_wave_position: equals the row-space result within tolerance, and
 *       each emitted segment sum equals the row's sequential sum on tiny
 *       inputs (brute-force emulation of one wave).
 */
#include "sw_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Sequential CSR SpMV: y[r] = sum_p val[p] * x[col[p]], p in [ro[r], ro[r+1]).
 * Follows benchmark/SparseBenchmarkUtils.cpp:211-229 (loop order, fp32
 * accumulator from 0) generalised from x == 1 to a real vector, which is
 * exactly the per-row body of ThreadPerRowSpMVPattern
 * (lib/Dialect/SparseWave/Transforms/SparseWaveToGPU.cpp:216-274:
 * mulf then addf onto the running sum). */
void oracle_spmv_csr_f32(int64_t rows, const int32_t *ro, const int32_t *col,
                         const float *val, const float *x, float *y) {
  for (int64_t r = 0; r < rows; ++r) {
    float sum = 0.0f;
    for (int32_t p = ro[r]; p < ro[r + 1]; ++p) {
      float prod = val[p] * x[col[p]];
      sum = sum + prod;
    }
    y[r] = sum;
  }
}

/* Per-row magnitude bound sum_p |val[p] * x[col[p]]| in double: the scale of
 * the fp32 tolerance 1e-5 * sum|a_ij x_j| stated for the hot path. */
void oracle_spmv_abs_bound(int64_t rows, const int32_t *ro, const int32_t *col,
                           const float *val, const float *x, double *bound) {
  for (int64_t r = 0; r < rows; ++r) {
    double s = 0.0;
    for (int32_t p = ro[r]; p < ro[r + 1]; ++p)
      s += fabs((double)val[p] * (double)x[col[p]]);
    bound[r] = s;
  }
}

/* COO SpMV: output zeroed, then each stored entry adds its product to its
 * row in storage order (duplicates and any entry order allowed).  Body of
 * ThreadPerNonzeroCOOSpMVPattern (SparseWaveToGPU.cpp:154-214: zero-fill,
 * then `atomic addf (val[p] * x[col[p]])` per entry) run sequentially; the
 * loop order of the expected output in benchmark/SparseBenchmarkUtils.cpp:
 * 231-251.  Also writes the per-row magnitude bound sum |val * x| (double)
 * when `bound` is not NULL. */
void oracle_spmv_coo_f32(int64_t rows, int64_t nnz, const int32_t *ri,
                         const int32_t *ci, const float *val, const float *x,
                         float *y, double *bound) {
  for (int64_t r = 0; r < rows; ++r) {
    y[r] = 0.0f;
    if (bound)
      bound[r] = 0.0;
  }
  for (int64_t p = 0; p < nnz; ++p) {
    const float product = val[p] * x[ci[p]];
    y[ri[p]] += product;
    if (bound)
      bound[ri[p]] += fabs((double)product);
  }
}

/* CSR SpMM, row-major rhs[m][k] and out[n][k].
 * Loop order of benchmark/SparseBenchmarkUtils.cpp:277-288 (row, output
 * column, position), which is also the per-thread body of
 * ThreadPerOutputSpMMPattern (SparseWaveToGPU.cpp:489-558). */
void oracle_spmm_csr_f32(int64_t rows, int64_t k, const int32_t *ro,
                         const int32_t *col, const float *val,
                         const float *rhs, float *out) {
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < k; ++c) {
      float sum = 0.0f;
      for (int32_t p = ro[r]; p < ro[r + 1]; ++p) {
        float prod = val[p] * rhs[(int64_t)col[p] * k + c];
        sum = sum + prod;
      }
      out[r * k + c] = sum;
    }
  }
}

/* Per-output magnitude bound for SpMM: sum_p |val[p] * rhs[col[p]][c]|. */
void oracle_spmm_abs_bound(int64_t rows, int64_t k, const int32_t *ro,
                           const int32_t *col, const float *val,
                           const float *rhs, double *bound) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < k; ++c) {
      double s = 0.0;
      for (int32_t p = ro[r]; p < ro[r + 1]; ++p)
        s += fabs((double)val[p] * (double)rhs[(int64_t)col[p] * k + c]);
      bound[r * k + c] = s;
    }
}

/* BSR SpMM with square b x b blocks stored row-major as [nnzb][b][b].
 * Per output element: loop over the block row's blocks, then over the b
 * local columns, fp32 accumulator from 0.  Follows
 * ThreadPerOutputBSRSpMMPattern (SparseWaveToGPU.cpp:560-665); block layout
 * from include/sparsewave/Dialect/SparseWave/IR/SparseWaveOps.td:133-137. */
void oracle_bsr_spmm_f32(int64_t rows, int64_t k, int64_t b,
                         const int32_t *bro, const int32_t *bcol,
                         const float *bval, const float *rhs, float *out) {
  int64_t block_rows = rows / b;
  for (int64_t br = 0; br < block_rows; ++br)
    for (int64_t lr = 0; lr < b; ++lr) {
      int64_t r = br * b + lr;
      for (int64_t c = 0; c < k; ++c) {
        float sum = 0.0f;
        for (int32_t bp = bro[br]; bp < bro[br + 1]; ++bp) {
          const float *blk = bval + (int64_t)bp * b * b + lr * b;
          int64_t rbase = (int64_t)bcol[bp] * b;
          for (int64_t lc = 0; lc < b; ++lc) {
            float prod = blk[lc] * rhs[(rbase + lc) * k + c];
            sum = sum + prod;
          }
        }
        out[r * k + c] = sum;
      }
    }
}

/* Magnitude bound for BSR SpMM outputs (double). */
void oracle_bsr_abs_bound(int64_t rows, int64_t k, int64_t b,
                          const int32_t *bro, const int32_t *bcol,
                          const float *bval, const float *rhs, double *bound) {
  int64_t block_rows = rows / b;
  for (int64_t br = 0; br < block_rows; ++br)
    for (int64_t lr = 0; lr < b; ++lr) {
      int64_t r = br * b + lr;
      for (int64_t c = 0; c < k; ++c) {
        double s = 0.0;
        for (int32_t bp = bro[br]; bp < bro[br + 1]; ++bp) {
          const float *blk = bval + (int64_t)bp * b * b + lr * b;
          int64_t rbase = (int64_t)bcol[bp] * b;
          for (int64_t lc = 0; lc < b; ++lc)
            s += fabs((double)blk[lc] * (double)rhs[(rbase + lc) * k + c]);
        }
        bound[r * k + c] = s;
      }
    }
}

/* SDDMM: for every stored (r, c) at position p,
 *   dot = sum_{i<kdim} lhs[r][i] * rhs[i][c]   (sequential, fp32 from 0)
 *   out[p] = combine(val[p], dot)
 * ThreadPerRowSDDMMPattern (SparseWaveToGPU.cpp:667-750).  The scalar
 * region is one of the forms the reference emits:
 *   SW_ORACLE_SDDMM_MUL    sample * dot   (SparseWaveOps.td:178-183,
 *                          test/Dialect/SparseWave/sddmm-runtime.mlir)
 *   SW_ORACLE_SDDMM_AFFINE sample*beta + dot*alpha
 *                          (examples/pytorch/integration/
 *                           SparseAttentionToSparseWave.cpp:270-283)
 *   SW_ORACLE_SDDMM_DOT    dot */
void oracle_sddmm_csr_f32(int64_t rows, int64_t kdim, int64_t cols,
                          const int32_t *ro, const int32_t *col,
                          const float *val, const float *lhs,
                          const float *rhs, float *out, int kind, float alpha,
                          float beta) {
  for (int64_t r = 0; r < rows; ++r)
    for (int32_t p = ro[r]; p < ro[r + 1]; ++p) {
      int64_t c = col[p];
      float dot = 0.0f;
      for (int64_t i = 0; i < kdim; ++i) {
        float prod = lhs[r * kdim + i] * rhs[i * cols + c];
        dot = dot + prod;
      }
      float res;
      if (kind == SW_ORACLE_SDDMM_MUL) {
        res = val[p] * dot;
      } else if (kind == SW_ORACLE_SDDMM_AFFINE) {
        float s = val[p] * beta;
        float d = dot * alpha;
        res = s + d;
      } else {
        res = dot;
      }
      out[p] = res;
    }
}

/* arith.maximumf: NaN-propagating maximum (used by csr_row_reduce max). */
static float maximumf(float a, float b) {
  if (isnan(a) || isnan(b))
    return NAN;
  if (a == b && a == 0.0f)
    return signbit(a) ? b : a;
  return a > b ? a : b;
}

/* CSR row reduction: sum (identity 0) or max (identity -inf, maximumf).
 * ThreadPerRowCSRRowReducePattern (SparseWaveToGPU.cpp:752-818);
 * identities from SparseWaveOps.td:225-257. */
void oracle_csr_row_reduce_f32(int64_t rows, const int32_t *ro,
                               const float *val, float *out, int kind) {
  for (int64_t r = 0; r < rows; ++r) {
    float acc = kind == SW_ORACLE_REDUCE_SUM ? 0.0f : -INFINITY;
    for (int32_t p = ro[r]; p < ro[r + 1]; ++p)
      acc = kind == SW_ORACLE_REDUCE_SUM ? acc + val[p] : maximumf(acc, val[p]);
    out[r] = acc;
  }
}

/* CSR row-wise map: out[p] = f(val[p], row_values[r]).
 * ThreadPerRowCSRRowwiseMapPattern (SparseWaveToGPU.cpp:820-878).  Regions
 * the attention bundle emits (SparseAttentionToSparseWave.cpp:288-309):
 * exp(v - m) and v / s; sub and mul complete the elementwise family. */
void oracle_csr_rowwise_map_f32(int64_t rows, const int32_t *ro,
                                const float *val, const float *row_values,
                                float *out, int kind) {
  for (int64_t r = 0; r < rows; ++r) {
    float rv = row_values[r];
    for (int32_t p = ro[r]; p < ro[r + 1]; ++p) {
      float v = val[p];
      float res;
      switch (kind) {
      case SW_ORACLE_MAP_EXP_SUB:
        res = expf(v - rv);
        break;
      case SW_ORACLE_MAP_DIV:
        res = v / rv;
        break;
      case SW_ORACLE_MAP_SUB:
        res = v - rv;
        break;
      default:
        res = v * rv;
        break;
      }
      out[p] = res;
    }
  }
}

/* The six-kernel sparse attention chain in the order the reference emits it
 * (SparseAttentionToSparseWave.cpp:270-312): scores = sddmm(affine),
 * row_max, exp(s - max), row_sum, s / sum, output = spmm(scores, value).
 * transposed_key is [d][cols]; value is [cols][dv]. */
void oracle_sparse_attention_f32(int64_t rows, int64_t cols, int64_t d,
                                 int64_t dv, const int32_t *ro,
                                 const int32_t *col, const float *mask_values,
                                 const float *query,
                                 const float *transposed_key,
                                 const float *value, float *scores,
                                 float *row_max, float *row_sum, float *output,
                                 float alpha, float beta) {
  oracle_sddmm_csr_f32(rows, d, cols, ro, col, mask_values, query,
                       transposed_key, scores, SW_ORACLE_SDDMM_AFFINE, alpha,
                       beta);
  oracle_csr_row_reduce_f32(rows, ro, scores, row_max, SW_ORACLE_REDUCE_MAX);
  oracle_csr_rowwise_map_f32(rows, ro, scores, row_max, scores,
                             SW_ORACLE_MAP_EXP_SUB);
  oracle_csr_row_reduce_f32(rows, ro, scores, row_sum, SW_ORACLE_REDUCE_SUM);
  oracle_csr_rowwise_map_f32(rows, ro, scores, row_sum, scores,
                             SW_ORACLE_MAP_DIV);
  oracle_spmm_csr_f32(rows, dv, ro, col, scores, value, output);
}

/* fp32 -> bf16, round to nearest with ties to even: the 16 dropped low bits
 * of the binary32 pattern round the kept upper half (a carry may ripple into
 * the exponent, reaching infinity above the largest bf16), and a NaN keeps
 * its sign and becomes a quiet NaN.  This is the conversion the bf16 paths
 * apply once to every stored result (the bfloat16 format keeps the binary32
 * sign, exponent and the top 7 fraction bits). */
static uint16_t round_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u)
    return (uint16_t)((u >> 16) | 0x0040u);
  const uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

static float widen_bf16(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

void oracle_round_bf16(int64_t n, const float *in, uint16_t *out) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = round_bf16(in[i]);
}

void oracle_bf16_to_f32(int64_t n, const uint16_t *in, float *out) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = widen_bf16(in[i]);
}

/* A result as a bf16 buffer stores it (rounded, kept as its fp32 value). */
static void store_bf16(int64_t n, float *v) {
  for (int64_t i = 0; i < n; ++i)
    v[i] = widen_bf16(round_bf16(v[i]));
}

/* The six-op attention chain on bf16 buffers (the bf16 option of the
 * attention bundle): the ops of SparseAttentionToSparseWave.cpp:270-312 in
 * order, each computing in fp32 from its bf16 operands exactly as the fp32
 * restatements above do, and each storing its result rounded to bf16 -- the
 * scores after the SDDMM, the exponentials, the row sums, the normalised
 * scores and the output (a row maximum is one of its bf16 inputs, so it
 * needs no rounding).  Every input must already hold bf16 values; outputs
 * are returned as the fp32 values of their bf16 patterns.  The reference's
 * ops require one element type for all value operands
 * (SparseWaveOps.cpp:374-425); computing each op in fp32 rather than in the
 * element type is this build's stated choice. */
void oracle_sparse_attention_bf16(int64_t rows, int64_t cols, int64_t d,
                                  int64_t dv, const int32_t *ro,
                                  const int32_t *col, const float *mask_values,
                                  const float *query,
                                  const float *transposed_key,
                                  const float *value, float *scores,
                                  float *row_max, float *row_sum,
                                  float *output, float alpha, float beta) {
  const int64_t nnz = ro[rows];
  oracle_sddmm_csr_f32(rows, d, cols, ro, col, mask_values, query,
                       transposed_key, scores, SW_ORACLE_SDDMM_AFFINE, alpha,
                       beta);
  store_bf16(nnz, scores);
  oracle_csr_row_reduce_f32(rows, ro, scores, row_max, SW_ORACLE_REDUCE_MAX);
  oracle_csr_rowwise_map_f32(rows, ro, scores, row_max, scores,
                             SW_ORACLE_MAP_EXP_SUB);
  store_bf16(nnz, scores);
  oracle_csr_row_reduce_f32(rows, ro, scores, row_sum, SW_ORACLE_REDUCE_SUM);
  store_bf16(rows, row_sum);
  oracle_csr_rowwise_map_f32(rows, ro, scores, row_sum, scores,
                             SW_ORACLE_MAP_DIV);
  store_bf16(nnz, scores);
  oracle_spmm_csr_f32(rows, dv, ro, col, scores, value, output);
  store_bf16(rows * dv, output);
}

/* Row recovery for a CSR position: search [1, rows+1) of row_offsets for the
 * first offset greater than the position, then subtract one.  Exactly the
 * unsigned midpoint/select sequence of buildCSRRowSearch
 * (lib/Dialect/SparseWave/Transforms/SparsePositionToSCF.cpp:225-271). */
int64_t oracle_csr_row_at_position(int64_t rows, const int32_t *ro,
                                   int64_t position) {
  uint64_t lower = 1, upper = (uint64_t)rows + 1;
  while (lower < upper) {
    uint64_t mid = lower + (upper - lower) / 2;
    uint64_t off = (uint64_t)(int64_t)ro[mid];
    if (off <= (uint64_t)position)
      lower = mid + 1;
    else
      upper = mid;
  }
  return (int64_t)lower - 1;
}

void oracle_csr_rows_at_positions(int64_t rows, const int32_t *ro,
                                  int64_t count, const int64_t *positions,
                                  int32_t *out_rows) {
  for (int64_t i = 0; i < count; ++i)
    out_rows[i] = (int32_t)oracle_csr_row_at_position(rows, ro, positions[i]);
}

/* Balanced contiguous partition of [lower, upper) over worker_count workers:
 * begin = lower + w*base + min(w, rem), size = base + (w < rem).
 * LowerPositionSpacePattern (SparsePositionToSCF.cpp:190-223), contract in
 * SparseWaveOps.td:621-659. */
void oracle_position_space(int64_t lower, int64_t upper, int64_t worker,
                           int64_t worker_count, int64_t *begin,
                           int64_t *end) {
  uint64_t span = (uint64_t)(upper - lower);
  uint64_t base = span / (uint64_t)worker_count;
  uint64_t rem = span % (uint64_t)worker_count;
  uint64_t w = (uint64_t)worker;
  uint64_t before = w < rem ? w : rem;
  uint64_t b = (uint64_t)lower + (w * base + before);
  *begin = (int64_t)b;
  *end = (int64_t)(b + base + (w < rem ? 1u : 0u));
}

/* One wave of buildWavePrefixSegmentedReduction
 * (lib/Dialect/SparseWave/Transforms/SparseGPUUtils.cpp:247-292) emulated
 * lane by lane: shuffle-up by 1, 2, 4, ... < W on key and value; a lane adds
 * the shifted value when it is active, the source lane exists and the keys
 * are equal.  segment_end[l] = active[l] && !(next lane exists, is active and
 * has the same key).  Active lanes must form a prefix. */
void oracle_wave_segmented_scan(int wave, const int64_t *key,
                                const float *value_in, const uint8_t *active,
                                float *value_out, uint8_t *segment_end) {
  float cur[1024];
  float next[1024];
  for (int l = 0; l < wave; ++l)
    cur[l] = value_in[l];
  for (int off = 1; off < wave; off <<= 1) {
    for (int l = 0; l < wave; ++l) {
      int src = l - off;
      int combine = active[l] && src >= 0 && key[l] == key[src];
      next[l] = combine ? cur[l] + cur[src] : cur[l];
    }
    memcpy(cur, next, sizeof(float) * (size_t)wave);
  }
  for (int l = 0; l < wave; ++l) {
    value_out[l] = cur[l];
    int same_next = (l + 1 < wave) && active[l + 1] && key[l] == key[l + 1];
    segment_end[l] = (uint8_t)(active[l] && !same_next);
  }
}

/* wave-per-position SpMV with the reference's schedule, emulated serially:
 * zero the output (SparsePositionScheduling.cpp:31-47), G = max(ceil(nnz/B),1)
 * blocks and G*(B/W) waves (:337-352), wave w owns position_space(w) of
 * [0, nnz) (:357-360), lane l handles begin+l, row recovered by the row
 * search, product val*x, wave segmented scan, one atomic add per segment end
 * (:363-394).  Waves are applied in order, so the result is the one a GPU
 * produces when its atomics land in wave order. */
void oracle_spmv_wave_position_f32(int64_t rows, int64_t nnz,
                                   const int32_t *ro, const int32_t *col,
                                   const float *val, const float *x, float *y,
                                   int64_t block, int wave) {
  for (int64_t r = 0; r < rows; ++r)
    y[r] = 0.0f;
  int64_t grid = (nnz + block - 1) / block;
  if (grid < 1)
    grid = 1;
  int64_t waves = grid * (block / wave);
  int64_t key[1024];
  float v[1024], out[1024];
  uint8_t act[1024], seg[1024];
  for (int64_t w = 0; w < waves; ++w) {
    int64_t b, e;
    oracle_position_space(0, nnz, w, waves, &b, &e);
    for (int l = 0; l < wave; ++l) {
      int64_t p = b + l;
      act[l] = (uint8_t)(p < e);
      if (act[l]) {
        key[l] = oracle_csr_row_at_position(rows, ro, p);
        v[l] = val[p] * x[col[p]];
      } else {
        key[l] = 0;
        v[l] = 0.0f;
      }
    }
    oracle_wave_segmented_scan(wave, key, v, act, out, seg);
    for (int l = 0; l < wave; ++l)
      if (seg[l])
        y[key[l]] += out[l];
  }
}

/* Multi-threaded variant of oracle_spmv_csr_f32 for the labelled
 * all-cores CPU figure (same per-row arithmetic, rows split statically). */
#ifdef _OPENMP
#include <omp.h>
#endif
void oracle_spmv_csr_f32_mt(int64_t rows, const int32_t *ro,
                            const int32_t *col, const float *val,
                            const float *x, float *y) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t r = 0; r < rows; ++r) {
    float sum = 0.0f;
    for (int32_t p = ro[r]; p < ro[r + 1]; ++p) {
      float prod = val[p] * x[col[p]];
      sum = sum + prod;
    }
    y[r] = sum;
  }
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
