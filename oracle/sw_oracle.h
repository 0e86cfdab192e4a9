/* CPU oracle for the SparseWave sparse hot path -- test infrastructure only.
 * See sw_oracle.c for the reference citations and the parity pins. */
#ifndef SW_ORACLE_H
#define SW_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { SW_ORACLE_SDDMM_MUL = 0, SW_ORACLE_SDDMM_AFFINE = 1, SW_ORACLE_SDDMM_DOT = 2 };
enum { SW_ORACLE_REDUCE_SUM = 0, SW_ORACLE_REDUCE_MAX = 1 };
enum {
  SW_ORACLE_MAP_EXP_SUB = 0,
  SW_ORACLE_MAP_DIV = 1,
  SW_ORACLE_MAP_SUB = 2,
  SW_ORACLE_MAP_MUL = 3
};

void oracle_spmv_csr_f32(int64_t rows, const int32_t *ro, const int32_t *col,
                         const float *val, const float *x, float *y);
void oracle_spmv_csr_f32_mt(int64_t rows, const int32_t *ro,
                            const int32_t *col, const float *val,
                            const float *x, float *y);
int oracle_num_threads(void);
void oracle_spmv_abs_bound(int64_t rows, const int32_t *ro, const int32_t *col,
                           const float *val, const float *x, double *bound);
void oracle_spmv_coo_f32(int64_t rows, int64_t nnz, const int32_t *ri,
                         const int32_t *ci, const float *val, const float *x,
                         float *y, double *bound);
void oracle_spmm_csr_f32(int64_t rows, int64_t k, const int32_t *ro,
                         const int32_t *col, const float *val,
                         const float *rhs, float *out);
void oracle_spmm_abs_bound(int64_t rows, int64_t k, const int32_t *ro,
                           const int32_t *col, const float *val,
                           const float *rhs, double *bound);
void oracle_bsr_spmm_f32(int64_t rows, int64_t k, int64_t b,
                         const int32_t *bro, const int32_t *bcol,
                         const float *bval, const float *rhs, float *out);
void oracle_bsr_abs_bound(int64_t rows, int64_t k, int64_t b,
                          const int32_t *bro, const int32_t *bcol,
                          const float *bval, const float *rhs, double *bound);
void oracle_sddmm_csr_f32(int64_t rows, int64_t kdim, int64_t cols,
                          const int32_t *ro, const int32_t *col,
                          const float *val, const float *lhs,
                          const float *rhs, float *out, int kind, float alpha,
                          float beta);
void oracle_csr_row_reduce_f32(int64_t rows, const int32_t *ro,
                               const float *val, float *out, int kind);
void oracle_csr_rowwise_map_f32(int64_t rows, const int32_t *ro,
                                const float *val, const float *row_values,
                                float *out, int kind);
void oracle_sparse_attention_f32(int64_t rows, int64_t cols, int64_t d,
                                 int64_t dv, const int32_t *ro,
                                 const int32_t *col, const float *mask_values,
                                 const float *query,
                                 const float *transposed_key,
                                 const float *value, float *scores,
                                 float *row_max, float *row_sum, float *output,
                                 float alpha, float beta);
void oracle_round_bf16(int64_t n, const float *in, uint16_t *out);
void oracle_bf16_to_f32(int64_t n, const uint16_t *in, float *out);
void oracle_sparse_attention_bf16(int64_t rows, int64_t cols, int64_t d,
                                  int64_t dv, const int32_t *ro,
                                  const int32_t *col, const float *mask_values,
                                  const float *query,
                                  const float *transposed_key,
                                  const float *value, float *scores,
                                  float *row_max, float *row_sum,
                                  float *output, float alpha, float beta);
int64_t oracle_csr_row_at_position(int64_t rows, const int32_t *ro,
                                   int64_t position);
void oracle_csr_rows_at_positions(int64_t rows, const int32_t *ro,
                                  int64_t count, const int64_t *positions,
                                  int32_t *out_rows);
void oracle_position_space(int64_t lower, int64_t upper, int64_t worker,
                           int64_t worker_count, int64_t *begin, int64_t *end);
void oracle_wave_segmented_scan(int wave, const int64_t *key,
                                const float *value_in, const uint8_t *active,
                                float *value_out, uint8_t *segment_end);
void oracle_spmv_wave_position_f32(int64_t rows, int64_t nnz,
                                   const int32_t *ro, const int32_t *col,
                                   const float *val, const float *x, float *y,
                                   int64_t block, int wave);

#ifdef __cplusplus
}
#endif
#endif
