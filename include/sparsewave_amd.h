/*
 * sparsewave_amd.h -- C ABI of the MI355X (gfx950, Wave64) SparseWave hot path.
 *
 * Plain pointers and sizes only.  Every pointer argument is a device pointer
 * (hipMalloc / torch CUDA tensor memory) unless stated otherwise; the caller
 * owns every buffer, outputs included.  All work is enqueued on `stream`
 * (a hipStream_t passed as void*, NULL = the default stream) with no host
 * synchronisation and no allocation.  Functions return SW_OK (0) or a
 * negative SW_ERR_* code; sw_last_error() then returns a message that
 * paraphrases the reference's diagnostic.  Index arrays are i32, values f32
 * (bf16 where the name says so).
 *
 * bf16 entry points (_bf16): every value buffer of the op -- inputs and
 * outputs alike -- holds bf16 as raw 16-bit patterns (uint16_t), because
 * the reference's ops require one element type for all of their value
 * operands (SparseWaveOps.cpp:340-372 for bsr_spmm, :374-425 for sddmm, and
 * the same rule for spmm, csr_row_reduce and csr_rowwise_map).  Kernels
 * widen to fp32, accumulate in fp32 (on the matrix cores where the name of
 * the mapping says mfma) and round each stored result to nearest even once.
 * The reference's own lowering of a bf16 op would also accumulate in bf16;
 * fp32 accumulation is the more accurate choice and parity with the fp32
 * path is tolerance-based (rel-L2 <= 1e-2).
 *
 * Sizes: CSR operands take nnz <= INT32_MAX - 65536 and rows <= INT32_MAX - 1
 * (larger: SW_ERR_INVALID_SHAPE before any launch); COO takes any nnz.
 * Every mapping runs at those limits: a launch of more than 2^32 - 1
 * work-items, which one grid dimension cannot hold, is folded into a 2-D
 * grid, and the BSR SpMM past about 8.4 million block rows computes with
 * its thread-per-output kernel.
 *
 * Citations are path:line into the reference (sott0n/SparseWaveComp).
 */
#ifndef SPARSEWAVE_AMD_H
#define SPARSEWAVE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SW_OK 0
#define SW_ERR_INVALID_OPTION (-1)   /* option value rejected */
#define SW_ERR_INVALID_SHAPE (-2)    /* shapes inconsistent with the op */
#define SW_ERR_INVALID_ARGUMENT (-3) /* null pointer, misaligned, bad kind */
#define SW_ERR_HIP (-4)              /* a HIP runtime call failed */

/*
 * Lowering options.  Field names are the reference's option names with '-'
 * replaced by '_' (sparsewave-to-amdgpu-pipeline,
 * include/sparsewave/Target/AMDGPU/Pipelines.h:108-191, and
 * convert-sparsewave-to-gpu,
 * include/sparsewave/Dialect/SparseWave/Transforms/Passes.td:186-241).
 * Defaults (sw_options_init) are the reference defaults except
 * wavefront_size, which is 64 because gfx950 runs Wave64 only.
 * The last block of fields is specific to this Wave64 build.
 */
typedef struct sw_options {
  char spmv_mapping[32];            /* thread-per-row | wave-per-row | block-per-row |
                                       thread-per-position | wave-per-position |
                                       wave-per-row-balanced (Wave64 extension:
                                       each row summed whole by the wave whose
                                       nonzero chunk holds its first position;
                                       no atomics, bit-identical repeats) */
  int64_t spmv_block_size;          /* 1..1024, default 256 */
  int64_t spmv_position_chunk_size; /* thread-per-position chunk, default 1 */
  char spmv_position_reduction[16]; /* atomic | segmented (thread-per-position) */
  int64_t position_block_size;      /* position-parallel init kernels, default 256 */
  char spmm_mapping[32];            /* thread-per-output | wave-per-row-tile |
                                       thread-per-position | wave-per-position |
                                       row-tile-mfma | wave-per-row-balanced |
                                       wave-per-row-tile-lds (the last four
                                       are Wave64 extensions; -lds stages the
                                       RHS rows in LDS) */
  int64_t spmm_block_size;          /* 1..1024, default 256 */
  int64_t spmm_tile_size;           /* 1..32, default 4 */
  int64_t spmm_position_chunk_size; /* default 1 */
  int64_t sddmm_block_size;         /* default 256 */
  int64_t row_reduction_block_size; /* default 256 */
  int64_t rowwise_map_block_size;   /* default 256 */
  int64_t elementwise_block_size;   /* default 256 (accepted, no op uses it) */
  int64_t wavefront_size;           /* must be 64 */
  /* Wave64 extensions (no reference counterpart). */
  int64_t spmv_lanes_per_row;       /* wave-per-row: lanes per row group,
                                       power of two 1..64, default 64 = one
                                       wave per row */
  int64_t spmv_positions_per_lane;  /* wave-per-position: consecutive
                                       positions per lane 1,2,4,8,16;
                                       default 1 = the reference schedule */
  int64_t spmm_lanes_per_row;       /* wave-per-row-tile: lanes per (row,
                                       tile) group, power of two, default 64 */
  int64_t bsr_use_mfma;             /* BSR SpMM: 1 = MFMA tiles when the block
                                       size allows it (default), 0 = the
                                       thread-per-output kernel */
  int64_t sddmm_lanes_per_row;      /* SDDMM: 1 = thread-per-row (reference,
                                       default); 64 = one wave per row with
                                       lanes split over the dot products */
  int64_t spmm_positions_per_lane;  /* SpMM wave-per-position: consecutive
                                       positions per lane group 1,2,4,8,16;
                                       default 4 */
  char sddmm_mapping[32];           /* thread-per-row (reference, default) |
                                       wave-per-row | row-tile-mfma (16-row
                                       tiles on the matrix cores; tiles whose
                                       rows do not share column structure,
                                       and kdim not in {64,128,256}, use the
                                       vector path) */
} sw_options;

/* Fill `opts` with the defaults. */
void sw_options_init(sw_options *opts);

/* Set one option by its reference name, e.g. ("spmv-mapping",
 * "wave-per-row") or ("spmv-block-size", "128").  Unknown names are
 * SW_ERR_INVALID_OPTION.  Target options of the reference pipeline
 * (chip, wavefront-size, rocm-path, ...) are accepted; chip must name
 * gfx950. */
int sw_options_set(sw_options *opts, const char *name, const char *value);

/* Parse a reference pipeline option string: whitespace separated name=value
 * pairs, optionally wrapped in the pass name and braces, e.g.
 * "sparsewave-to-amdgpu-pipeline{chip=gfx950 spmv-mapping=wave-per-row}". */
int sw_options_parse(sw_options *opts, const char *text);

/* Check option values the way convert-sparsewave-to-gpu and
 * schedule-sparsewave-position do
 * (lib/Dialect/SparseWave/Transforms/SparseWaveToGPU.cpp:1265-1397,
 *  lib/Dialect/SparseWave/Transforms/SparsePositionScheduling.cpp:411-465),
 * with the Wave32 requirements restated for Wave64. */
int sw_validate_options(const sw_options *opts);

/* Message of the last failing call on this thread ("" if none). */
const char *sw_last_error(void);

/* Library version string. */
const char *sw_version(void);

/*
 * sparsewave.spmv: output[rows] = A * vector with A in CSR.
 * Operands in op order (SparseWaveOps.td:17-52): row_offsets[rows+1],
 * column_indices[nnz], values[nnz], vector[cols], output[rows].
 * Replaces the kernels generated by ThreadPerRowSpMVPattern,
 * WavePerRowSpMVPattern, BlockPerRowSpMVPattern (SparseWaveToGPU.cpp:216-487)
 * and the position schedules (SparsePositionScheduling.cpp:135-403),
 * selected by opts->spmv_mapping.  Row mappings overwrite output; position
 * mappings zero it first (the reference's init kernel) then accumulate.
 */
int sw_spmv_csr_f32(const int32_t *row_offsets, const int32_t *column_indices,
                    const float *values, const float *vector, float *output,
                    int64_t rows, int64_t cols, int64_t nnz,
                    const sw_options *opts, void *stream);

/*
 * sparsewave.coo_spmv: output[rows] = A * vector with A in COO form.
 * Operands in op order (SparseWaveOps.td:54-88): row_indices[nnz],
 * column_indices[nnz], values[nnz], vector[cols], output[rows]; entries in
 * any order, repeated coordinates add up.  The output is zeroed, then
 * accumulated.  Replaces ThreadPerNonzeroCOOSpMVPattern
 * (SparseWaveToGPU.cpp:154-214), which reads only spmv-block-size; with
 * spmv-mapping=wave-per-position a run-segmented kernel (one atomic per run
 * of equal adjacent rows, spmv-positions-per-lane entries per lane) is used
 * instead.
 */
int sw_spmv_coo_f32(const int32_t *row_indices, const int32_t *column_indices,
                    const float *values, const float *vector, float *output,
                    int64_t rows, int64_t cols, int64_t nnz,
                    const sw_options *opts, void *stream);

/*
 * Gather floor, a diagnostic with no counterpart in the reference: reads
 * column_indices[nnz] and values[nnz] once and gathers vector[col] once per
 * entry, with no row structure, and writes
 * partial[w] = sum of values[p] * vector[column_indices[p]] over
 * p in [512 w, 512 w + 512) for w < ceil(nnz / 512).  Its time is the floor
 * under any CSR SpMV schedule that reads each nonzero and gathers x once;
 * bench.py reports the headline SpMV against it.
 */
int sw_spmv_gather_floor_f32(const int32_t *column_indices,
                             const float *values, const float *vector,
                             float *partial, int64_t nnz, void *stream);

/*
 * sparsewave.spmm: output[rows][k] = A * rhs[cols][k], dense matrices
 * row-major.  Operand order and the 5-buffer bundle ABI of
 * SparseWaveOps.td:91-124 / tools/sparsewave-bundle/sparsewave_bundle_ir.py:11-17.
 * Kernels of ThreadPerOutputSpMMPattern and WavePerRowTileSpMMPattern
 * (SparseWaveToGPU.cpp:489-558, 1057-1256) and the thread-per-position
 * schedule (PositionSpMMDecomposition.cpp:19-73).
 */
int sw_spmm_csr_f32(const int32_t *row_offsets, const int32_t *column_indices,
                    const float *values, const float *rhs, float *output,
                    int64_t rows, int64_t cols, int64_t nnz, int64_t k,
                    const sw_options *opts, void *stream);

/* sparsewave.spmm on bf16 memrefs (values, rhs and output bf16), the output
 * SpMM of the bf16 attention chain.  Mappings thread-per-output,
 * wave-per-row-tile, wave-per-row-balanced and row-tile-mfma (bf16 matrix
 * cores when k % 64 == 0); thread-per-position and wave-per-position add
 * partial sums into the output and are rejected with
 * SW_ERR_INVALID_OPTION. */
int sw_spmm_csr_bf16(const int32_t *row_offsets,
                     const int32_t *column_indices, const uint16_t *values,
                     const uint16_t *rhs, uint16_t *output, int64_t rows,
                     int64_t cols, int64_t nnz, int64_t k,
                     const sw_options *opts, void *stream);

/*
 * sparsewave.bsr_spmm: output[rows][k] = A * rhs[cols][k], A in BSR with
 * square block_size blocks stored row-major [nnzb][b][b]
 * (SparseWaveOps.td:126-169; verifier SparseWaveOps.cpp:144-207,340-372;
 * kernel ThreadPerOutputBSRSpMMPattern, SparseWaveToGPU.cpp:560-665).
 * rows and cols must be divisible by block_size.
 */
int sw_bsr_spmm_f32(const int32_t *block_row_offsets,
                    const int32_t *block_column_indices,
                    const float *block_values, const float *rhs, float *output,
                    int64_t rows, int64_t cols, int64_t nnzb, int64_t k,
                    int64_t block_size, const sw_options *opts, void *stream);

/* sparsewave.bsr_spmm on bf16 memrefs: block values, rhs and output all
 * bf16 (BSRSpMMOp::verify, SparseWaveOps.cpp:355-360, requires the output
 * to have the block values' element type).  fp32 accumulation, the output
 * rounded to bf16.  Same operands as sw_bsr_spmm_f32. */
int sw_bsr_spmm_bf16(const int32_t *block_row_offsets,
                     const int32_t *block_column_indices,
                     const uint16_t *block_values, const uint16_t *rhs,
                     uint16_t *output, int64_t rows, int64_t cols,
                     int64_t nnzb, int64_t k, int64_t block_size,
                     const sw_options *opts, void *stream);

/* Extension with no reference op: bf16 block values and rhs, fp32 output
 * (the fp32 accumulators stored unrounded).  A caller binding
 * sparsewave.bsr_spmm on bf16 memrefs uses sw_bsr_spmm_bf16 instead. */
int sw_bsr_spmm_bf16_f32out(const int32_t *block_row_offsets,
                            const int32_t *block_column_indices,
                            const uint16_t *block_values, const uint16_t *rhs,
                            float *output, int64_t rows, int64_t cols,
                            int64_t nnzb, int64_t k, int64_t block_size,
                            const sw_options *opts, void *stream);

/*
 * BSR slab floor, a diagnostic with no counterpart in the reference: the
 * launch that sw_bsr_spmm_f32 / _bf16 / _bf16_f32out make on the matrix
 * cores for these operands (16 x 16 blocks; value_bytes 4 with k % 4 == 0,
 * or 2 with k % 8 == 0; 16-byte aligned rhs and output; output_bytes 4, or 2
 * for the bf16 output) with its grid, block order, block and RHS-slab
 * loads, LDS reduction and stores unchanged and the block products replaced
 * by an XOR of the 32-bit words each lane loads.  Every output element of a
 * lane's region holds that XOR (its low 16 bits for a bf16 output); the
 * regions and the words follow the MFMA kernels' lane layout.  Its time is
 * the floor of the kernels' memory trips; bench.py reports the BSR SpMM
 * against it.
 */
int sw_bsr_slab_floor(const int32_t *block_row_offsets,
                      const int32_t *block_column_indices,
                      const void *block_values, const void *rhs, void *output,
                      int64_t rows, int64_t cols, int64_t nnzb, int64_t k,
                      int value_bytes, int output_bytes, void *stream);

/* Scalar regions the reference attaches to sddmm
 * (SparseWaveOps.td:171-223).  SW_SDDMM_AFFINE is the attention form
 * sample*beta + dot*alpha (SparseAttentionToSparseWave.cpp:270-283). */
#define SW_SDDMM_MUL 0    /* sample * dot */
#define SW_SDDMM_AFFINE 1 /* sample * beta + dot * alpha */
#define SW_SDDMM_DOT 2    /* dot */

/*
 * sparsewave.sddmm: output_values[p] = region(values[p], lhs[r,:] . rhs[:,c])
 * for every stored (r, c) at position p.  lhs[rows][kdim], rhs[kdim][cols]
 * row-major.  ThreadPerRowSDDMMPattern (SparseWaveToGPU.cpp:667-750).
 * sddmm-mapping=row-tile-mfma runs 16-row v_mfma_f32_16x16x4_f32 tiles for
 * kdim in {64,128,256}; with kdim 64 or 128, at least 4 entries, and
 * output_values not overlapping values (or SW_SDDMM_DOT), the tiles are the
 * fused attention kernel's product phase.  Other kdim take one wave per row.
 */
int sw_sddmm_csr_f32(const int32_t *row_offsets, const int32_t *column_indices,
                     const float *values, const float *lhs, const float *rhs,
                     float *output_values, int64_t rows, int64_t cols,
                     int64_t nnz, int64_t kdim, int combine, float alpha,
                     float beta, const sw_options *opts, void *stream);

/* sparsewave.sddmm on bf16 memrefs (SDDMMOp::verify,
 * SparseWaveOps.cpp:374-425: values, lhs, rhs and output values share one
 * element type).  The region is evaluated in fp32 on the fp32 dot product
 * and rounded once.  sddmm-mapping=row-tile-mfma with kdim in {64,128,256}
 * runs v_mfma_f32_16x16x32_bf16 tiles (lhs 16-byte aligned); with kdim 64
 * or 128 as for fp32, through the bf16 fused attention kernel. */
int sw_sddmm_csr_bf16(const int32_t *row_offsets,
                      const int32_t *column_indices, const uint16_t *values,
                      const uint16_t *lhs, const uint16_t *rhs,
                      uint16_t *output_values, int64_t rows, int64_t cols,
                      int64_t nnz, int64_t kdim, int combine, float alpha,
                      float beta, const sw_options *opts, void *stream);

/*
 * sparsewave.csr_row_reduce: output[r] = fold over row r's stored values.
 * kind "sum" (identity 0) or "max" (identity -inf, NaN-propagating maximum)
 * (SparseWaveOps.td:225-257; ThreadPerRowCSRRowReducePattern,
 * SparseWaveToGPU.cpp:752-818).  column_indices may be NULL (unused).
 */
int sw_csr_row_reduce_f32(const int32_t *row_offsets,
                          const int32_t *column_indices, const float *values,
                          float *output, int64_t rows, int64_t nnz,
                          const char *kind, const sw_options *opts,
                          void *stream);

/* csr_row_reduce on bf16 memrefs: fp32 fold, the result rounded to bf16 (a
 * maximum is exact). */
int sw_csr_row_reduce_bf16(const int32_t *row_offsets,
                           const int32_t *column_indices,
                           const uint16_t *values, uint16_t *output,
                           int64_t rows, int64_t nnz, const char *kind,
                           const sw_options *opts, void *stream);

/* Scalar regions of csr_rowwise_map (attention: exp-sub and div,
 * SparseAttentionToSparseWave.cpp:288-309). */
#define SW_MAP_EXP_SUB 0 /* exp(value - row_value) */
#define SW_MAP_DIV 1     /* value / row_value */
#define SW_MAP_SUB 2     /* value - row_value */
#define SW_MAP_MUL 3     /* value * row_value */

/*
 * sparsewave.csr_rowwise_map: output_values[p] = f(values[p], row_values[r]).
 * output_values may alias values (the attention chain maps in place).
 * ThreadPerRowCSRRowwiseMapPattern (SparseWaveToGPU.cpp:820-878).
 */
int sw_csr_rowwise_map_f32(const int32_t *row_offsets,
                           const int32_t *column_indices, const float *values,
                           const float *row_values, float *output_values,
                           int64_t rows, int64_t nnz, int map,
                           const sw_options *opts, void *stream);

/* csr_rowwise_map on bf16 memrefs: f evaluated in fp32, rounded once. */
int sw_csr_rowwise_map_bf16(const int32_t *row_offsets,
                            const int32_t *column_indices,
                            const uint16_t *values,
                            const uint16_t *row_values,
                            uint16_t *output_values, int64_t rows,
                            int64_t nnz, int map, const sw_options *opts,
                            void *stream);

/*
 * The sparse-attention chain: the six ops of
 * examples/pytorch/integration/SparseAttentionToSparseWave.cpp:230-315 in
 * order -- scores = sddmm(affine alpha, beta), row_max, exp(s - max),
 * row_sum, s / sum, output = scores * value.  Buffers follow the bundle's
 * ten-buffer ABI (tools/sparsewave-bundle/sparsewave_bundle_ir.py:82-93):
 * query[rows][d], transposed_key[d][cols], value[cols][dv],
 * scores[nnz], row_maximum[rows], row_sum[rows], output[rows][dv].
 */
int sw_sparse_attention_f32(const int32_t *row_offsets,
                            const int32_t *column_indices,
                            const float *mask_values, const float *query,
                            const float *transposed_key, const float *value,
                            float *scores, float *row_maximum, float *row_sum,
                            float *output, int64_t rows, int64_t cols,
                            int64_t nnz, int64_t d, int64_t dv, float alpha,
                            float beta, const sw_options *opts, void *stream);

/*
 * The same chain with all ten buffers' values in bf16 (the bf16 option of
 * the attention bundle): the six ops on bf16 buffers, each op computing in
 * fp32 and storing its result rounded to bf16 -- scores after the SDDMM,
 * the exponentials, row sums and normalised scores, then the output.  The
 * fused one-kernel form (sddmm-mapping=row-tile-mfma sddmm-lanes-per-row=64
 * spmm-mapping=row-tile-mfma, d in {64,128}, dv % 64 == 0, query 16-byte and
 * value / output 8-byte aligned) keeps the scores in registers and rounds
 * them at the same points, with Q K^T on v_mfma_f32_16x16x32_bf16 and P V on
 * v_mfma_f32_16x16x16_bf16.
 */
int sw_sparse_attention_bf16(const int32_t *row_offsets,
                             const int32_t *column_indices,
                             const uint16_t *mask_values,
                             const uint16_t *query,
                             const uint16_t *transposed_key,
                             const uint16_t *value, uint16_t *scores,
                             uint16_t *row_maximum, uint16_t *row_sum,
                             uint16_t *output, int64_t rows, int64_t cols,
                             int64_t nnz, int64_t d, int64_t dv, float alpha,
                             float beta, const sw_options *opts,
                             void *stream);

/*
 * Attention tile floor, a diagnostic with no counterpart in the reference:
 * the fused one-kernel launch of sw_sparse_attention_f32 (value_bytes 4) or
 * _bf16 (value_bytes 2) for these buffers -- d of 64 or 128, dv a multiple
 * of 16 (fp32) or 64 (bf16, with 16-byte aligned query and 8-byte aligned
 * value and output), nnz >= 4 -- with its loads, structure check and
 * barrier, score / row / output stores and output reduction unchanged, and
 * every product, exponential and division replaced by an XOR of the words
 * each lane loads (so the two softmax barriers go too).  The outputs hold
 * those XORs as bit patterns; tiles whose rows do not share the last row's
 * columns take the fused kernel's row path and compute the chain.  Its
 * time is the floor of the tile's chain of memory trips; bench.py reports
 * the fused attention against it.
 */
int sw_attention_tile_floor(const int32_t *row_offsets,
                            const int32_t *column_indices,
                            const void *mask_values, const void *query,
                            const void *transposed_key, const void *value,
                            void *scores, void *row_maximum, void *row_sum,
                            void *output, int64_t rows, int64_t cols,
                            int64_t nnz, int64_t d, int64_t dv,
                            int value_bytes, void *stream);

/*
 * sparsewave.csr_row_at_position for a batch of positions:
 * out_rows[i] = (first j in [1, rows+1) with row_offsets[j] > positions[i]) - 1,
 * the row search of SparsePositionToSCF.cpp:225-271 that the position
 * mappings run.  positions[i] must lie in [0, nnz).
 */
int sw_csr_row_at_position(const int32_t *row_offsets, int64_t rows,
                           const int64_t *positions, int32_t *out_rows,
                           int64_t count, void *stream);

/* ---- Host-side matrix files -------------------------------------------- */
/* These run on the host only and make no HIP call: every pointer below is
 * host memory, and the readers allocate their results with malloc.  They
 * load the reference harness's workloads (SuiteSparse Matrix Market files
 * and the SWCSR001 / SWCOO001 / SWBSR001 binaries it converts them to). */

/*
 * A sparse matrix in host memory, as the benchmark harness holds it
 * (benchmark/benchmark_utils.py:56-177 returns the same fields).  The
 * arrays are malloc'ed by the library when it returns one (free with
 * sw_host_matrix_free); a caller building one for a writer owns them.
 * row_indices / column_indices / values are the COO entries (nnz each);
 * row_offsets (rows + 1) is set, and has_row_offsets = 1, when the entries
 * are grouped by row in row order (always after a Matrix Market or CSR read,
 * for a COO read only when the file stores them that way).  Values are kept
 * in double until written, as the reference writer holds Python floats.
 */
typedef struct sw_host_matrix {
  int64_t rows, columns, nnz;
  int32_t *row_offsets;
  int32_t *row_indices;
  int32_t *column_indices;
  double *values;
  int32_t has_row_offsets;
  char field[16];    /* "real" | "integer" | "pattern" ("" for binaries) */
  char symmetry[16]; /* "general" | "symmetric" ("" for binaries) */
  int64_t min_row_nnz, max_row_nnz;
  double mean_row_nnz;
} sw_host_matrix;

/*
 * A padded BSR matrix with the COO entries it was built from
 * (convert_to_bsr, benchmark/benchmark_utils.py:240-312): rows / columns
 * padded up to multiples of block_size, blocks row-major [nnzb][b][b],
 * repeated coordinates added up.
 */
typedef struct sw_host_bsr {
  int64_t rows, columns, nnzb, block_size;
  int64_t original_rows, original_columns, nnz;
  int32_t *block_row_offsets;    /* rows / block_size + 1 */
  int32_t *block_column_indices; /* nnzb */
  double *block_values;          /* nnzb * block_size^2 */
  int32_t *input_row_indices;    /* nnz */
  int32_t *input_column_indices; /* nnz */
  double *input_values;          /* nnz */
  double block_density, internal_zero_fraction, storage_overhead;
} sw_host_bsr;

void sw_host_matrix_free(sw_host_matrix *m);
void sw_host_bsr_free(sw_host_bsr *b);

/* Matrix Market coordinate reader (benchmark/benchmark_utils.py:56-177):
 * real / integer / pattern, general / symmetric (off-diagonal entries
 * mirrored), 1-based indices, finite values that fit f32, entry count as
 * declared; entries sorted by (row, column), repeated coordinates kept in
 * file order.  Errors name the file and line. */
int sw_matrix_market_read(const char *path, sw_host_matrix **out);

/* SWCSR001 / SWCOO001 writers (benchmark/benchmark_utils.py:180-237): the
 * 8-byte magic, rows, columns, nnz as little-endian u64, then i32 / f32
 * arrays (CSR: row offsets, column indices, values; COO: row indices,
 * column indices, values). */
int sw_csr_binary_write(const char *path, const sw_host_matrix *m);
int sw_coo_binary_write(const char *path, const sw_host_matrix *m);

/* Readers of the same files (benchmark/SparseBenchmarkUtils.cpp:83-141),
 * which also check the index structure (offsets 0..nnz, non-decreasing,
 * indices in range) so the result can go to the GPU as is. */
int sw_csr_binary_read(const char *path, sw_host_matrix **out);
int sw_coo_binary_read(const char *path, sw_host_matrix **out);

/* COO -> padded BSR (benchmark/benchmark_utils.py:240-312). */
int sw_convert_to_bsr(const sw_host_matrix *m, int64_t block_size,
                      sw_host_bsr **out);

/* SWBSR001 writer / reader (benchmark/benchmark_utils.py:315-379,
 * benchmark/SparseBenchmarkUtils.cpp:143-185): magic, rows, columns, nnzb,
 * block size, original rows, original columns, original nnz (u64), then
 * block-row offsets, block-column indices, block values, and the original
 * COO row indices, column indices and values. */
int sw_bsr_binary_write(const char *path, const sw_host_bsr *m);
int sw_bsr_binary_read(const char *path, sw_host_bsr **out);

#ifdef __cplusplus
}
#endif

#endif /* SPARSEWAVE_AMD_H */
