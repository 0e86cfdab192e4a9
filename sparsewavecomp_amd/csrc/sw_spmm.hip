// sparsewave.spmm on gfx950 behind sw_spmm_csr_f32.
//
// Reference kernels (generated IR):
//   thread-per-output    SparseWaveToGPU.cpp:489-558
//   wave-per-row-tile    SparseWaveToGPU.cpp:1057-1256
//   thread-per-position  PositionSpMMDecomposition.cpp:19-73 +
//                        SparsePositionScheduling.cpp:135-194
#include "sw_device.h"
#include "sw_internal.h"

#include <algorithm>

using namespace swd;

namespace {

// thread-per-output: one thread per C[r, c], sequential over the row.
__global__ __launch_bounds__(1024) void spmm_thread_per_output(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ rhs,
    float *__restrict__ out, int64_t rows, int64_t k) {
  int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * k)
    return;
  int64_t r = e / k, c = e - r * k;
  int32_t s = ro[r], t = ro[r + 1];
  float acc = 0.0f;
  for (int32_t p = s; p < t; ++p)
    acc = __builtin_fmaf(val[p], rhs[(int64_t)col[p] * k + c], acc);
  out[e] = acc;
}

// wave-per-row-tile, Wave64 lane layout.
//
// A group of G lanes owns one (row, tile) work unit; G = 64 is the
// reference's wave per row tile, smaller G packs 64/G units into a wave for
// short rows.  Inside the group, CL "column lanes" each own V consecutive
// output columns of the tile (V = 4 uses 128-bit RHS loads) and PL = G/CL
// "position lanes" stride the row.  Each position lane reads val[p] and
// col[p] once and reuses them for all of its columns; the partial sums are
// reduced across the PL position lanes with xor shuffles, and the first
// position lane stores its V outputs (one contiguous T-column store per
// group).  Full and tail tiles share the code; tail columns are masked.
template <int V, int CL, int G>
__global__ __launch_bounds__(1024) void spmm_row_tile(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ rhs,
    float *__restrict__ out, int64_t rows, int64_t k, int32_t tile,
    int64_t tiles_per_row) {
  constexpr int PL = G / CL;
  const int units_per_block = blockDim.x / G;
  const int64_t unit = (int64_t)blockIdx.x * units_per_block + threadIdx.x / G;
  const int gl = threadIdx.x & (G - 1);
  const int pl = gl / CL;
  const int cl = gl % CL;
  const bool unit_ok = unit < rows * tiles_per_row;
  int64_t r = 0, c0 = 0;
  if (unit_ok) {
    r = unit / tiles_per_row;
    c0 = (unit - r * tiles_per_row) * tile;
  }
  const int64_t cb = c0 + (int64_t)cl * V;
  const int64_t cend = std::min<int64_t>(c0 + tile, k);
  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i)
    acc[i] = 0.0f;
  if (unit_ok && cb < cend) {
    const int32_t s = ro[r], e = ro[r + 1];
    if (V == 4 && cb + 4 <= cend) {
      for (int32_t p = s + pl; p < e; p += PL) {
        const float v = ld_stream(val + p);
        const int64_t c = ld_stream(col + p);
        const v4f b = *reinterpret_cast<const v4f *>(rhs + c * k + cb);
        acc[0] = __builtin_fmaf(v, b.x, acc[0]);
        if constexpr (V == 4) {
          acc[1] = __builtin_fmaf(v, b.y, acc[1]);
          acc[2] = __builtin_fmaf(v, b.z, acc[2]);
          acc[3] = __builtin_fmaf(v, b.w, acc[3]);
        }
      }
    } else {
      for (int32_t p = s + pl; p < e; p += PL) {
        const float v = ld_stream(val + p);
        const int64_t c = ld_stream(col + p);
        const float *b = rhs + c * k + cb;
#pragma unroll
        for (int i = 0; i < V; ++i)
          if (cb + i < cend)
            acc[i] = __builtin_fmaf(v, b[i], acc[i]);
      }
    }
  }
  // reduce over the position lanes of the group (lane bits >= log2 CL)
#pragma unroll
  for (int off = CL; off < G; off <<= 1) {
#pragma unroll
    for (int i = 0; i < V; ++i)
      acc[i] += __shfl_xor(acc[i], off, 64);
  }
  if (unit_ok && pl == 0 && cb < cend) {
    float *o = out + r * k + cb;
    if (V == 4 && cb + 4 <= cend) {
      *reinterpret_cast<v4f *>(o) = v4f{acc[0], acc[V > 1 ? 1 : 0],
                                        acc[V > 2 ? 2 : 0], acc[V > 3 ? 3 : 0]};
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i)
        if (cb + i < cend)
          o[i] = acc[i];
    }
  }
}

__global__ __launch_bounds__(1024) void spmm_fill_zero(float *__restrict__ y,
                                                       int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n)
    y[i] = 0.0f;
}

// thread-per-position: iteration i = p*K + c over [0, nnz*K), chunked per
// worker, atomic add into the flattened output at row(p)*K + c.
__global__ __launch_bounds__(1024) void spmm_thread_position(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ rhs,
    float *__restrict__ out, int32_t rows, int64_t k, int64_t iterations,
    int64_t chunk) {
  int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t b = w * chunk;
  if (b >= iterations)
    return;
  int64_t e = std::min<int64_t>(b + chunk, iterations);
  for (int64_t i = b; i < e; ++i) {
    int64_t p = i / k, c = i - p * k;
    int r = row_search_lane(ro, 1u, (uint32_t)rows + 1u, (int32_t)p);
    unsafeAtomicAdd(out + (int64_t)r * k + c, val[p] * rhs[(int64_t)col[p] * k + c]);
  }
}

template <int V, int CL, int G>
void launch_tile(int64_t grid, int64_t B, hipStream_t st, const int32_t *ro,
                 const int32_t *col, const float *val, const float *rhs,
                 float *out, int64_t rows, int64_t k, int32_t tile,
                 int64_t tpr) {
  hipLaunchKernelGGL((spmm_row_tile<V, CL, G>), dim3((unsigned)grid),
                     dim3((unsigned)B), 0, st, ro, col, val, rhs, out, rows, k,
                     tile, tpr);
}

template <int V, int CL>
void dispatch_g(int G, int64_t rows, int64_t tpr, int64_t B, hipStream_t st,
                const int32_t *ro, const int32_t *col, const float *val,
                const float *rhs, float *out, int64_t k, int32_t tile,
                int64_t *grid_out) {
  int64_t units = rows * tpr;
  int64_t grid = std::max<int64_t>(sw::ceil_div(units, B / G), 1);
  *grid_out = grid;
  if (grid > sw::kMaxGridX)
    return;
#define SW_TILE_CASE(GG)                                                      \
  case GG:                                                                    \
    if constexpr (GG >= CL)                                                   \
      launch_tile<V, CL, (GG >= CL ? GG : CL)>(grid, B, st, ro, col, val,     \
                                               rhs, out, rows, k, tile, tpr); \
    break;
  switch (G) {
    SW_TILE_CASE(1)
    SW_TILE_CASE(2)
    SW_TILE_CASE(4)
    SW_TILE_CASE(8)
    SW_TILE_CASE(16)
    SW_TILE_CASE(32)
    SW_TILE_CASE(64)
  }
#undef SW_TILE_CASE
}

int next_pow2(int v) {
  int p = 1;
  while (p < v)
    p <<= 1;
  return p;
}

} // namespace

namespace sw {

int launch_spmm(const int32_t *ro, const int32_t *col, const float *val,
                const float *rhs, float *out, int64_t rows, int64_t nnz,
                int64_t k, const sw_options &o, const char *what,
                hipStream_t st) {
  const int64_t B = o.spmm_block_size;
  if (streq(o.spmm_mapping, "thread-per-output")) {
    int64_t grid = std::max<int64_t>(ceil_div(rows * k, B), 1);
    int rc = check_grid(grid, what);
    if (rc)
      return rc;
    hipLaunchKernelGGL(spmm_thread_per_output, dim3((unsigned)grid),
                       dim3((unsigned)B), 0, st, ro, col, val, rhs, out, rows,
                       k);
    return launch_check("thread-per-output SpMM kernel");
  }
  if (streq(o.spmm_mapping, "thread-per-position")) {
    int64_t n_out = rows * k;
    if (n_out > 0) {
      int64_t g0 = ceil_div(n_out, o.position_block_size);
      int rc = check_grid(g0, what);
      if (rc)
        return rc;
      hipLaunchKernelGGL(spmm_fill_zero, dim3((unsigned)g0),
                         dim3((unsigned)o.position_block_size), 0, st, out,
                         n_out);
      rc = launch_check("SpMM output initialisation kernel");
      if (rc)
        return rc;
    }
    int64_t iters = nnz * k;
    if (iters == 0)
      return SW_OK;
    int64_t chunk = o.spmm_position_chunk_size;
    int64_t grid = std::max<int64_t>(ceil_div(ceil_div(iters, chunk), B), 1);
    int rc = check_grid(grid, what);
    if (rc)
      return rc;
    hipLaunchKernelGGL(spmm_thread_position, dim3((unsigned)grid),
                       dim3((unsigned)B), 0, st, ro, col, val, rhs, out,
                       (int32_t)rows, k, iters, chunk);
    return launch_check("thread-per-position SpMM kernel");
  }
  // wave-per-row-tile
  const int T = (int)o.spmm_tile_size;
  const int64_t tpr = ceil_div(k, T);
  const bool vec = (T % 4 == 0) && (k % 4 == 0) && aligned16(rhs) &&
                   aligned16(out);
  const int V = vec ? 4 : 1;
  const int CL = next_pow2(ceil_div(T, V));
  const int G = std::max<int>((int)o.spmm_lanes_per_row, CL);
  int64_t grid = 0;
  const int32_t tile = (int32_t)T;
#define SW_CL_CASE(VV, CC)                                                    \
  if (V == VV && CL == CC)                                                    \
    dispatch_g<VV, CC>(G, rows, tpr, B, st, ro, col, val, rhs, out, k, tile,  \
                       &grid);
  SW_CL_CASE(4, 1)
  SW_CL_CASE(4, 2)
  SW_CL_CASE(4, 4)
  SW_CL_CASE(4, 8)
  SW_CL_CASE(1, 1)
  SW_CL_CASE(1, 2)
  SW_CL_CASE(1, 4)
  SW_CL_CASE(1, 8)
  SW_CL_CASE(1, 16)
  SW_CL_CASE(1, 32)
#undef SW_CL_CASE
  if (grid == 0)
    return fail(SW_ERR_INVALID_OPTION,
                "no wave-per-row-tile kernel for tile size %d", T);
  int rc = check_grid(grid, what);
  if (rc)
    return rc;
  return launch_check("wave-per-row-tile SpMM kernel");
}

} // namespace sw

extern "C" int sw_spmm_csr_f32(const int32_t *row_offsets,
                               const int32_t *column_indices,
                               const float *values, const float *rhs,
                               float *output, int64_t rows, int64_t cols,
                               int64_t nnz, int64_t k, const sw_options *opts,
                               void *stream) {
  sw::clear_error();
  sw_options o;
  int rc = sw::resolve_options(opts, &o);
  if (rc)
    return rc;
  rc = sw::check_csr(row_offsets, column_indices, values, rows, nnz, true);
  if (rc)
    return rc;
  if (cols < 0 || k < 0)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "expected non-negative rhs shape, but got %lld x %lld",
                    (long long)cols, (long long)k);
  if (rows == 0 || k == 0)
    return SW_OK;
  if (!output || (nnz > 0 && !rhs))
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "rhs or output pointer is null");
  return sw::launch_spmm(row_offsets, column_indices, values, rhs, output,
                         rows, nnz, k, o, "SpMM", sw::as_stream(stream));
}
