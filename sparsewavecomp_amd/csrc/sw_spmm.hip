// sparsewave.spmm on gfx950 behind sw_spmm_csr_f32.
//
// Reference kernels (generated IR):
//   thread-per-output    SparseWaveToGPU.cpp:489-558
//   wave-per-row-tile    SparseWaveToGPU.cpp:1057-1256
//   thread-per-position  PositionSpMMDecomposition.cpp:19-73 +
//                        SparsePositionScheduling.cpp:135-194
//   wave-per-position    Wave64 extension: the SpMV position schedule
//                        (SparsePositionScheduling.cpp:318-403) over
//                        (position, column tile) pairs
#include "sw_device.h"
#include "sw_spmm_tile.h"
#include "sw_internal.h"

#include <algorithm>

using namespace swd;

namespace {

// thread-per-output: one thread per C[r, c], sequential over the row.
// Products are added in position order with kOutputDeep positions' loads
// and rhs gathers in flight while that many remain, then four: the kernel's
// time is the longest rows' chain of memory trips.
constexpr int kOutputDeep = 16;

// rhs[c][j].  NARROW (the host's guarantee that 4 * rhs_rows * k fits 32
// bits): the wave-uniform base rhs plus a 32-bit lane byte offset, which the
// load takes directly; otherwise a 64-bit lane address, whose multiply by k
// costs more than the load (configuration 3, thread-per-output: K=64
// 1797 -> 1381 us, K=4 685 -> 653 us with the narrow form).
template <bool NARROW, typename T>
__device__ __forceinline__ float rhs_at(const T *__restrict__ rhs, int32_t c,
                                        int64_t k, int64_t j) {
  if constexpr (NARROW)
    return tof(*at_bytes(rhs, (uint32_t)sizeof(T) *
                                  ((uint32_t)c * (uint32_t)k + (uint32_t)j)));
  else
    return ldv(rhs + (int64_t)c * k + j);
}

// ROW (k and the block size multiples of 64): a wave's 64 outputs lie in
// one row, so the row index is put in a scalar register and the row's
// column and value loads become scalar loads shared by the wave.
template <bool NARROW, bool ROW, typename T>
__global__ __launch_bounds__(1024) void spmm_thread_per_output(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const T *__restrict__ val, const T *__restrict__ rhs,
    T *__restrict__ out, int64_t rows, int64_t k) {
  int64_t e = block_id() * blockDim.x + threadIdx.x;
  if (e >= rows * k)
    return;
  int64_t r = e / k, c = e - r * k;
  if constexpr (ROW) // rows * k < 2^31 * 64: the row fits 32 bits
    r = __builtin_amdgcn_readfirstlane((int32_t)r);
  int32_t s = ro[r], t = ro[r + 1];
  float acc = 0.0f;
  int32_t p = s;
  for (; p + kOutputDeep - 1 < t; p += kOutputDeep) {
    float v[kOutputDeep], b[kOutputDeep];
    int32_t cc[kOutputDeep];
#pragma unroll
    for (int u = 0; u < kOutputDeep; ++u) {
      v[u] = ldv(val + p + u);
      cc[u] = col[p + u];
    }
#pragma unroll
    for (int u = 0; u < kOutputDeep; ++u)
      b[u] = rhs_at<NARROW>(rhs, cc[u], k, c);
#pragma unroll
    for (int u = 0; u < kOutputDeep; ++u)
      acc = __builtin_fmaf(v[u], b[u], acc);
  }
  for (; p + 3 < t; p += 4) {
    float v[4], b[4];
    int32_t cc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v[u] = ldv(val + p + u);
      cc[u] = col[p + u];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      b[u] = rhs_at<NARROW>(rhs, cc[u], k, c);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      acc = __builtin_fmaf(v[u], b[u], acc);
  }
  for (; p < t; ++p)
    acc = __builtin_fmaf(ldv(val + p), rhs_at<NARROW>(rhs, col[p], k, c), acc);
  stv(out + e, acc);
}

// wave-per-row-tile, Wave64 lane layout.
//
// wave-per-row-tile: one (row, tile) unit per group of G lanes, the units in
// XCD-contiguous order (sw_spmm_tile.h holds the unit's code).
template <int V, int CL, int G, typename T>
__global__ __launch_bounds__(1024) void spmm_row_tile(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const T *__restrict__ val, const T *__restrict__ rhs,
    T *__restrict__ out, int64_t rows, int64_t k, int32_t tile,
    int64_t tiles_per_row) {
  const int units_per_block = blockDim.x / G;
  const int64_t unit =
      xcd_contiguous(block_id(), grid_blocks()) * units_per_block +
      threadIdx.x / G;
  spmm_row_tile_unit<V, CL, G, T>(ro, col, val, rhs, out, rows, k, tile,
                                  tiles_per_row, unit, threadIdx.x & (G - 1));
}

__global__ __launch_bounds__(1024) void spmm_fill_zero(float *__restrict__ y,
                                                       int64_t n) {
  int64_t i = block_id() * blockDim.x + threadIdx.x;
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
  int64_t w = block_id() * blockDim.x + threadIdx.x;
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


// wave-per-position SpMM (Wave64 extension of the position schedule).
//
// The nonzeros are cut into units of P consecutive positions exactly as in
// the SpMV position kernel, and the output columns into tiles of CL*V.  A
// wave owns one (position chunk, column tile): its 64 lanes form PL = 64/CL
// "virtual lanes" of CL lanes each; virtual lane vl walks unit chunk*PL+vl
// and each of its CL lanes accumulates V consecutive output columns
// (V = 4: 128-bit RHS gathers).  Row recovery (wave-uniform scalar searches
// plus an LDS window of row boundaries), the in-lane walk, the segmented scan
// over the virtual lanes (stride CL) and the one-atomic-per-segment emission
// follow the SpMV kernel.  Position balance makes rows of any length cost the
// same, which the row-tile mapping cannot offer for rows thousands long.
template <int V, int CL, int P, bool SR>
__global__ __launch_bounds__(1024) void spmm_wave_position(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ rhs,
    float *__restrict__ out, int32_t rows, int32_t nnz, int64_t k,
    int64_t units, int64_t chunks, int64_t tiles, bool vec) {
  constexpr int PL = kWave / CL;
  const int lane = lane_id();
  const int64_t wave =
      block_id() * (blockDim.x / kWave) + wave_in_group();
  if (wave >= chunks * tiles)
    return;
  const int64_t chunk = wave / tiles;
  const int64_t tile = wave - chunk * tiles;
  const int64_t wbeg = chunk * PL * P;
  const int64_t wend = std::min<int64_t>((chunk + 1) * PL * P, nnz);
  if (wbeg >= wend)
    return;
  const int vl = lane / CL, cl = lane % CL;
  const int64_t cb = tile * (CL * V) + (int64_t)cl * V;
  const bool col_ok = cb < k;
  const int64_t u = chunk * PL + vl;
  const bool active = u < units;
  const int32_t p0 = active ? (int32_t)(u * P) : 0;
  const int32_t pe =
      active ? (int32_t)std::min<int64_t>(u * P + P, (int64_t)nnz) : 0;

  float vv[P];
  float g[P][V];
#pragma unroll
  for (int q = 0; q < P; ++q) {
    vv[q] = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i)
      g[q][i] = 0.0f;
  }
  if (active && col_ok) {
    int32_t cc[P];
    bool full = false;
    if constexpr (P >= 4) {
      full = vec && pe - p0 == P;
      if (full) {
#pragma unroll
        for (int q = 0; q < P; q += 4) {
          v4i c4 = ld_stream(reinterpret_cast<const v4i *>(col + p0 + q));
          v4f v4 = ld_stream(reinterpret_cast<const v4f *>(val + p0 + q));
          cc[q] = c4.x, cc[q + 1] = c4.y, cc[q + 2] = c4.z, cc[q + 3] = c4.w;
          vv[q] = v4.x, vv[q + 1] = v4.y, vv[q + 2] = v4.z, vv[q + 3] = v4.w;
        }
      }
    }
    if (!full) {
#pragma unroll
      for (int q = 0; q < P; ++q) {
        cc[q] = -1;
        if (p0 + q < pe) {
          cc[q] = ld_stream(col + p0 + q);
          vv[q] = ld_stream(val + p0 + q);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < P; ++q) {
      if (full || p0 + q < pe) {
        const float *b = rhs + (int64_t)cc[q] * k + cb;
        if constexpr (V == 4) {
          const v4f b4 = *reinterpret_cast<const v4f *>(b);
          g[q][0] = b4.x;
          g[q][V > 1 ? 1 : 0] = b4.y;
          g[q][V > 2 ? 2 : 0] = b4.z;
          g[q][V > 3 ? 3 : 0] = b4.w;
        } else {
          g[q][0] = b[0];
        }
      }
    }
  }

  const int first_row =
      row_search_uniform(ro, 1u, (uint32_t)rows + 1u, (int32_t)wbeg);
  const int last_row = row_search_gallop(ro, (uint32_t)first_row + 1u,
                                         (uint32_t)rows + 1u,
                                         (int32_t)(wend - 1));
  __shared__ int32_t window[1024 / kWave][kWave];
  int32_t *win = window[wave_in_group()];
  const int span = last_row - first_row;
  const bool use_win = span < kWave;
  if (use_win) {
    const int j = first_row + 1 + lane;
    win[lane] = j <= first_row + 1 + span ? ro[j] : INT32_MAX;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  int lrow = 0, row = 0, closed = 0;
  float head[V], acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i)
    head[i] = acc[i] = 0.0f;
  if (active) {
    int32_t next;
    if (use_win) {
      int lo = 0, hi = span;
      while (lo < hi) {
        int mid = (lo + hi) >> 1;
        if (win[mid] <= p0)
          lo = mid + 1;
        else
          hi = mid;
      }
      lrow = first_row + lo;
      next = win[lo];
    } else {
      lrow = row_search_lane(ro, (uint32_t)first_row + 1u,
                             (uint32_t)last_row + 2u, p0);
      next = ro[lrow + 1];
    }
    row = lrow;
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const int32_t p = p0 + q;
      if (p < pe) {
        while (p >= next) {
          if (closed == 0) {
#pragma unroll
            for (int i = 0; i < V; ++i)
              head[i] = acc[i];
          } else if (col_ok) {
            float *o = out + (int64_t)row * k + cb;
#pragma unroll
            for (int i = 0; i < V; ++i)
              o[i] = acc[i]; // row began and ended inside this lane
          }
          ++closed;
#pragma unroll
          for (int i = 0; i < V; ++i)
            acc[i] = 0.0f;
          ++row;
          next = use_win ? win[row - first_row] : ro[row + 1];
        }
#pragma unroll
        for (int i = 0; i < V; ++i)
          acc[i] = __builtin_fmaf(vv[q], g[q][i], acc[i]);
      }
    }
  }

  // segmented scan of the virtual lanes' tails (lanes l and l - CL*j share
  // a column slot)
  const int key = active ? row : -1;
  float sc[V];
#pragma unroll
  for (int i = 0; i < V; ++i)
    sc[i] = active ? acc[i] : 0.0f;
  if constexpr (CL == 1) {
#pragma unroll
    for (int i = 0; i < V; ++i)
      sc[i] = wave_segmented_scan(key, sc[i]);
  } else {
#pragma unroll
    for (int off = CL; off < kWave; off <<= 1) {
      const int k2 = __shfl_up(key, off, kWave);
      const bool take = lane >= off && k2 == key;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float v2 = __shfl_up(sc[i], off, kWave);
        sc[i] += take ? v2 : 0.0f;
      }
    }
  }
  int prev_key = __shfl_up(key, CL, kWave);
  if (lane < CL)
    prev_key = INT32_MIN;
  float prev_sc[V];
#pragma unroll
  for (int i = 0; i < V; ++i)
    prev_sc[i] = __shfl_up(sc[i], CL, kWave);
  int next_lrow = __shfl_down(active ? lrow : -2, CL, kWave);
  if (lane >= kWave - CL)
    next_lrow = -2;
  // With SR (output rows of whole cache lines) only the chunk's first and
  // last rows, which can own positions of other chunks, are accumulated
  // atomically (position_init zeroed them) and the rest are stored;
  // otherwise every segment is an atomic add into a zeroed output (narrow
  // rows: scattered partial-line stores from several XCDs measured slower
  // than atomics).
  const bool first_shared = !SR || ro[first_row] < wbeg;
  const bool last_shared = !SR || ro[last_row + 1] > wend;
  if (active && col_ok) {
    if (closed > 0) {
      float *o = out + (int64_t)lrow * k + cb;
      const bool carry = prev_key == lrow;
      const bool shared = (lrow == first_row && first_shared) ||
                          (lrow == last_row && last_shared);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        const float h = head[i] + (carry ? prev_sc[i] : 0.0f);
        if (shared)
          unsafeAtomicAdd(o + i, h);
        else
          o[i] = h;
      }
    }
    if (next_lrow != row) {
      float *o = out + (int64_t)row * k + cb;
      const bool shared = (row == first_row && first_shared) ||
                          (row == last_row && last_shared);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        if (shared)
          unsafeAtomicAdd(o + i, sc[i]);
        else
          o[i] = sc[i];
      }
    }
  }
}

template <int V, int CL, int P>
void launch_wpos(int64_t grid, int64_t B, hipStream_t st, const int32_t *ro,
                 const int32_t *col, const float *val, const float *rhs,
                 float *out, int32_t rows, int32_t nnz, int64_t k,
                 int64_t units, int64_t chunks, int64_t tiles, bool vec,
                 bool store_rows) {
  // the store-emission variant exists for 128-bit lanes of >= 8-lane tiles
  // only (k >= 32)
  if constexpr (V == 4 && CL >= 8) {
    if (store_rows) {
      hipLaunchKernelGGL((spmm_wave_position<V, CL, P, true>),
                         sw::grid_dim(grid, B), dim3((unsigned)B), 0, st, ro,
                         col, val, rhs, out, rows, nnz, k, units, chunks,
                         tiles, vec);
      return;
    }
  }
  hipLaunchKernelGGL((spmm_wave_position<V, CL, P, false>),
                     sw::grid_dim(grid, B), dim3((unsigned)B), 0, st, ro, col,
                     val, rhs, out, rows, nnz, k, units, chunks, tiles, vec);
}

template <int V, int CL>
bool dispatch_wpos_p(int P, int64_t grid, int64_t B, hipStream_t st,
                     const int32_t *ro, const int32_t *col, const float *val,
                     const float *rhs, float *out, int32_t rows, int32_t nnz,
                     int64_t k, int64_t units, int64_t chunks, int64_t tiles,
                     bool vec, bool sr) {
  switch (P) {
  case 1: launch_wpos<V, CL, 1>(grid, B, st, ro, col, val, rhs, out, rows, nnz, k, units, chunks, tiles, vec, sr); return true;
  case 2: launch_wpos<V, CL, 2>(grid, B, st, ro, col, val, rhs, out, rows, nnz, k, units, chunks, tiles, vec, sr); return true;
  case 4: launch_wpos<V, CL, 4>(grid, B, st, ro, col, val, rhs, out, rows, nnz, k, units, chunks, tiles, vec, sr); return true;
  case 8: launch_wpos<V, CL, 8>(grid, B, st, ro, col, val, rhs, out, rows, nnz, k, units, chunks, tiles, vec, sr); return true;
  case 16: launch_wpos<V, CL, 16>(grid, B, st, ro, col, val, rhs, out, rows, nnz, k, units, chunks, tiles, vec, sr); return true;
  }
  return false;
}


// Row r of C computed by one wave: lanes over the output columns, sequential
// over the row's positions (the fallback of the tile kernel).
template <typename T>
__device__ __forceinline__ void spmm_row_wave(const int32_t *__restrict__ ro,
                                              const int32_t *__restrict__ col,
                                              const T *__restrict__ val,
                                              const T *__restrict__ rhs,
                                              T *__restrict__ out, int64_t r,
                                              int64_t k) {
  const int32_t s = ro[r], e = ro[r + 1];
  for (int64_t c = lane_id(); c < k; c += kWave) {
    float acc = 0.0f;
    for (int32_t p = s; p < e; ++p)
      acc = __builtin_fmaf(ldv(val + p), ldv(rhs + (int64_t)col[p] * k + c),
                           acc);
    stv(out + r * k + c, acc);
  }
}

// SpMM over 16-row tiles on the matrix cores (k % 16 == 0).
//
// For a tile whose rows share the last row's column structure
// (tile_prefix_ok_block), C[r0 .. r0+15][n0 .. n0+15] is a dense product of
// the tile's values (zero past each row's end) with the rhs rows of the last
// row's columns, 16 stored entries (four v_mfma_f32_16x16x4_f32 steps) at a
// time: lane (i, g) supplies val[ro[r0+i] + t0+4g+s], lane (j, g) supplies
// rhs[c_{t0+4g+s}][n0+j].  The W waves split the stored entries (wave w
// takes the 32-entry chunks w, w+W, ...), each accumulates four 16-column
// output tiles, and the partial tiles are summed through LDS.  Tiles without
// the shared structure are computed row by row.  Eight waves per tile
// (17.6 us on configuration 5, four: 21.9 us) give the chip enough waves:
// 8192 rows are only 512 tiles.
template <int W>
__global__ __launch_bounds__(64 * W) void spmm_tile_mfma(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ rhs,
    float *__restrict__ out, int32_t rows, int64_t k) {
  constexpr int CH = 2; // 16-entry chunks per step
  __shared__ float part[W][4][4][kWave]; // [wave][n tile][v][lane]
  if (block_id() * 16 >= rows)
    return; // a folded grid's surplus workgroup (workgroup-uniform)
  const int r0 = (int)block_id() * 16;
  const int nt = std::min(16, rows - r0);
  const int wave = wave_in_group();
  const int l = lane_id(), i = l & 15, g = l >> 4;
  // the row bounds are requested before the structure check waits; loads
  // are unconditional from clamped, valid addresses (a guarded load becomes
  // a branch that waits for it on the spot)
  const int last = r0 + nt - 1;
  const int32_t bl = ro[last];
  const int32_t len_last = ro[last + 1] - bl;
  const int ic = i < nt ? i : nt - 1;
  const int32_t ra = ro[r0 + ic];
  const int32_t la = i < nt ? ro[r0 + ic + 1] - ra : 0;
  __shared__ int verdict;
  __shared__ int nonfinite_out; // an output of the tile is inf or NaN
  if (threadIdx.x == 0)
    nonfinite_out = 0; // read only after the check's barriers
  if (!tile_prefix_ok_block(ro, col, r0, nt, &verdict)) {
    for (int r = r0 + wave; r < r0 + nt; r += W)
      spmm_row_wave(ro, col, val, rhs, out, r, k);
    return;
  }
  bool nonfinite = false;
  for (int64_t nb = 0; nb < k; nb += 64) {
    const int ntiles = (int)std::min<int64_t>(4, (k - nb) / 16);
    v4f acc[4];
#pragma unroll
    for (int n = 0; n < 4; ++n)
      acc[n] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int32_t t0 = wave * 16 * CH; t0 < len_last; t0 += W * 16 * CH) {
      float a[CH][4];
      int64_t c[CH][4];
#pragma unroll
      for (int h = 0; h < CH; ++h)
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const int32_t t = t0 + 16 * h + 4 * g + st;
          const int32_t tc = std::min(t, len_last - 1); // len_last > 0 here
          // rows shorter than t read the last row's entry, then drop it
          const float x = val[t < la ? ra + t : bl + tc];
          const int32_t cx = col[bl + tc];
          a[h][st] = t < la ? x : 0.0f;
          c[h][st] = t < len_last ? (int64_t)cx : -1;
        }
      float bv[CH][4][4];
#pragma unroll
      for (int h = 0; h < CH; ++h)
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int st = 0; st < 4; ++st) {
            // tiles n >= ntiles read tile 0 again: their outputs are never
            // stored, and a select on the wave-uniform n < ntiles would
            // become a branch around each load (configuration-5 mask, K=64:
            // 15.9 -> 14.7 us, K=128: 26.8 -> 24.8 us without it)
            const bool in = c[h][st] >= 0;
            const int nn = n < ntiles ? n : 0;
            const float x = rhs[(in ? c[h][st] : 0) * k + nb + 16 * nn + i];
            bv[h][n][st] = in ? x : 0.0f;
          }
      // keep the step's loads ahead of its MFMAs (left alone, the compiler
      // interleaves load, wait, MFMA)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int h = 0; h < CH; ++h)
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int st = 0; st < 4; ++st)
            acc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[h][st],
                                                          bv[h][n][st], acc[n],
                                                          0, 0, 0);
    }
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        part[wave][n][v][l] = acc[n][v];
    __syncthreads();
    if (wave < ntiles) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w)
          sum += part[w][wave][v][l];
        const int rr = 4 * g + v;
        if (rr < nt) {
          out[(int64_t)(r0 + rr) * k + nb + 16 * wave + i] = sum;
          nonfinite |= !__builtin_isfinite(sum);
        }
      }
      if (__builtin_amdgcn_ballot_w64(nonfinite) != 0 && lane_id() == 0)
        nonfinite_out = 1;
    }
    __syncthreads();
  }
  // The tile's rows share each MFMA's B operand, so an inf or NaN in a B row
  // that a shorter row leaves out reaches that row as 0 * inf; the last row
  // holds every entry, so the tile then has a non-finite output.  Such a
  // tile is recomputed row by row, adding exactly each row's own entries.
  if (nonfinite_out != 0) // workgroup-uniform after the barrier above
    for (int r = r0 + wave; r < r0 + nt; r += W)
      spmm_row_wave(ro, col, val, rhs, out, r, k);
}


// SpMM over 16-row tiles, bf16 (k % 64 == 0; rhs and out 8-byte aligned).
// The fp32 kernel's tiles, waves, structure check and fallbacks, with one
// v_mfma_f32_16x16x16_bf16 per 16 stored entries and output tile: lane
// (i, g) supplies val[ro[r0+i] + t0+4g .. t0+4g+3] (zero past the row), and
// the four output tiles of a 64-column block interleave their columns (tile
// n's column j is column 4j + n of the block), so one 64-bit load of an rhs
// row gives a lane its B values for all four tiles.
template <int W>
__global__ __launch_bounds__(64 * W) void spmm_tile_mfma_bf16(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const uint16_t *__restrict__ val, const uint16_t *__restrict__ rhs,
    uint16_t *__restrict__ out, int32_t rows, int64_t k) {
  constexpr int CH = 2; // 16-entry chunks per step
  __shared__ float part[W][4][4][kWave]; // [wave][n tile][v][lane]
  if (block_id() * 16 >= rows)
    return; // a folded grid's surplus workgroup (workgroup-uniform)
  const int r0 = (int)block_id() * 16;
  const int nt = std::min(16, rows - r0);
  const int wave = wave_in_group();
  const int l = lane_id(), i = l & 15, g = l >> 4;
  const int last = r0 + nt - 1;
  const int32_t bl = ro[last];
  const int32_t len_last = ro[last + 1] - bl;
  const int ic = i < nt ? i : nt - 1;
  const int32_t ra = ro[r0 + ic];
  const int32_t la = i < nt ? ro[r0 + ic + 1] - ra : 0;
  __shared__ int verdict;
  __shared__ int nonfinite_out;
  if (threadIdx.x == 0)
    nonfinite_out = 0;
  if (!tile_prefix_ok_block(ro, col, r0, nt, &verdict)) {
    for (int r = r0 + wave; r < r0 + nt; r += W)
      spmm_row_wave(ro, col, val, rhs, out, r, k);
    return;
  }
  bool nonfinite = false;
  for (int64_t nb = 0; nb < k; nb += 64) {
    v4f acc[4];
#pragma unroll
    for (int n = 0; n < 4; ++n)
      acc[n] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int32_t t0 = wave * 16 * CH; t0 < len_last; t0 += W * 16 * CH) {
      v2u a[CH], bq[CH][4];
#pragma unroll
      for (int h = 0; h < CH; ++h) {
        float av[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const int32_t t = t0 + 16 * h + 4 * g + st;
          const int32_t tc = std::min(t, len_last - 1); // len_last > 0 here
          const float x = tof(val[t < la ? ra + t : bl + tc]);
          const int64_t cx = col[bl + tc];
          av[st] = t < la ? x : 0.0f;
          // rhs[c][nb + 4i .. nb + 4i + 3] (row 0, zeroed, past len_last)
          const v2u y = *reinterpret_cast<const v2u *>(
              rhs + (t < len_last ? cx : 0) * k + nb + 4 * i);
          bq[h][st] = t < len_last ? y : v2u{0u, 0u};
        }
        a[h] = v2u{pack_bf16x2(av[0], av[1]), pack_bf16x2(av[2], av[3])};
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int h = 0; h < CH; ++h)
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const v2u bn = v2u{bf16_pair(bq[h][0], bq[h][1], n),
                             bf16_pair(bq[h][2], bq[h][3], n)};
          acc[n] = mfma_16x16x16_bf16(a[h], bn, acc[n]);
        }
    }
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        part[wave][n][v][l] = acc[n][v];
    __syncthreads();
    if (wave < 4) {
      // wave w finishes rows 4g + w, columns nb + 4i .. nb + 4i + 3
      float o[4];
      bool nf = false;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w)
          sum += part[w][n][wave][l];
        o[n] = sum;
        nf |= !__builtin_isfinite(sum);
      }
      const int rr = 4 * g + wave;
      if (rr < nt) {
        *reinterpret_cast<v2u *>(out + (int64_t)(r0 + rr) * k + nb + 4 * i) =
            v2u{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
        nonfinite |= nf;
      }
      if (__builtin_amdgcn_ballot_w64(nonfinite) != 0 && lane_id() == 0)
        nonfinite_out = 1;
    }
    __syncthreads();
  }
  if (nonfinite_out != 0) // workgroup-uniform after the barrier above
    for (int r = r0 + wave; r < r0 + nt; r += W)
      spmm_row_wave(ro, col, val, rhs, out, r, k);
}

// wave-per-row-tile with the RHS rows staged in LDS (Wave64 extension
// wave-per-row-tile-lds; fp32, k % 4 == 0, tile % 4 == 0, rhs 16-byte
// aligned): the "dense RHS tiles in LDS" form of the row tile.  A wave owns
// one (row, tile) unit, its lanes split into PL = 64 / CL position groups of
// CL column lanes (4 columns each).  Per step every group takes U
// positions; the 16-byte RHS slices of all of them go from global memory
// straight into LDS with global_load_lds_dwordx4 (lane l's bytes land in
// slot l of the step's 1 KB), so no VGPR holds them in flight.  After the
// wave's loads complete, each lane reads its slots back and accumulates; the
// groups' partial sums meet in an xor butterfly.  Configuration 3 measured it
// slower than the register form: the RHS rows are gathered at random and
// each is used once, so LDS adds a round trip and no reuse.
constexpr int kLdsTileSteps = 4;

template <int CL>
__global__ __launch_bounds__(256) void spmm_row_tile_lds(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ rhs,
    float *__restrict__ out, int64_t rows, int64_t k, int32_t tile,
    int64_t tiles_per_row) {
  constexpr int PL = kWave / CL, U = kLdsTileSteps;
  __shared__ v4f stage[4][U][kWave];
  const int wave = wave_in_group(), l = lane_id();
  const int64_t unit = block_id() * 4 + wave;
  if (unit >= rows * tiles_per_row)
    return; // wave-uniform; the kernel has no workgroup barrier
  const int64_t r = unit / tiles_per_row;
  const int64_t c0 = (unit - r * tiles_per_row) * tile;
  const int pl = l / CL, cl = l % CL;
  const int64_t cb = c0 + 4 * cl;
  const bool col_ok = cb + 4 <= std::min<int64_t>(c0 + tile, k);
  // lanes past the tile load (and ignore) the tile's first columns
  const int64_t cload = col_ok ? cb : c0;
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  const int32_t s = ro[r], e = ro[r + 1];
  for (int32_t p0 = s; p0 < e; p0 += PL * U) {
    float v[U];
    int64_t cc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int32_t q = p0 + pl + u * PL;
      const int32_t qc = q < e ? q : e - 1; // always a position of the row
      const float x = val[qc];
      v[u] = q < e ? x : 0.0f;
      cc[u] = col[qc];
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      __builtin_amdgcn_global_load_lds(
          (const void *)(rhs + cc[u] * k + cload),
          (void __attribute__((address_space(3))) *)&stage[wave][u][0], 16,
          0, 0);
    __builtin_amdgcn_s_waitcnt(0); // the LDS-direct loads have landed
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int u = 0; u < U; ++u)
      acc += v[u] * stage[wave][u][l];
    __builtin_amdgcn_wave_barrier(); // slots read before the next step
  }
#pragma unroll
  for (int off = CL; off < kWave; off <<= 1) {
    acc.x += __shfl_xor(acc.x, off, kWave);
    acc.y += __shfl_xor(acc.y, off, kWave);
    acc.z += __shfl_xor(acc.z, off, kWave);
    acc.w += __shfl_xor(acc.w, off, kWave);
  }
  if (pl == 0 && col_ok)
    st4_nt(out + r * k + cb, acc);
}

// Row-owner SpMM for wide rhs (Wave64 extension, k % 4 == 0).
//
// The nonzeros are cut into chunks of `chunk` positions; wave w owns the
// rows whose first position falls in its chunk (rows starting past the last
// chunk, i.e. trailing empty rows, belong to the last one), so every output
// row has exactly one writer: plain 128-bit stores, no zero fill, no
// atomics, and the row assignment is balanced by nonzeros, not by rows.  The
// wave computes one row at a time: its 64 lanes form PL = 64/CL groups of CL
// lanes, each lane holding 4 output columns of the CL*4-column tile; the
// groups take positions s+g, s+g+PL, ... U at a time (U = 16 for rows longer
// than 512 positions, 4 otherwise), and the groups' partial rows meet in an
// xor butterfly.
template <int CL, typename T>
__global__ __launch_bounds__(256) void spmm_row_owner(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const T *__restrict__ val, const T *__restrict__ rhs,
    T *__restrict__ out, int32_t rows, int32_t nnz, int64_t k,
    int64_t chunk, int64_t chunks, int64_t tiles) {
  constexpr int PL = kWave / CL;
  const int64_t wave =
      block_id() * (blockDim.x / kWave) + wave_in_group();
  if (wave >= chunks * tiles)
    return;
  const int64_t c = wave / tiles;
  const int64_t t = wave - c * tiles;
  const int lane = lane_id();
  const int vl = lane / CL, cl = lane % CL;
  const int64_t cb = t * (CL * 4) + (int64_t)cl * 4;
  const bool col_ok = cb < k;
  // owned rows: first r with ro[r] >= c*chunk .. (last chunk: to rows)
  const int r0 = 1 + row_search_uniform(ro, 0u, (uint32_t)rows + 1u,
                                         (int32_t)(c * chunk) - 1);
  const int r1 = c == chunks - 1
                     ? rows
                     : 1 + row_search_uniform(ro, (uint32_t)r0,
                                              (uint32_t)rows + 1u,
                                              (int32_t)((c + 1) * chunk) - 1);
  for (int r = r0; r < r1 && r < rows; ++r) {
    const int32_t s = ro[r], e = ro[r + 1];
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    if (col_ok) {
      if (e - s > 512) {
        constexpr int U = 16;
        for (int32_t p = s + vl; p < e; p += PL * U) {
          v4f b[U];
          float v[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int32_t q = p + u * PL;
            v[u] = q < e ? tof(ld_stream(val + q)) : 0.0f;
            const int64_t cc = q < e ? ld_stream(col + q) : 0;
            b[u] = ld4(rhs + cc * k + cb);
          }
#pragma unroll
          for (int u = 0; u < U; ++u)
            acc += v[u] * b[u];
        }
      } else {
        constexpr int U = 4;
        for (int32_t p = s + vl; p < e; p += PL * U) {
          v4f b[U];
          float v[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int32_t q = p + u * PL;
            v[u] = q < e ? tof(ld_stream(val + q)) : 0.0f;
            const int64_t cc = q < e ? ld_stream(col + q) : 0;
            b[u] = ld4(rhs + cc * k + cb);
          }
#pragma unroll
          for (int u = 0; u < U; ++u)
            acc += v[u] * b[u];
        }
      }
    }
#pragma unroll
    for (int off = CL; off < kWave; off <<= 1) {
      acc.x += __shfl_xor(acc.x, off, kWave);
      acc.y += __shfl_xor(acc.y, off, kWave);
      acc.z += __shfl_xor(acc.z, off, kWave);
      acc.w += __shfl_xor(acc.w, off, kWave);
    }
    if (vl == 0 && col_ok)
      st4_nt(out + (int64_t)r * k + cb, acc);
  }
}

template <int V, int CL, int G, typename T>
void launch_tile(int64_t grid, int64_t B, hipStream_t st, const int32_t *ro,
                 const int32_t *col, const T *val, const T *rhs, T *out,
                 int64_t rows, int64_t k, int32_t tile, int64_t tpr) {
  hipLaunchKernelGGL((spmm_row_tile<V, CL, G, T>), sw::grid_dim(grid, B),
                     dim3((unsigned)B), 0, st, ro, col, val, rhs, out, rows, k,
                     tile, tpr);
}

template <int V, int CL, typename T>
void dispatch_g(int G, int64_t rows, int64_t tpr, int64_t B, hipStream_t st,
                const int32_t *ro, const int32_t *col, const T *val,
                const T *rhs, T *out, int64_t k, int32_t tile,
                int64_t *grid_out) {
  int64_t units = rows * tpr;
  int64_t grid = std::max<int64_t>(sw::ceil_div(units, B / G), 1);
  *grid_out = grid;
  if (grid > sw::grid_row(B) * sw::kMaxGridY)
    return; // the caller's check_grid reports it
#define SW_TILE_CASE(GG)                                                      \
  case GG:                                                                    \
    if constexpr (GG >= CL)                                                   \
      launch_tile<V, CL, (GG >= CL ? GG : CL), T>(grid, B, st, ro, col, val,  \
                                                  rhs, out, rows, k, tile,    \
                                                  tpr);                       \
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

int launch_fill_zero(float *y, int64_t n, int64_t block, hipStream_t st);
int launch_position_init(const int32_t *ro, float *out, int64_t rows,
                         int64_t k, int64_t chunk, int64_t P, int64_t units,
                         int64_t waves, hipStream_t st);

// The mappings that need no partial sums in the output: thread-per-output,
// row-tile-mfma, wave-per-row-balanced and wave-per-row-tile, for fp32 and
// bf16.  Returns 1 (and sets *rc) when it handled the mapping.
template <typename T>
bool launch_spmm_rows(const int32_t *ro, const int32_t *col, const T *val,
                      const T *rhs, T *out, int64_t rows, int64_t rhs_rows,
                      int64_t nnz, int64_t k, const sw_options &o,
                      const char *what, hipStream_t st, int *rc) {
  const int64_t B = o.spmm_block_size;
  // vector rhs / out access: 16 bytes (fp32) or 8 bytes (bf16) per 4 columns
  auto vec_ok = [](const void *p) {
    return (reinterpret_cast<uintptr_t>(p) & (4 * sizeof(T) - 1)) == 0;
  };
  if (streq(o.spmm_mapping, "thread-per-output")) {
    int64_t grid = std::max<int64_t>(ceil_div(rows * k, B), 1);
    *rc = check_grid(grid, B, what);
    if (*rc)
      return true;
    dim3 g = grid_dim(grid, B), b((unsigned)B);
    const bool row = k % kWave == 0 && B % kWave == 0 && rows <= INT32_MAX;
    if (narrow_offsets(rhs_rows, k) && row)
      hipLaunchKernelGGL((spmm_thread_per_output<true, true, T>), g, b, 0, st,
                         ro, col, val, rhs, out, rows, k);
    else if (narrow_offsets(rhs_rows, k))
      hipLaunchKernelGGL((spmm_thread_per_output<true, false, T>), g, b, 0,
                         st, ro, col, val, rhs, out, rows, k);
    else if (row)
      hipLaunchKernelGGL((spmm_thread_per_output<false, true, T>), g, b, 0,
                         st, ro, col, val, rhs, out, rows, k);
    else
      hipLaunchKernelGGL((spmm_thread_per_output<false, false, T>), g, b, 0,
                         st, ro, col, val, rhs, out, rows, k);
    *rc = launch_check("thread-per-output SpMM kernel");
    return true;
  }
  if (streq(o.spmm_mapping, "row-tile-mfma")) {
    int64_t grid = ceil_div(rows, 16);
    if constexpr (sizeof(T) == 4) {
      if (k % 16 == 0) {
        *rc = check_grid(grid, 512, what);
        if (*rc)
          return true;
        hipLaunchKernelGGL(spmm_tile_mfma<8>, grid_dim(grid, 512), dim3(512),
                           0, st, ro, col, val, rhs, out, (int32_t)rows, k);
        *rc = launch_check("SpMM tile MFMA kernel");
        return true;
      }
    } else {
      if (k % 64 == 0 && vec_ok(rhs) && vec_ok(out)) {
        *rc = check_grid(grid, 512, what);
        if (*rc)
          return true;
        hipLaunchKernelGGL(spmm_tile_mfma_bf16<8>, grid_dim(grid, 512),
                           dim3(512), 0, st, ro, col, val, rhs, out,
                           (int32_t)rows, k);
        *rc = launch_check("SpMM tile MFMA kernel");
        return true;
      }
    }
  }
  if ((streq(o.spmm_mapping, "wave-per-row-balanced") ||
       (sizeof(T) == 2 && streq(o.spmm_mapping, "row-tile-mfma"))) &&
      k % 4 == 0 && vec_ok(rhs) && vec_ok(out)) {
    const int CL = std::min(16, next_pow2((int)std::min<int64_t>(k / 4, 16)));
    const int64_t chunk = 64 * o.spmm_positions_per_lane;
    const int64_t chunks = std::max<int64_t>(ceil_div(nnz, chunk), 1);
    const int64_t tiles = ceil_div(k, (int64_t)CL * 4);
    // the kernel is compiled for at most 256 threads per workgroup
    const int64_t OB = std::min<int64_t>(B, 256);
    const int64_t grid = ceil_div(chunks * tiles, OB / 64);
    *rc = check_grid(grid, OB, what);
    if (*rc)
      return true;
#define SW_OWNER(CC)                                                          \
  case CC:                                                                    \
    hipLaunchKernelGGL((spmm_row_owner<CC, T>), grid_dim(grid, OB),           \
                       dim3((unsigned)OB), 0, st, ro, col, val, rhs, out,     \
                       (int32_t)rows, (int32_t)nnz, k, chunk, chunks, tiles); \
    break;
    switch (CL) {
      SW_OWNER(1) SW_OWNER(2) SW_OWNER(4) SW_OWNER(8) SW_OWNER(16)
    }
#undef SW_OWNER
    *rc = launch_check("row-owner SpMM kernel");
    return true;
  }
  if constexpr (sizeof(T) == 4) {
    const int64_t Tt = o.spmm_tile_size;
    if (streq(o.spmm_mapping, "wave-per-row-tile-lds") && k % 4 == 0 &&
        Tt % 4 == 0 && aligned16(rhs) && aligned16(out)) {
      const int64_t tpr = ceil_div(k, Tt);
      const int64_t grid = std::max<int64_t>(ceil_div(rows * tpr, 4), 1);
      *rc = check_grid(grid, 256, what);
      if (*rc)
        return true;
      const int CL = next_pow2((int)(Tt / 4));
#define SW_LDS_TILE(CC)                                                       \
  case CC:                                                                    \
    hipLaunchKernelGGL(spmm_row_tile_lds<CC>, grid_dim(grid, 256),            \
                       dim3(256), 0, st, ro, col, val, rhs, out, rows, k,     \
                       (int32_t)Tt, tpr);                                     \
    break;
      switch (CL) { SW_LDS_TILE(1) SW_LDS_TILE(2) SW_LDS_TILE(4) SW_LDS_TILE(8) }
#undef SW_LDS_TILE
      *rc = launch_check("LDS-staged row-tile SpMM kernel");
      return true;
    }
  }
  // wave-per-row-tile-lds outside its shapes takes the register row tile
  const bool row_tile = streq(o.spmm_mapping, "wave-per-row-tile") ||
                        streq(o.spmm_mapping, "wave-per-row-tile-lds");
  if (!row_tile && sizeof(T) == 4)
    return false; // fp32: the position schedule
  // wave-per-row-tile (bf16 also for the shapes the mappings above decline)
  const int T_ = (int)o.spmm_tile_size;
  const int64_t tpr = ceil_div(k, T_);
  const bool vec = (T_ % 4 == 0) && (k % 4 == 0) && vec_ok(rhs) && vec_ok(out);
  const int V = vec ? 4 : 1;
  const int CL = next_pow2(ceil_div(T_, V));
  const int G = std::max<int>((int)o.spmm_lanes_per_row, CL);
  int64_t grid = 0;
  const int32_t tile = (int32_t)T_;
#define SW_CL_CASE(VV, CC)                                                    \
  if (V == VV && CL == CC)                                                    \
    dispatch_g<VV, CC, T>(G, rows, tpr, B, st, ro, col, val, rhs, out, k,     \
                          tile, &grid);
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
  if (grid == 0) {
    *rc = fail(SW_ERR_INVALID_OPTION,
               "no wave-per-row-tile kernel for tile size %d", T_);
    return true;
  }
  *rc = check_grid(grid, B, what);
  if (*rc)
    return true;
  *rc = launch_check("wave-per-row-tile SpMM kernel");
  return true;
}

int launch_spmm(const int32_t *ro, const int32_t *col, const float *val,
                const float *rhs, float *out, int64_t rows, int64_t rhs_rows,
                int64_t nnz, int64_t k, const sw_options &o, const char *what,
                hipStream_t st) {
  const int64_t B = o.spmm_block_size;
  int rc = SW_OK;
  if (launch_spmm_rows<float>(ro, col, val, rhs, out, rows, rhs_rows, nnz, k,
                              o, what, st, &rc))
    return rc;
  if (streq(o.spmm_mapping, "thread-per-position")) {
    int64_t n_out = rows * k;
    if (n_out > 0) {
      int64_t g0 = ceil_div(n_out, o.position_block_size);
      int rc = check_grid(g0, o.position_block_size, what);
      if (rc)
        return rc;
      hipLaunchKernelGGL(spmm_fill_zero, grid_dim(g0, o.position_block_size),
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
    int rc = check_grid(grid, B, what);
    if (rc)
      return rc;
    hipLaunchKernelGGL(spmm_thread_position, grid_dim(grid, B),
                       dim3((unsigned)B), 0, st, ro, col, val, rhs, out,
                       (int32_t)rows, k, iters, chunk);
    return launch_check("thread-per-position SpMM kernel");
  }
  // wave-per-position, and row-tile-mfma with k not a multiple of 16 and
  // wave-per-row-balanced without 128-bit rows: the position schedule
  {
    const bool v4 = (k % 4 == 0) && aligned16(rhs) && aligned16(out);
    const int V = v4 ? 4 : 1;
    const int CL = std::min(16, next_pow2((int)std::min<int64_t>(
                                    ceil_div(k, V), 16)));
    const int P = (int)o.spmm_positions_per_lane;
    const int64_t PL = 64 / CL;
    const int64_t units = ceil_div(nnz, P);
    const int64_t chunks = ceil_div(units, PL);
    const int64_t tiles = ceil_div(k, (int64_t)CL * V);
    const int64_t grid = ceil_div(chunks * tiles, B / 64);
    int rc = check_grid(grid, B, what);
    if (rc)
      return rc;
    // rows of at least one 128-byte line are stored; narrower rows go
    // through atomics into a fully zeroed output
    const bool store_rows = V == 4 && CL >= 8 && k >= 32;
    if (store_rows)
      // chunks of PL*P positions: zero the rows that span chunks, and the
      // empty rows
      rc = launch_position_init(ro, out, rows, k, PL * P, P, units,
                                std::max<int64_t>(chunks, 1), st);
    else
      rc = launch_fill_zero(out, rows * k, B, st);
    if (rc)
      return rc;
    if (nnz == 0)
      return SW_OK;
    const bool vec = aligned16(col) && aligned16(val);
    bool ok = false;
#define SW_WPOS(VV, CC)                                                       \
  if (V == VV && CL == CC)                                                    \
    ok = dispatch_wpos_p<VV, CC>(P, grid, B, st, ro, col, val, rhs, out,      \
                                 (int32_t)rows, (int32_t)nnz, k, units,       \
                                 chunks, tiles, vec, store_rows);
    SW_WPOS(4, 1) SW_WPOS(4, 2) SW_WPOS(4, 4) SW_WPOS(4, 8) SW_WPOS(4, 16)
    SW_WPOS(1, 1) SW_WPOS(1, 2) SW_WPOS(1, 4) SW_WPOS(1, 8) SW_WPOS(1, 16)
#undef SW_WPOS
    if (!ok)
      return fail(SW_ERR_INVALID_OPTION, "no wave-per-position SpMM kernel");
    return launch_check("wave-per-position SpMM kernel");
  }
}

int launch_spmm(const int32_t *ro, const int32_t *col, const uint16_t *val,
                const uint16_t *rhs, uint16_t *out, int64_t rows,
                int64_t rhs_rows, int64_t nnz, int64_t k, const sw_options &o,
                const char *what, hipStream_t st) {
  int rc = check_bf16_spmm_mapping(o);
  if (rc)
    return rc;
  launch_spmm_rows<uint16_t>(ro, col, val, rhs, out, rows, rhs_rows, nnz, k,
                             o, what, st, &rc);
  return rc;
}

} // namespace sw

namespace {

template <typename T>
int spmm_entry(const int32_t *row_offsets, const int32_t *column_indices,
               const T *values, const T *rhs, T *output, int64_t rows,
               int64_t cols, int64_t nnz, int64_t k, const sw_options *opts,
               void *stream) {
  sw::clear_error();
  sw_options o;
  int rc = sw::resolve_options(opts, &o);
  if (rc)
    return rc;
  rc = sw::check_csr(row_offsets, column_indices, values, rows, nnz, true);
  if (!rc)
    rc = sw::check_value_alignment(sizeof(T), {values, rhs, output});
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
                         rows, cols, nnz, k, o, "SpMM", sw::as_stream(stream));
}

} // namespace

extern "C" int sw_spmm_csr_f32(const int32_t *row_offsets,
                               const int32_t *column_indices,
                               const float *values, const float *rhs,
                               float *output, int64_t rows, int64_t cols,
                               int64_t nnz, int64_t k, const sw_options *opts,
                               void *stream) {
  return spmm_entry<float>(row_offsets, column_indices, values, rhs, output,
                           rows, cols, nnz, k, opts, stream);
}

extern "C" int sw_spmm_csr_bf16(const int32_t *row_offsets,
                                const int32_t *column_indices,
                                const uint16_t *values, const uint16_t *rhs,
                                uint16_t *output, int64_t rows, int64_t cols,
                                int64_t nnz, int64_t k, const sw_options *opts,
                                void *stream) {
  return spmm_entry<uint16_t>(row_offsets, column_indices, values, rhs,
                              output, rows, cols, nnz, k, opts, stream);
}
