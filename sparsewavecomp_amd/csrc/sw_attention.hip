// sparsewave.sddmm, csr_row_reduce, csr_rowwise_map and the six-kernel
// sparse-attention chain on gfx950.
//
// Reference kernels (generated IR):
//   sddmm            ThreadPerRowSDDMMPattern, SparseWaveToGPU.cpp:667-750
//   csr_row_reduce   ThreadPerRowCSRRowReducePattern, SparseWaveToGPU.cpp:752-818
//   csr_rowwise_map  ThreadPerRowCSRRowwiseMapPattern, SparseWaveToGPU.cpp:820-878
//   attention chain  examples/pytorch/integration/SparseAttentionToSparseWave.cpp:230-315
//
// Each op has the reference's thread-per-row kernel and a Wave64 kernel that
// gives a row to a wave (lanes over positions: coalesced CSR reads and, for
// SDDMM, coalesced reads of the dense right-hand side when a row's columns
// are contiguous, as in block masks).
#include "sw_device.h"
#include "sw_internal.h"
#include "sw_sddmm_tile64.h"

#include <algorithm>
#include <cmath>
#include <type_traits>

using namespace swd;

namespace sw {
int launch_spmm(const int32_t *ro, const int32_t *col, const float *val,
                const float *rhs, float *out, int64_t rows, int64_t rhs_rows,
                int64_t nnz, int64_t k, const sw_options &o, const char *what,
                hipStream_t st);
int launch_spmm(const int32_t *ro, const int32_t *col, const uint16_t *val,
                const uint16_t *rhs, uint16_t *out, int64_t rows,
                int64_t rhs_rows, int64_t nnz, int64_t k, const sw_options &o,
                const char *what, hipStream_t st);
}

namespace {

// waves per 16-row SDDMM tile (4: 20.9 us on configuration 5; 8: 24.6 us)
constexpr int kSddmmTileWaves = 4;

__device__ __forceinline__ float combine_sddmm(int kind, float sample,
                                               float dot, float alpha,
                                               float beta) {
  if (kind == SW_SDDMM_MUL)
    return sample * dot;
  if (kind == SW_SDDMM_AFFINE)
    return sample * beta + dot * alpha;
  return dot;
}

// arith.maximumf: NaN propagates, +0 is above -0 -- the IEEE 754-2019
// maximum, which gfx950 computes in one v_maximum3_f32 (llvm.maximum)
__device__ __forceinline__ float maximumf(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}

// A result as its op stores it: unchanged in fp32, rounded to bf16 (and
// widened back) for bf16 buffers.  The fused bf16 kernels round each
// intermediate where the separate ops would store it, so every bf16 schedule
// computes the six ops on bf16 buffers.
template <typename T>
__device__ __forceinline__ float as_stored(float v) {
  if constexpr (sizeof(T) == 4)
    return v;
  else
    return bf16_to_f32(f32_to_bf16(v));
}

__device__ __forceinline__ float map_value(int kind, float v, float rv) {
  switch (kind) {
  case SW_MAP_EXP_SUB:
    return expf(v - rv);
  case SW_MAP_DIV:
    return v / rv;
  case SW_MAP_SUB:
    return v - rv;
  default:
    return v * rv;
  }
}

// ---- SDDMM -----------------------------------------------------------------
// Thread-per-row (the reference's mapping and launch).  TKB > 0 (kdim = 64
// TKB, a block size that is a multiple of 64, for bf16 a 16-byte aligned
// lhs, which the host checks): each wave first tries its 64 consecutive
// rows as one matrix-core tile (sw_sddmm_tile64.h); rows of a tile without
// the shared column prefix are then computed by their own threads as below.
template <typename T, int RP, int LB, int TKB = 0>
__global__ __launch_bounds__(LB) void sddmm_thread_per_row(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const T *__restrict__ val, const T *__restrict__ lhs,
    const T *__restrict__ rhs, T *__restrict__ out, int32_t rows,
    int64_t cols, int32_t kdim, int kind, float alpha, float beta) {
  if constexpr (TKB > 0) {
    __shared__ int32_t lcol[LB / kWave][sw_tile64::kTileCols];
    const int64_t r0 = block_id() * blockDim.x +
                       (int64_t)wave_in_group() * kWave;
    if (r0 >= rows)
      return; // wave-uniform
    auto combine = [&](float sample, float dot) {
      return combine_sddmm(kind, sample, dot, alpha, beta);
    };
    if (val != nullptr ? sw_tile64::sddmm_tile64<T, TKB, true, true>(
                             ro, col, val, lhs, rhs, out, rows, cols, r0,
                             lcol[wave_in_group()], combine)
                       : sw_tile64::sddmm_tile64<T, TKB, false, false>(
                             ro, col, val, lhs, rhs, out, rows, cols, r0,
                             lcol[wave_in_group()], combine))
      return;
  }
  int64_t r = block_id() * blockDim.x + threadIdx.x;
  if (r >= rows)
    return;
  const T *a = lhs + r * kdim;
  // RP positions at a time, sixteen terms of each in flight: the
  // launch has one thread per row (8192 rows are 128 waves), so a row is a
  // chain of memory trips and registers are plentiful (LB, the launch
  // bound, sets how many).  Each position's dot is still added term by term
  // in order.
  const int32_t e = ro[r + 1];
  for (int32_t p = ro[r]; p < e; p += RP) {
    int64_t c[RP];
    float dot[RP];
#pragma unroll
    for (int j = 0; j < RP; ++j) {
      c[j] = col[std::min(p + j, e - 1)];
      dot[j] = 0.0f;
    }
    // the dot products of the step's positions, whose columns are cc
    auto dots = [&](const auto &cc) __attribute__((always_inline)) {
      int32_t i = 0;
      for (; i + 15 < kdim; i += 16) {
        float av[16], bv[RP][16];
#pragma unroll
        for (int u = 0; u < 16; ++u)
          av[u] = ldv(a + i + u);
#pragma unroll
        for (int j = 0; j < RP; ++j)
#pragma unroll
          for (int u = 0; u < 16; ++u)
            bv[j][u] = ldv(rhs + (int64_t)(i + u) * cols + cc[j]);
#pragma unroll
        for (int j = 0; j < RP; ++j)
#pragma unroll
          for (int u = 0; u < 16; ++u)
            dot[j] = __builtin_fmaf(av[u], bv[j][u], dot[j]);
      }
      for (; i < kdim; ++i) {
        const float av = ldv(a + i);
#pragma unroll
        for (int j = 0; j < RP; ++j)
          dot[j] = __builtin_fmaf(av, ldv(rhs + (int64_t)i * cols + cc[j]),
                                  dot[j]);
      }
    };
    // fp32: rows of a block-structured mask share their columns position
    // by position (83% of configuration 5's steps).  When every active
    // lane's step has the first active lane's columns, the rhs addresses are
    // wave-uniform and the rhs values scalar loads (configuration 5: 479 ->
    // 416 us).  The products and their order are the same either way.  (bf16
    // elements at odd columns cannot be scalar loads; the test alone made
    // it slower, 423 -> 475 us.)
    bool uniform = false;
    if constexpr (sizeof(T) == 4) {
      bool same = true;
#pragma unroll
      for (int j = 0; j < RP; ++j)
        same &= (int32_t)c[j] ==
                __builtin_amdgcn_readfirstlane((int32_t)c[j]);
      uniform = __builtin_amdgcn_ballot_w64(!same) == 0;
    }
    if (uniform) {
      int32_t cu[RP];
#pragma unroll
      for (int j = 0; j < RP; ++j)
        cu[j] = __builtin_amdgcn_readfirstlane((int32_t)c[j]);
      dots(cu);
    } else {
      dots(c);
    }
#pragma unroll
    for (int j = 0; j < RP; ++j)
      if (p + j < e)
        stv(out + p + j,
            combine_sddmm(kind, val != nullptr ? ldv(val + p + j) : 0.0f,
                          dot[j], alpha, beta));
  }
}

// One wave computes the SDDMM entries of row r: lane l takes positions
// start+l, start+l+64, ...; the row of lhs is held 64 values at a time, one
// per lane, and broadcast with v_readlane.
template <typename T>
__device__ __forceinline__ void sddmm_row_wave(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const T *__restrict__ val, const T *__restrict__ lhs,
    const T *__restrict__ rhs, T *__restrict__ out, int64_t r,
    int64_t cols, int32_t kdim, int kind, float alpha, float beta) {
  const int l = lane_id();
  const int32_t s = ro[r], e = ro[r + 1];
  const T *a = lhs + r * kdim;
  for (int32_t p0 = s; p0 < e; p0 += 4 * kWave) {
    float dot[4] = {0.f, 0.f, 0.f, 0.f};
    int64_t c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int32_t p = p0 + j * kWave + l;
      c[j] = p < e ? (int64_t)col[p] : 0;
    }
    for (int32_t i0 = 0; i0 < kdim; i0 += kWave) {
      const float mine = (i0 + l < kdim) ? ldv(a + i0 + l) : 0.0f;
      const int n = std::min<int32_t>(kWave, kdim - i0);
      for (int t = 0; t < n; ++t) {
        const float av =
            __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), t));
        const T *rrow = rhs + (int64_t)(i0 + t) * cols;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          dot[j] = __builtin_fmaf(av, ldv(rrow + c[j]), dot[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int32_t p = p0 + j * kWave + l;
      if (p < e)
        stv(out + p, combine_sddmm(kind, val != nullptr ? ldv(val + p) : 0.0f,
                                   dot[j], alpha, beta));
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void sddmm_wave_per_row(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const T *__restrict__ val, const T *__restrict__ lhs,
    const T *__restrict__ rhs, T *__restrict__ out, int32_t rows,
    int64_t cols, int32_t kdim, int kind, float alpha, float beta) {
  const int64_t r = block_id() * (blockDim.x / kWave) +
                    wave_in_group();
  if (r >= rows)
    return; // wave-uniform
  sddmm_row_wave(ro, col, val, lhs, rhs, out, r, cols, kdim, kind, alpha,
                 beta);
}

// SDDMM over 16-row tiles on the matrix cores (kdim = 64 * KB).
//
// A workgroup of W waves owns rows r0 .. r0+15.  When every row's columns
// are a prefix of the last row's (tile_prefix_ok_block), the tile's dot products
// for 16 of the last row's columns at a time are one 16 x 16 x kdim product
//   D = lhs[r0 .. r0+15][:] * rhs[:][c_t0 .. c_t0+15]
// computed with v_mfma_f32_16x16x4_f32 (lane (i, g) supplies
// lhs[r0+i][16g+s] at step s, lane (j, g) supplies rhs[16g+s][c_j]); wave w
// takes the column chunks w, w+W, ...  Each result lands at its CSR position
// ro[row] + t when t is inside that row.  Tiles without the shared structure
// are computed row by row on the vector ALUs.
//
// Latency: the row bounds and lhs rows are requested before the structure
// check waits, and a chunk pair's sampled values before its rhs loads wait
// (checking the structure inside the chunk loop instead measured slower).
template <int KB, int W>
__global__ __launch_bounds__(64 * W) void sddmm_tile_mfma(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ lhs,
    const float *__restrict__ rhs, float *__restrict__ out, int32_t rows,
    int64_t cols, int32_t kdim, int kind, float alpha, float beta) {
  if (block_id() * 16 >= rows)
    return; // a folded grid's surplus workgroup (workgroup-uniform)
  const int r0 = (int)block_id() * 16;
  const int nt = std::min(16, rows - r0);
  const int wave = wave_in_group();
  const int l = lane_id(), i = l & 15, g = l >> 4;
  // loads are unconditional from clamped, valid addresses, their values
  // selected afterwards (a guarded load becomes a branch that waits for it
  // on the spot)
  int32_t rb[4], rl[4];
  {
    int32_t b[5];
#pragma unroll
    for (int v = 0; v < 5; ++v)
      b[v] = ro[std::min(r0 + 4 * g + v, rows)];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      rb[v] = b[v];
      rl[v] = 4 * g + v < nt ? b[v + 1] - b[v] : 0;
    }
  }
  float qa[16 * KB];
  const int64_t qrow = (int64_t)std::min(r0 + i, rows - 1) * kdim;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      const float x = lhs[qrow + kb * 64 + 16 * g + st];
      qa[kb * 16 + st] = i < nt ? x : 0.0f;
    }
  __shared__ int verdict;
  if (!tile_prefix_ok_block(ro, col, r0, nt, &verdict)) {
    for (int r = r0 + wave; r < r0 + nt; r += W)
      sddmm_row_wave(ro, col, val, lhs, rhs, out, r, cols, kdim, kind, alpha,
                     beta);
    return;
  }
  const int last = r0 + nt - 1;
  const int32_t bl = ro[last];
  const int32_t len_last = ro[last + 1] - bl;
  // two column chunks per iteration (W chunks apart): two independent
  // accumulators and 32 outstanding rhs loads per lane
  for (int32_t t0 = wave * 16; t0 < len_last; t0 += 32 * W) {
    const int32_t t1 = t0 + 16 * W;
    const bool two = t1 < len_last; // wave-uniform
    const int32_t ta = t0 + i, tb = t1 + i;
    const int64_t cj0 = ta < len_last ? (int64_t)col[bl + ta] : 0;
    const int64_t cj1 = two && tb < len_last ? (int64_t)col[bl + tb] : 0;
    float s0[4], s1[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      // position bl is inside the last row, always a valid index
      const bool in0 = val != nullptr && ta < rl[v];
      const bool in1 = val != nullptr && two && tb < rl[v];
      const float x0 = val != nullptr ? val[in0 ? rb[v] + ta : bl] : 0.0f;
      const float x1 = val != nullptr ? val[in1 ? rb[v] + tb : bl] : 0.0f;
      s0[v] = in0 ? x0 : 0.0f;
      s1[v] = in1 ? x1 : 0.0f;
    }
    v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      float bv0[16], bv1[16];
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const float *rrow = rhs + (int64_t)(kb * 64 + 16 * g + st) * cols;
        bv0[st] = rrow[cj0];
        bv1[st] = two ? rrow[cj1] : 0.0f;
      }
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[kb * 16 + st], bv0[st],
                                                    acc0, 0, 0, 0);
        if (two)
          acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[kb * 16 + st],
                                                      bv1[st], acc1, 0, 0, 0);
      }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if (ta < rl[v])
        out[rb[v] + ta] = combine_sddmm(kind, s0[v], acc0[v], alpha, beta);
      if (two && tb < rl[v])
        out[rb[v] + tb] = combine_sddmm(kind, s1[v], acc1[v], alpha, beta);
    }
  }
}

template <bool MAX, typename T>
__global__ __launch_bounds__(1024) void row_reduce_thread(
    const int32_t *__restrict__ ro, const T *__restrict__ val,
    T *__restrict__ out, int32_t rows) {
  int64_t r = block_id() * blockDim.x + threadIdx.x;
  if (r >= rows)
    return;
  float acc = MAX ? -INFINITY : 0.0f;
  const int32_t e = ro[r + 1];
  int32_t p = ro[r];
  // sixteen loads in flight while that many remain (as unaligned vector
  // loads), combined in position order (a thread's row is a chain of memory
  // trips); the last partial step loads sixteen too, from positions clamped
  // to the row's last entry, and selects the ones in the row (one trip
  // instead of one per remaining entry)
  for (; p + 15 < e; p += 16) {
    T v[16];
    __builtin_memcpy(v, val + p, sizeof v);
#pragma unroll
    for (int u = 0; u < 16; ++u)
      acc = MAX ? maximumf(acc, tof(v[u])) : acc + tof(v[u]);
  }
  if (p < e) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      v[u] = ldv(val + (p + u < e ? p + u : e - 1));
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (MAX)
        acc = p + u < e ? maximumf(acc, v[u]) : acc;
      else
        acc = p + u < e ? acc + v[u] : acc;
  }
  stv(out + r, acc);
}

__device__ __forceinline__ float wave_max(float v) {
  v = maximumf(v, dpp_f<kQuadXor1>(-INFINITY, v));
  v = maximumf(v, dpp_f<kQuadXor2>(-INFINITY, v));
  v = maximumf(v, dpp_f<kRowHalfMirror>(-INFINITY, v));
  v = maximumf(v, dpp_f<kRowMirror>(-INFINITY, v));
  v = maximumf(v, swizzle_xor16(v));
  v = maximumf(v, shfl_xor32(v));
  return v;
}

template <bool MAX, typename T>
__global__ __launch_bounds__(256) void row_reduce_wave(
    const int32_t *__restrict__ ro, const T *__restrict__ val,
    T *__restrict__ out, int32_t rows) {
  const int64_t r = block_id() * (blockDim.x / kWave) +
                    wave_in_group();
  if (r >= rows)
    return;
  const int l = lane_id();
  float acc = MAX ? -INFINITY : 0.0f;
  for (int32_t p = ro[r] + l; p < ro[r + 1]; p += kWave)
    acc = MAX ? maximumf(acc, ldv(val + p)) : acc + ldv(val + p);
  acc = MAX ? wave_max(acc) : group_sum<kWave>(acc);
  if (l == 0)
    stv(out + r, acc);
}

// ---- row-wise map ----------------------------------------------------------
// (KIND a template argument: the map is straight-line code, with no switch
// per entry)
template <typename T, int KIND>
__global__ __launch_bounds__(1024) void rowwise_map_thread(
    const int32_t *__restrict__ ro, const T *val,
    const T *__restrict__ rowv, T *out, int32_t rows) {
  constexpr int kind = KIND;
  int64_t r = block_id() * blockDim.x + threadIdx.x;
  if (r >= rows)
    return;
  const float rv = ldv(rowv + r);
  const int32_t e = ro[r + 1];
  int32_t p = ro[r];
  // sixteen entries loaded before they are written back: out may be val
  // itself (in place), and each entry is read before its own write; both
  // as (unaligned) vector accesses, so that a lane's 16 entries take 4 (2
  // for bf16) memory instructions instead of 16.  The next 16 entries are
  // requested before this step's stores (the ranges are disjoint), so that
  // waiting for them does not wait for the stores as well (one counter
  // tracks both).
  if (p + 15 < e) {
    T v[16];
    __builtin_memcpy(v, val + p, sizeof v);
    for (; p + 31 < e; p += 16) {
      T next[16];
      __builtin_memcpy(next, val + p + 16, sizeof next);
#pragma unroll
      for (int u = 0; u < 16; ++u)
        stv(&v[u], map_value(kind, tof(v[u]), rv));
      __builtin_memcpy(out + p, v, sizeof v);
#pragma unroll
      for (int u = 0; u < 16; ++u)
        v[u] = next[u];
    }
#pragma unroll
    for (int u = 0; u < 16; ++u)
      stv(&v[u], map_value(kind, tof(v[u]), rv));
    __builtin_memcpy(out + p, v, sizeof v);
    p += 16;
  }
  // the last partial step: sixteen loads from positions clamped to the row's
  // last entry (one trip), then the stores of the entries in the row
  if (p < e) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      v[u] = ldv(val + (p + u < e ? p + u : e - 1));
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (p + u < e)
        stv(out + p + u, map_value(kind, v[u], rv));
  }
}

template <typename T>
__global__ __launch_bounds__(256) void rowwise_map_wave(
    const int32_t *__restrict__ ro, const T *val,
    const T *__restrict__ rowv, T *out, int32_t rows, int kind) {
  const int64_t r = block_id() * (blockDim.x / kWave) +
                    wave_in_group();
  if (r >= rows)
    return;
  const float rv = ldv(rowv + r);
  for (int32_t p = ro[r] + lane_id(); p < ro[r + 1]; p += kWave)
    stv(out + p, map_value(kind, ldv(val + p), rv));
}


// The four row ops of the attention chain fused (row max, exp(s - max), row
// sum, s / sum): one wave per row.  Rows of up to 64 * kSoftmaxRegs entries
// stay in registers between the ops (one read and one write of the scores);
// longer rows take a max pass and two read/write passes.  rowMaximum and
// rowSum are written as the separate ops would write them.
constexpr int kSoftmaxRegs = 8;

template <typename T>
__global__ __launch_bounds__(256) void row_softmax_wave(
    const int32_t *__restrict__ ro, T *scores, T *__restrict__ rmax,
    T *__restrict__ rsum, int32_t rows) {
  const int64_t r = block_id() * (blockDim.x / kWave) +
                    wave_in_group();
  if (r >= rows)
    return;
  const int l = lane_id();
  const int32_t s = ro[r], e = ro[r + 1];
  float m = -INFINITY;
  float sum = 0.0f;
  if (e > s && e - s <= kWave * kSoftmaxRegs) { // wave-uniform
    float v[kSoftmaxRegs];
#pragma unroll
    for (int j = 0; j < kSoftmaxRegs; ++j) {
      // unconditional load from a clamped index, then select (a guarded
      // load would wait on the spot)
      const int32_t p = s + l + j * kWave;
      const float x = ldv(scores + (p < e ? p : e - 1));
      v[j] = p < e ? x : -INFINITY;
      m = maximumf(m, v[j]);
    }
    m = wave_max(m);
#pragma unroll
    for (int j = 0; j < kSoftmaxRegs; ++j)
      if (s + l + j * kWave < e) {
        v[j] = as_stored<T>(expf(v[j] - m));
        sum += v[j];
      }
    sum = as_stored<T>(group_sum<kWave>(sum));
#pragma unroll
    for (int j = 0; j < kSoftmaxRegs; ++j) {
      const int32_t p = s + l + j * kWave;
      if (p < e)
        stv(scores + p, v[j] / sum);
    }
  } else {
    for (int32_t p = s + l; p < e; p += kWave)
      m = maximumf(m, ldv(scores + p));
    m = wave_max(m);
    for (int32_t p = s + l; p < e; p += kWave) {
      const float v = as_stored<T>(expf(ldv(scores + p) - m));
      stv(scores + p, v);
      sum += v;
    }
    sum = as_stored<T>(group_sum<kWave>(sum));
    for (int32_t p = s + l; p < e; p += kWave)
      stv(scores + p, ldv(scores + p) / sum);
  }
  if (l == 0) {
    stv(rmax + r, m);
    stv(rsum + r, sum);
  }
}

// Row r of the attention output computed by one wave from the row's
// normalised scores (the fused kernel's per-row path): lanes over the output
// columns, sequential over the row's positions.
template <typename T>
__device__ __forceinline__ void attention_row_output(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const T *scores, const T *__restrict__ value, T *__restrict__ out,
    int64_t r, int64_t dv) {
  const int32_t s = ro[r], e = ro[r + 1];
  for (int64_t c = lane_id(); c < dv; c += kWave) {
    float acc = 0.0f;
    for (int32_t p = s; p < e; ++p)
      acc = __builtin_fmaf(ldv(scores + p),
                           ldv(value + (int64_t)col[p] * dv + c), acc);
    stv(out + r * dv + c, acc);
  }
}

// One row's softmax in global memory by one wave (the fused kernel's
// per-row path): the long-row branch of row_softmax_wave.
template <typename T>
__device__ __forceinline__ void attention_row_softmax(
    const int32_t *__restrict__ ro, T *scores, T *__restrict__ rmax,
    T *__restrict__ rsum, int64_t r) {
  const int l = lane_id();
  const int32_t s = ro[r], e = ro[r + 1];
  float m = -INFINITY, sum = 0.0f;
  for (int32_t p = s + l; p < e; p += kWave)
    m = maximumf(m, ldv(scores + p));
  m = wave_max(m);
  for (int32_t p = s + l; p < e; p += kWave) {
    const float v = as_stored<T>(expf(ldv(scores + p) - m));
    stv(scores + p, v);
    sum += v;
  }
  sum = as_stored<T>(group_sum<kWave>(sum));
  for (int32_t p = s + l; p < e; p += kWave)
    stv(scores + p, ldv(scores + p) / sum);
  if (l == 0) {
    stv(rmax + r, m);
    stv(rsum + r, sum);
  }
}

// The attention chain fused over 16-row tiles (d = 64 * KB, dv % 16 == 0):
// scores = alpha * Q K^T + beta * mask on the mask's positions, the row
// softmax (rowMaximum, rowSum and the normalised scores written as the
// separate ops write them), and output = P V, in one kernel.  A tile whose
// rows share the last row's column structure (tile_prefix_ok_block) and
// whose last row holds at most kFusedCols entries keeps its scores in
// registers.  Wave w takes the 16-entry chunks k = 0..3 at entries
// t0(k) = 16 (w + W k) of the last row:
//   A. S^T = K_chunk Q^T with 16 x 16 x 4 MFMAs (the gathered K rows as the
//      A operand, Q as the B operand), so that lane (i, g) holds the scores
//      of row i at entries t0 + 4g .. t0 + 4g + 3, which is the A operand
//      the P V product takes;
//   B. the row maxima, then the row sums, are reduced over the four lanes of
//      a row in each wave and over the waves through LDS (two barriers);
//      every final score, row maximum and row sum is written once;
//   C. output = P V from those registers against the gathered V rows, the
//      waves' partial output tiles summed through LDS.
// The scores thus cross HBM once (written) instead of five times, and the
// chain is one launch.  Other tiles run row by row: each wave computes a row's
// scores, softmax and output in global memory.
//
// The loads are batched so that the chain of dependent memory trips is
// short: (1) the tile's row offsets (one load, spread to the lanes by
// permutes) and its Q rows; (2) the rows' column indices for the structure
// check; (3) the K^T gathers and mask windows of chunks 0-1, then of chunks
// 2-3; the V rows of chunks 0-1 fly over the softmax.  Entries past the last row read the last row's
// final column, so no load is guarded; their scores are never used and
// their P is zero.  A V row that is inf or NaN makes the tile's output
// non-finite wherever it is read (0 * inf); such tiles are recomputed row by
// row from the stored scores, adding exactly each row's own entries.
// Scheduling barriers keep each batch of loads together and in order, so
// that waiting for one batch leaves the later ones in flight.
constexpr int kFusedCols = 512;
constexpr int kFusedWaves = 8;
constexpr int kFusedChunks = kFusedCols / (16 * kFusedWaves);

// The host guarantees that the byte offsets into mask / scores (positions),
// K^T (kdim * cols) and V (cols * dv) fit 32 bits and that nnz >= 4
// (amax = nnz - 4, the last 4-entry window of the mask).
//
// IL (dv % 64 == 0, V and the output 16-byte aligned): the four 16-column
// output tiles of a 64-column block interleave -- tile n's column j is
// output column 4j + n of the block -- so that one 128-bit load of a V row
// gives a lane its values for all four tiles, and one 128-bit store writes
// four outputs of a row.
// SO (SDDMM only): the kernel serves the sddmm op on its own -- mask is the
// op's sample values, q its lhs, kt its rhs, scores its output, and `kind`
// its region; the tile stores its scores and ends (value, rmax, rsum, out
// and dv are unused).  The attention chain takes the affine region.
// NS (with SO; no sample values, mask is null): every sample reads as zero
// and no sample window is loaded.
// FLOOR (the chain only; the tile-floor diagnostic sw_attention_tile_floor):
// the same loads, structure check, barrier, stores and output reduction,
// with every product, exponential and division replaced by an XOR of the
// words the lane loaded and without the softmax's two barriers.  Its time is
// the floor of the tile's chain of memory trips.
// (at most 128 VGPRs: the two workgroups of a CU need four waves per SIMD)
template <int KB, int W, bool IL, bool SO, bool NS = false, bool FLOOR = false>
__global__ __launch_bounds__(64 * W, 4) void attention_tile_fused(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ mask, const float *__restrict__ q,
    const float *__restrict__ kt, const float *__restrict__ value,
    float *scores, float *__restrict__ rmax, float *__restrict__ rsum,
    float *__restrict__ out, int32_t rows, int64_t cols, int32_t kdim,
    int64_t dv, float alpha, float beta, uint32_t amax, int kind) {
  const int region = SO ? kind : SW_SDDMM_AFFINE;
  static_assert(W == 8 && kFusedCols == 8 * kWave && kFusedChunks == 4,
                "check layout");
  static_assert(SO || !NS, "the attention chain reads its mask");
  static_assert(!(SO && FLOOR), "the floor runs the chain");
  __shared__ float part[W][4][4][kWave]; // [wave][n tile][v][lane]
  __shared__ float wred[2][W][16];       // [max, sum][wave][row]
  __shared__ int32_t lcol[kFusedCols];   // the last row's columns
  __shared__ int wshared[W]; // each wave's rows share the last row's columns
  __shared__ int v_nonfinite; // an output of the tile is inf or NaN
  if (block_id() * 16 >= rows)
    return; // a folded grid's surplus workgroup (workgroup-uniform)
  const int r0 = (int)block_id() * 16;
  const int nt = std::min(16, rows - r0);
  const int wave = wave_in_group();
  const int l = lane_id(), i = l & 15, g = l >> 4;
  // 1. lanes 0..nt hold ro[r0 .. r0 + nt]; Q row r0 + i, elements
  //    kb 64 + 16 g + st (the B operand of step st)
  const int32_t my_ro = ro[r0 + (l < nt ? l : nt)];
  float qa[16 * KB];
  const int64_t qrow = (int64_t)std::min(r0 + i, rows - 1) * kdim;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v4f x;
      __builtin_memcpy(&x, q + qrow + kb * 64 + 16 * g + 4 * u, sizeof x);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        qa[kb * 16 + 4 * u + e] = i < nt ? x[e] : 0.0f;
    }
  __builtin_amdgcn_sched_barrier(0);
  // row i's first position and length (0 past nt); the permutes run on
  // every lane, as a permute reads zero from a lane that is switched off
  const int ic = i < nt ? i : nt - 1;
  const int32_t rbase = __builtin_amdgcn_ds_bpermute(ic << 2, my_ro);
  const int32_t rnext = __builtin_amdgcn_ds_bpermute((ic + 1) << 2, my_ro);
  const int32_t la = i < nt ? rnext - rbase : 0;
  const int32_t bl = __builtin_amdgcn_readlane(my_ro, nt - 1);
  const int32_t len_last = __builtin_amdgcn_readlane(my_ro, nt) - bl;
  // first entry of this wave's chunk k (entries past len_last: no chunk)
  auto chunk_t0 = [&](int k) __attribute__((always_inline)) {
    return 16 * (wave + W * k);
  };
  // entry (k, v) of lane (i, g): row i, entry chunk_t0(k) + 4g + v
  auto valid = [&](int k, int v) __attribute__((always_inline)) {
    return chunk_t0(k) + 4 * g + v < la;
  };
  // row i's mask values at entries t0(k) + 4g .. + 3: the raw window, read
  // from position min(e, amax) for the window's first position e and
  // shifted by e - min(e, amax) where the values are used
  auto window_at = [&](int k) __attribute__((always_inline)) {
    const uint32_t e = rbase + chunk_t0(k) + 4 * g;
    return e < amax ? e : amax;
  };
  // The structure check and the LDS copy of the last row's column indices
  // share one batch of loads: wave w compares rows w and w + W (at most two,
  // nt <= 16 = 2W) against the last row, a row of at most kFusedCols entries
  // being 8 loads per lane, and stores entries [64w, 64w + 64) of the last
  // row to LDS, where both products read their K / V row indices.
  bool ok = len_last <= kFusedCols; // workgroup-uniform
  if (ok) {
    if (threadIdx.x == 0)
      v_nonfinite = 0;
    int32_t x[2][8], yl[8];
    // unconditional loads from clamped, valid positions (nnz > 0): a row's
    // first position as the wave-uniform base (scalar registers) and the
    // clamped entry index as a 32-bit lane offset (4 nnz fits 32 bits)
    auto row_entry = [&](int32_t b, int32_t len, int32_t t)
        __attribute__((always_inline)) {
      const int32_t *rb = col + (len > 0 ? b : 0);
      return *at_bytes(rb, 4u * (uint32_t)std::min(t, std::max(len - 1, 0)));
    };
#pragma unroll
    for (int u = 0; u < 8; ++u)
      yl[u] = row_entry(bl, len_last, l + u * kWave);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int rr = wave + h * W;
      const int rc = rr < nt - 1 ? rr : 0; // rows past nt-2 are not checked
      const int32_t b = __builtin_amdgcn_readlane(my_ro, rc);
      const int32_t len = __builtin_amdgcn_readlane(my_ro, rc + 1) - b;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        x[h][u] = row_entry(b, len, l + u * kWave);
    }
    // without branches: a compare inside a branch would pull its loads
    // into the branch
    bool mine = true;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int rr = wave + h * W;
      const int rc = rr < nt - 1 ? rr : 0;
      const int32_t b = __builtin_amdgcn_readlane(my_ro, rc);
      const int32_t len = __builtin_amdgcn_readlane(my_ro, rc + 1) - b;
      bool same = len <= len_last;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        same &= (l + u * kWave >= len) | (x[h][u] == yl[u]);
      mine &= (rr >= nt - 1) | same;
    }
    // wave w stores the last row's entries 64w .. 64w + 63; those past the
    // row hold its final column (the clamped loads above), so that the
    // gathers read lcol without clamping an index
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (u == wave)
        lcol[l + u * kWave] = yl[u];
    const bool shared_cols = __builtin_amdgcn_ballot_w64(!mine) == 0;
    if (l == 0)
      wshared[wave] = shared_cols;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < W; ++w)
      ok &= wshared[w] != 0;
  }
  if (!ok) { // workgroup-uniform
    for (int r = r0 + wave; r < r0 + nt; r += W) {
      sddmm_row_wave(ro, col, mask, q, kt, scores, r, cols, kdim, region,
                     alpha, beta);
      if constexpr (!SO) {
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        attention_row_softmax(ro, scores, rmax, rsum, r);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        attention_row_output(ro, col, scores, value, out, r, dv);
      }
    }
    return;
  }
  // 3. the gathers; entries past the last row read its final column
  // K_chunk rows (A operand of step kb 16 + st): K^T[kb 64 + 16 g + st][c]
  // for the column c of entry t0 + i -- the lane's byte offset (16 g rows
  // and c columns on) plus the wave-uniform offset of row kb 64 + st, as
  // buffer loads, whose wave-uniform offset costs no vector instruction
  // (configuration 5: 21.2 -> 20.3 us; d = 128: 31.2 -> 28.5 us)
  const __amdgpu_buffer_rsrc_t kt_rsrc =
      buffer_rsrc(kt, 4u * (uint32_t)kdim * (uint32_t)cols);
  auto gather_k = [&](int k, float (&a)[16 * KB])
      __attribute__((always_inline)) {
    const uint32_t cj = lcol[chunk_t0(k) + i];
    const uint32_t ko = 4u * (16u * g * (uint32_t)cols + cj);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int st = 0; st < 16; ++st)
        a[kb * 16 + st] = buffer_load_f32(
            kt_rsrc, ko, 4u * (uint32_t)(kb * 64 + st) * (uint32_t)cols);
  };
  // V rows (B operand of P V, [n tile][st]): for t = t0(k) + 4g + st, lane
  // (j, g) takes V[c_t][nb + 4j + n] (IL) or V[c_t][nb + 16n + j]; tiles
  // n >= ntiles read tile 0 again -- their outputs are never stored, so
  // their values need no select (a select on the wave-uniform n < ntiles
  // would become a branch around each load)
  auto load_v = [&](int k, int64_t nb, float (&bv)[4][4])
      __attribute__((always_inline)) {
    const int ntiles = (int)std::min<int64_t>(4, (dv - nb) / 16);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int32_t t = chunk_t0(k) + 4 * g + st;
      const uint32_t c = lcol[t];
      if constexpr (IL) {
        const uint32_t vo = 4u * (c * (uint32_t)dv + 4u * (uint32_t)i);
        const v4f x = *reinterpret_cast<const v4f *>(at_bytes(value + nb, vo));
#pragma unroll
        for (int n = 0; n < 4; ++n)
          bv[n][st] = x[n];
      } else {
        const uint32_t vo = 4u * (c * (uint32_t)dv + (uint32_t)i);
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          const int nn = n < ntiles ? n : 0; // wave-uniform
          bv[n][st] = *at_bytes(value + nb + 16 * nn, vo);
        }
      }
    }
  };
  auto load_window = [&](int k, v4f &w) __attribute__((always_inline)) {
    if constexpr (NS)
      w = v4f{0.f, 0.f, 0.f, 0.f};
    else
      __builtin_memcpy(&w, mask + window_at(k), sizeof(v4f));
  };
  // A. S^T per chunk: sv[k][v] = score (i, t0(k) + 4g + v)
  float sv[kFusedChunks][4];
  auto sddmm_chunk = [&](int k, const float (&a)[16 * KB], const v4f &w)
      __attribute__((always_inline)) {
    if constexpr (FLOOR) {
      uint32_t x = 0;
#pragma unroll
      for (int st = 0; st < 16 * KB; ++st)
        x ^= __float_as_uint(a[st]);
#pragma unroll
      for (int v = 0; v < 4; ++v)
        sv[k][v] = __uint_as_float(x ^ __float_as_uint(w[v]));
      return;
    }
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    if (chunk_t0(k) < len_last) { // wave-uniform
      // two independent chains of products (even and odd K steps): one
      // chain of 16 dependent MFMAs held the wave (18.0 -> 17.6 us; four
      // chains: no faster at d = 64, slower at d = 128)
      v4f acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 16 * KB; st += 2) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[st], qa[st], acc, 0, 0,
                                                   0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[st + 1], qa[st + 1],
                                                    acc1, 0, 0, 0);
      }
      acc += acc1;
    }
    const uint32_t d = rbase + chunk_t0(k) + 4 * g - window_at(k);
    const v4f x = {d == 0 ? w.x : d == 1 ? w.y : d == 2 ? w.z : w.w,
                   d == 0 ? w.y : d == 1 ? w.z : w.w, d == 0 ? w.z : w.w, w.w};
#pragma unroll
    for (int v = 0; v < 4; ++v)
      sv[k][v] = combine_sddmm(region, valid(k, v) ? x[v] : 0.0f, acc[v],
                               alpha, beta);
  };
  float bv[kFusedChunks][4][4];
  // two chunks' K^T gathers and mask windows per batch; a chunk past the
  // last row's entries loads nothing (each branch holds its loads and the
  // products that take them, so no branch waits for a load it does not use)
#pragma unroll
  for (int k0 = 0; k0 < kFusedChunks; k0 += 2) {
    if (chunk_t0(k0 + 1) < len_last) { // wave-uniform
      float a[2][16 * KB];
      v4f w[2];
      gather_k(k0, a[0]);
      gather_k(k0 + 1, a[1]);
      load_window(k0, w[0]);
      load_window(k0 + 1, w[1]);
      __builtin_amdgcn_sched_barrier(0);
      sddmm_chunk(k0, a[0], w[0]);
      sddmm_chunk(k0 + 1, a[1], w[1]);
    } else {
      if (chunk_t0(k0) < len_last) {
        float a[16 * KB];
        v4f w;
        gather_k(k0, a);
        load_window(k0, w);
        __builtin_amdgcn_sched_barrier(0);
        sddmm_chunk(k0, a, w);
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          sv[k0][v] = 0.0f;
      }
#pragma unroll
      for (int v = 0; v < 4; ++v)
        sv[k0 + 1][v] = 0.0f;
    }
  }
  if constexpr (SO) {
    // the scores of entries t0(k) + 4g .. + 3 of row i: one (unaligned)
    // vector store when all four are the row's, else the row's ones one by
    // one
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k) {
      if (chunk_t0(k) >= len_last) // wave-uniform
        continue;
      float *dst = scores + rbase + chunk_t0(k) + 4 * g;
      if (valid(k, 3)) {
        const v4f x = v4f{sv[k][0], sv[k][1], sv[k][2], sv[k][3]};
        __builtin_memcpy(dst, &x, sizeof x);
      } else {
#pragma unroll
        for (int v = 0; v < 3; ++v)
          if (valid(k, v))
            dst[v] = sv[k][v];
      }
    }
    return;
  }
  // in flight over the softmax (the V rows of chunks 2-3 are loaded after
  // it: holding all four chunks' rows over it would take more registers
  // than four waves per SIMD leave)
  load_v(0, 0, bv[0]);
  load_v(1, 0, bv[1]);
  if constexpr (FLOOR) {
    // the scores' stores and the row outputs' stores, no softmax
    uint32_t x = 0;
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k) {
      if (chunk_t0(k) >= len_last) // wave-uniform
        continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        sv[k][v] = valid(k, v) ? sv[k][v] : 0.0f;
        x ^= __float_as_uint(sv[k][v]);
      }
      float *dst = scores + rbase + chunk_t0(k) + 4 * g;
      if (valid(k, 3)) {
        const v4f y = v4f{sv[k][0], sv[k][1], sv[k][2], sv[k][3]};
        __builtin_memcpy(dst, &y, sizeof y);
      } else {
#pragma unroll
        for (int v = 0; v < 3; ++v)
          if (valid(k, v))
            dst[v] = sv[k][v];
      }
    }
    if (wave == 0 && g == 0 && i < nt) {
      rmax[r0 + i] = __uint_as_float(x);
      rsum[r0 + i] = __uint_as_float(x);
    }
  } else {
  // B. row softmax: lanes (i, 0..3) of every wave hold row i's entries
  {
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (valid(k, v))
          m = maximumf(m, sv[k][v]);
    m = maximumf(m, swizzle_xor16(m));
    m = maximumf(m, shfl_xor32(m));
    if (g == 0)
      wred[0][wave][i] = m;
    __syncthreads();
    m = wred[0][0][i];
#pragma unroll
    for (int w = 1; w < W; ++w)
      m = maximumf(m, wred[0][w][i]);
    // per chunk of entries (a chunk past the last row is skipped whole),
    // each entry's value computed unconditionally and selected afterwards:
    // no branch per entry
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k) {
      if (chunk_t0(k) < len_last) { // wave-uniform
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float e = exp_by_exp2(sv[k][v] - m);
          sv[k][v] = valid(k, v) ? e : 0.0f;
          sum += sv[k][v];
        }
      }
    }
    sum += swizzle_xor16(sum);
    sum += shfl_xor32(sum);
    if (g == 0)
      wred[1][wave][i] = sum;
    __syncthreads();
    sum = wred[1][0][i];
#pragma unroll
    for (int w = 1; w < W; ++w)
      sum += wred[1][w][i];
    // one correctly rounded reciprocal per row, one multiply per entry
    // (within 1.5 ulp of the quotient)
    const float rsum_i = 1.0f / sum;
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k) {
      if (chunk_t0(k) >= len_last) { // wave-uniform
#pragma unroll
        for (int v = 0; v < 4; ++v)
          sv[k][v] = 0.0f;
        continue;
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) { // zero past the row: P V adds nothing
        const float p = sv[k][v] * rsum_i;
        sv[k][v] = valid(k, v) ? p : 0.0f;
      }
      // entries t0(k) + 4g .. + 3 of row i: one (unaligned) vector store
      // when all four are the row's, else the row's ones one by one
      float *dst = scores + rbase + chunk_t0(k) + 4 * g;
      if (valid(k, 3)) {
        const v4f x = v4f{sv[k][0], sv[k][1], sv[k][2], sv[k][3]};
        __builtin_memcpy(dst, &x, sizeof x);
      } else {
#pragma unroll
        for (int v = 0; v < 3; ++v)
          if (valid(k, v))
            dst[v] = sv[k][v];
      }
    }
    if (wave == 0 && g == 0 && i < nt) {
      rmax[r0 + i] = m;
      rsum[r0 + i] = sum;
    }
  }
  } // FLOOR
  // C. output = P V with P from sv (lane (i, g) holds P[i][t0(k)+4g+st],
  // the A operand of step st); the waves' partial tiles are summed in LDS
  auto mfma_chunk = [&](int k, const float (&b)[4][4], v4f (&acc)[4])
      __attribute__((always_inline)) {
    if constexpr (FLOOR) {
      if (chunk_t0(k) < len_last) // wave-uniform
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int st = 0; st < 4; ++st)
            acc[n][st] = __uint_as_float(__float_as_uint(acc[n][st]) ^
                                         __float_as_uint(sv[k][st]) ^
                                         __float_as_uint(b[n][st]));
      return;
    }
    if (chunk_t0(k) < len_last) // wave-uniform
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int st = 0; st < 4; ++st)
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(sv[k][st], b[n][st],
                                                        acc[n], 0, 0, 0);
  };
  // the waves' partial tiles combine by sum (by XOR in the floor)
  auto combine = [&](float a, float b) __attribute__((always_inline)) {
    if constexpr (FLOOR)
      return __uint_as_float(__float_as_uint(a) ^ __float_as_uint(b));
    else
      return a + b;
  };
  bool nonfinite = false;
  for (int64_t nb = 0; nb < dv; nb += 64) {
    const int ntiles = (int)std::min<int64_t>(4, (dv - nb) / 16);
    v4f acc[4];
#pragma unroll
    for (int n = 0; n < 4; ++n)
      acc[n] = v4f{0.f, 0.f, 0.f, 0.f};
    if (nb > 0) {
#pragma unroll
      for (int k = 0; k < kFusedChunks; ++k)
        load_v(k, nb, bv[k]);
    } else {
      load_v(2, 0, bv[2]);
      load_v(3, 0, bv[3]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k)
      mfma_chunk(k, bv[k], acc);
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        part[wave][n][v][l] = acc[n][v];
    __syncthreads();
    if constexpr (IL) {
      if (wave < 4) {
        // wave w finishes rows 4g + w, columns nb + 4i .. nb + 4i + 3
        v4f o;
        bool nf = false;
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          float sum = 0.0f;
#pragma unroll
          for (int w = 0; w < W; ++w)
            sum = combine(sum, part[w][n][wave][l]);
          o[n] = sum;
          nf |= !FLOOR && !__builtin_isfinite(sum);
        }
        const int rr = 4 * g + wave;
        if (rr < nt) {
          *reinterpret_cast<v4f *>(out + (int64_t)(r0 + rr) * dv + nb +
                                   4 * i) = o;
          nonfinite |= nf;
        }
        if (__builtin_amdgcn_ballot_w64(nonfinite) != 0 && l == 0)
          v_nonfinite = 1;
      }
    } else if (wave < ntiles) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w)
          sum = combine(sum, part[w][wave][v][l]);
        const int rr = 4 * g + v;
        if (rr < nt) {
          out[(int64_t)(r0 + rr) * dv + nb + 16 * wave + i] = sum;
          nonfinite |= !FLOOR && !__builtin_isfinite(sum);
        }
      }
      if (__builtin_amdgcn_ballot_w64(nonfinite) != 0 && l == 0)
        v_nonfinite = 1;
    }
    __syncthreads();
  }
  // workgroup-uniform; the barrier above also made every wave's stored
  // scores visible to the others
  if (v_nonfinite != 0)
    for (int r = r0 + wave; r < r0 + nt; r += W)
      attention_row_output(ro, col, scores, value, out, r, dv);
}

// ---- bf16 matrix-core kernels ----------------------------------------------
// The bf16 forms of the SDDMM tile and the fused attention tile: the same
// 16-row tiles, row structure check, fallbacks and outputs as the fp32
// kernels above, with bf16 operands on the matrix cores (fp32 accumulation):
//   Q K^T: v_mfma_f32_16x16x32_bf16, lane group g supplying K elements
//     32 s + 8 g .. 32 s + 8 g + 7 at step s -- one 128-bit load of a Q row
//     and eight 16-bit K^T gathers per lane and step;
//   P V:   v_mfma_f32_16x16x16_bf16 per 16-entry chunk, lane group g
//     supplying entries 4 g .. 4 g + 3 of the chunk, with four output tiles
//     whose columns interleave (tile n's column j is output column
//     4 j + n of the 64-column block), so that one 64-bit load of a V row
//     gives a lane its values for all four tiles.
// Every result is rounded to bf16 where the separate op would store it.

// the eight K^T values K^T[32 s + 8 g + e][c] (e = 0..7) as four bf16 pairs;
// base is K^T row 32 s, lane_off the byte offset of column c plus 8 g rows
__device__ __forceinline__ v4u gather_kt8(const uint16_t *base,
                                          uint32_t row_bytes,
                                          uint32_t lane_off) {
  uint32_t x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    x[e] = *at_bytes(at_bytes(base, e * row_bytes), lane_off);
  return v4u{x[0] | (x[1] << 16), x[2] | (x[3] << 16), x[4] | (x[5] << 16),
             x[6] | (x[7] << 16)};
}

// SDDMM over 16-row tiles, bf16 (kdim = 64 * KB; the host guarantees that
// 2 * kdim * cols and 2 * nnz fit 32 bits and that lhs is 16-byte aligned).
template <int KB, int W>
__global__ __launch_bounds__(64 * W) void sddmm_tile_mfma_bf16(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const uint16_t *__restrict__ val, const uint16_t *__restrict__ lhs,
    const uint16_t *__restrict__ rhs, uint16_t *__restrict__ out,
    int32_t rows, int64_t cols, int32_t kdim, int kind, float alpha,
    float beta) {
  constexpr int S = 2 * KB; // 32-deep K steps
  if (block_id() * 16 >= rows)
    return; // a folded grid's surplus workgroup (workgroup-uniform)
  const int r0 = (int)block_id() * 16;
  const int nt = std::min(16, rows - r0);
  const int wave = wave_in_group();
  const int l = lane_id(), i = l & 15, g = l >> 4;
  int32_t rb[4], rl[4];
  {
    int32_t b[5];
#pragma unroll
    for (int v = 0; v < 5; ++v)
      b[v] = ro[std::min(r0 + 4 * g + v, rows)];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      rb[v] = b[v];
      rl[v] = 4 * g + v < nt ? b[v + 1] - b[v] : 0;
    }
  }
  // A operand: lhs row r0 + i, elements 32 s + 8 g .. + 7
  v4u qa[S];
  const int64_t qrow = (int64_t)std::min(r0 + i, rows - 1) * kdim;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const v4u x = *reinterpret_cast<const v4u *>(lhs + qrow + 32 * s + 8 * g);
    qa[s] = i < nt ? x : v4u{0u, 0u, 0u, 0u};
  }
  __shared__ int verdict;
  if (!tile_prefix_ok_block(ro, col, r0, nt, &verdict)) {
    for (int r = r0 + wave; r < r0 + nt; r += W)
      sddmm_row_wave(ro, col, val, lhs, rhs, out, r, cols, kdim, kind, alpha,
                     beta);
    return;
  }
  const int last = r0 + nt - 1;
  const int32_t bl = ro[last];
  const int32_t len_last = ro[last + 1] - bl;
  const uint32_t row_bytes = 2u * (uint32_t)cols;
  for (int32_t t0 = wave * 16; t0 < len_last; t0 += 32 * W) {
    const int32_t t1 = t0 + 16 * W;
    const bool two = t1 < len_last; // wave-uniform
    const int32_t ta = t0 + i, tb = t1 + i;
    const uint32_t cj0 = ta < len_last ? (uint32_t)col[bl + ta] : 0u;
    const uint32_t cj1 = two && tb < len_last ? (uint32_t)col[bl + tb] : 0u;
    float s0[4], s1[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const bool in0 = val != nullptr && ta < rl[v];
      const bool in1 = val != nullptr && two && tb < rl[v];
      const float x0 = val != nullptr ? ldv(val + (in0 ? rb[v] + ta : bl)) : 0.f;
      const float x1 = val != nullptr ? ldv(val + (in1 ? rb[v] + tb : bl)) : 0.f;
      s0[v] = in0 ? x0 : 0.0f;
      s1[v] = in1 ? x1 : 0.0f;
    }
    const uint32_t lo0 = 2u * cj0 + 8u * g * row_bytes;
    const uint32_t lo1 = 2u * cj1 + 8u * g * row_bytes;
    v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    v4u b0[S], b1[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const uint16_t *base = rhs + (int64_t)(32 * s) * cols;
      b0[s] = gather_kt8(base, row_bytes, lo0);
      b1[s] = gather_kt8(base, row_bytes, lo1); // column 0 when !two
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      acc0 = mfma_16x16x32_bf16(qa[s], b0[s], acc0);
      if (two)
        acc1 = mfma_16x16x32_bf16(qa[s], b1[s], acc1);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if (ta < rl[v])
        stv(out + rb[v] + ta,
            combine_sddmm(kind, s0[v], acc0[v], alpha, beta));
      if (two && tb < rl[v])
        stv(out + rb[v] + tb,
            combine_sddmm(kind, s1[v], acc1[v], alpha, beta));
    }
  }
}

// The attention chain fused over 16-row tiles, bf16 (d = 64 * KB,
// dv % 64 == 0): the fp32 attention_tile_fused's tiles, waves, chunks,
// structure check and fallbacks, with the products on bf16 matrix cores.
// Its loads are batched so that the chain of dependent memory trips is short:
//   1. the tile's row offsets (one load, spread to the lanes by permutes) and
//      its Q rows;
//   2. the rows' column indices for the structure check, with every chunk's
//      mask window in flight over the check;
//   3. the K^T gathers of chunks 0-1, then of chunks 2-3 (none for chunks
//      past the last row); the V rows of chunks 0-1 fly over the second
//      batch (d = 64) or the softmax, those of chunks 2-3 over the softmax
//      (d = 64) or are loaded after it.
// The products do not wait for the structure check: its verdict is read at
// the softmax's first barrier, before anything is stored.  Entries past the
// last row read the last row's final column, so no load is guarded; their
// scores are never used and their P is zero.  A V row that is inf or NaN
// makes the tile's output non-finite wherever it is read (0 * inf), and such
// tiles are recomputed row by row, as in the fp32 kernel.
// The host guarantees that the byte offsets into mask / scores (2 * nnz),
// K^T (2 * d * cols) and V (2 * cols * dv) fit 32 bits, that nnz >= 4
// (amax = nnz - 4) and that Q is 16-byte and V 8-byte aligned.
// (at most 128 VGPRs: the two workgroups of a CU need four waves per SIMD)
// FLOOR: the tile-floor diagnostic, as for the fp32 kernel above.
template <int KB, int W, bool SO, bool NS = false, bool FLOOR = false>
__global__ __launch_bounds__(64 * W, 4) void attention_tile_fused_bf16(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const uint16_t *__restrict__ mask, const uint16_t *__restrict__ q,
    const uint16_t *__restrict__ kt, const uint16_t *__restrict__ value,
    uint16_t *scores, uint16_t *__restrict__ rmax, uint16_t *__restrict__ rsum,
    uint16_t *__restrict__ out, int32_t rows, int64_t cols, int32_t kdim,
    int64_t dv, float alpha, float beta, uint32_t amax, int kind) {
  static_assert(W == 8 && kFusedCols == 8 * kWave && kFusedChunks == 4,
                "check layout");
  constexpr int S = 2 * KB;
  // SO: the SDDMM alone (combine kind `kind`), its scores stored from
  // registers; no softmax and no P V.  NS (with SO): no sample values (mask
  // is null), every sample reads as zero
  const int region = SO ? kind : SW_SDDMM_AFFINE;
  static_assert(SO || !NS, "the attention chain reads its mask");
  static_assert(!(SO && FLOOR), "the floor runs the chain");
  __shared__ float part[W][4][4][kWave]; // [wave][n tile][v][lane]
  __shared__ float wred[2][W][16];       // [max, sum][wave][row]
  __shared__ int wshared[W]; // each wave's rows share the last row's columns
  __shared__ int v_nonfinite;
  if (block_id() * 16 >= rows)
    return; // a folded grid's surplus workgroup (workgroup-uniform)
  const int r0 = (int)block_id() * 16;
  const int nt = std::min(16, rows - r0);
  const int wave = wave_in_group();
  const int l = lane_id(), i = l & 15, g = l >> 4;
  // 1. lanes 0..nt hold ro[r0 .. r0 + nt]; Q row r0 + i, elements
  //    32 s + 8 g .. + 7 (the B operand of S^T = K_chunk Q^T)
  const int32_t my_ro = ro[r0 + (l < nt ? l : nt)];
  v4u qb[S];
  const int64_t qrow = (int64_t)std::min(r0 + i, rows - 1) * kdim;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const v4u x = *reinterpret_cast<const v4u *>(q + qrow + 32 * s + 8 * g);
    qb[s] = i < nt ? x : v4u{0u, 0u, 0u, 0u};
  }
  // (scheduling barriers keep each batch of loads together and in order,
  // so that waiting for one batch leaves the later ones in flight)
  __builtin_amdgcn_sched_barrier(0);
  // row i's first position and length (0 past nt); the permutes run on
  // every lane, as a permute reads zero from a lane that is switched off
  const int ic = i < nt ? i : nt - 1;
  const int32_t rbase = __builtin_amdgcn_ds_bpermute(ic << 2, my_ro);
  const int32_t rnext = __builtin_amdgcn_ds_bpermute((ic + 1) << 2, my_ro);
  const int32_t la = i < nt ? rnext - rbase : 0;
  const int32_t bl = __builtin_amdgcn_readlane(my_ro, nt - 1);
  const int32_t len_last = __builtin_amdgcn_readlane(my_ro, nt) - bl;
  auto chunk_t0 = [&](int k) __attribute__((always_inline)) {
    return 16 * (wave + W * k);
  };
  auto valid = [&](int k, int v) __attribute__((always_inline)) {
    return chunk_t0(k) + 4 * g + v < la;
  };
  // 2. row i's mask values at entries t0(k) + 4g .. + 3: the raw 8-byte
  //    window, read from position min(e, amax) for the window's first
  //    position e and shifted by e - min(e, amax) where the values are used
  auto window_at = [&](int k) __attribute__((always_inline)) {
    const uint32_t e = rbase + chunk_t0(k) + 4 * g;
    return e < amax ? e : amax;
  };
  uint64_t mw[kFusedChunks];
  // The structure check and the products run together: each wave checks its
  // rows against the last row and computes its chunks with the last row's
  // columns right away; the verdict is read at the softmax's first barrier,
  // before anything is stored, and a tile that fails it is redone row by
  // row.  The last row's column indices stay in registers: lane j of yl[u]
  // holds entry 64u + j (clamped to the last entry), and a lane takes the
  // column of an entry from there with a permute.
  bool ok = len_last <= kFusedCols; // workgroup-uniform
  if (threadIdx.x == 0)
    v_nonfinite = 0;
  // yk[k]: the yl register holding chunk k's entries 16 (w + 8k) .. + 15,
  // in lanes 16 (w & 3) .. + 15
  int32_t yk[kFusedChunks];
  auto col_of = [&](int k, int off) __attribute__((always_inline)) {
    return (uint32_t)__builtin_amdgcn_ds_bpermute(
        (16 * (wave & 3) + off) << 2, yk[k]);
  };
  // K_chunk rows (A operand): K^T[32 s + 8 g .. + 7][column of entry t0 + i]
  const uint32_t row_bytes = 2u * (uint32_t)cols;
  auto gather_k = [&](int k, v4u (&a)[S]) __attribute__((always_inline)) {
    const uint32_t ko = 2u * col_of(k, i) + 8u * g * row_bytes;
#pragma unroll
    for (int s = 0; s < S; ++s)
      a[s] = gather_kt8(kt + (int64_t)(32 * s) * cols, row_bytes, ko);
  };
  // V rows (B operand of P V): lane (j, g) takes V[c_t][nb + 4j .. + 3] for
  // t = t0(k) + 4g + st, tile n taking element n
  auto load_v = [&](int k, int64_t nb, v2u (&bv)[4])
      __attribute__((always_inline)) {
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const uint32_t c = col_of(k, 4 * g + st);
      const uint32_t vo = 2u * (c * (uint32_t)dv + 4u * (uint32_t)i);
      bv[st] = *reinterpret_cast<const v2u *>(at_bytes(value + nb, vo));
    }
  };
  // A. S^T per chunk: sv[k][v] = score (i, t0(k) + 4g + v), rounded to bf16
  float sv[kFusedChunks][4];
  auto sddmm_chunk = [&](int k, const v4u (&a)[S])
      __attribute__((always_inline)) {
    if constexpr (FLOOR) {
      uint32_t x = (uint32_t)mw[k] ^ (uint32_t)(mw[k] >> 32);
#pragma unroll
      for (int s2 = 0; s2 < S; ++s2)
        x ^= a[s2].x ^ a[s2].y ^ a[s2].z ^ a[s2].w;
#pragma unroll
      for (int v = 0; v < 4; ++v)
        sv[k][v] = __uint_as_float(x ^ (uint32_t)v);
      return;
    }
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    if (chunk_t0(k) < len_last) { // wave-uniform
#pragma unroll
      for (int s = 0; s < S; ++s)
        acc = mfma_16x16x32_bf16(a[s], qb[s], acc);
    }
    const uint32_t d = rbase + chunk_t0(k) + 4 * g - window_at(k);
    const uint64_t w = d < 4 ? mw[k] >> (16 * d) : 0ull;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float x = valid(k, v) ? bf16_to_f32((uint16_t)(w >> (16 * v)))
                                  : 0.0f;
      sv[k][v] = as_stored<uint16_t>(
          combine_sddmm(region, x, acc[v], alpha, beta));
    }
  };
  // two chunks' K^T gathers per batch; a chunk past the last row's entries
  // loads nothing (each branch holds its loads and the products that take
  // them, so no branch waits for a load it does not use)
  auto batch = [&](int k0) __attribute__((always_inline)) {
    if (chunk_t0(k0 + 1) < len_last) { // wave-uniform
      v4u a[2][S];
      gather_k(k0, a[0]);
      gather_k(k0 + 1, a[1]);
      __builtin_amdgcn_sched_barrier(0);
      sddmm_chunk(k0, a[0]);
      sddmm_chunk(k0 + 1, a[1]);
    } else {
      if (chunk_t0(k0) < len_last) {
        v4u a[S];
        gather_k(k0, a);
        __builtin_amdgcn_sched_barrier(0);
        sddmm_chunk(k0, a);
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          sv[k0][v] = 0.0f;
      }
#pragma unroll
      for (int v = 0; v < 4; ++v)
        sv[k0 + 1][v] = 0.0f;
    }
  };
  v2u bv[kFusedChunks][4];
  v2u pk[kFusedChunks]; // P as bf16 pairs: entries 4g, 4g + 1 | 4g + 2, 4g + 3
  if (ok) {
    int32_t x[2][8], yl[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int32_t t = l + u * kWave;
      yl[u] = col[len_last > 0 ? bl + std::min(t, len_last - 1) : 0];
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int rr = wave + h * W;
      const int rc = rr < nt - 1 ? rr : 0;
      const int32_t b = __builtin_amdgcn_readlane(my_ro, rc);
      const int32_t len = __builtin_amdgcn_readlane(my_ro, rc + 1) - b;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int32_t t = l + u * kWave;
        x[h][u] = col[len > 0 ? b + std::min(t, len - 1) : 0];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k) {
      if constexpr (NS)
        mw[k] = 0;
      else
        __builtin_memcpy(&mw[k], mask + window_at(k), sizeof(uint64_t));
    }
    __builtin_amdgcn_sched_barrier(0);
    // without branches: a compare inside a branch would pull its loads
    // into the branch, behind the mask windows
    bool mine = true;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int rr = wave + h * W;
      const int rc = rr < nt - 1 ? rr : 0;
      const int32_t b = __builtin_amdgcn_readlane(my_ro, rc);
      const int32_t len = __builtin_amdgcn_readlane(my_ro, rc + 1) - b;
      bool same = len <= len_last;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        same &= (l + u * kWave >= len) | (x[h][u] == yl[u]);
      mine &= (rr >= nt - 1) | same;
    }
    const bool shared_cols = __builtin_amdgcn_ballot_w64(!mine) == 0;
    if (l == 0)
      wshared[wave] = shared_cols;
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k)
      yk[k] = wave >= 4 ? yl[2 * k + 1] : yl[2 * k];
    batch(0);
    if constexpr (KB == 1 && !SO) { // in flight over the second batch and softmax
      load_v(0, 0, bv[0]);
      load_v(1, 0, bv[1]);
    }
    batch(2);
    if constexpr (SO) {
    } else if constexpr (KB == 1) { // in flight over the softmax
      load_v(2, 0, bv[2]);
      load_v(3, 0, bv[3]);
    } else {
      load_v(0, 0, bv[0]);
      load_v(1, 0, bv[1]);
    }
    if constexpr (!SO && !FLOOR) {
      // B. row softmax on the stored (bf16) scores, each op's result
      // rounded: this wave's row maxima
      float m = -INFINITY;
#pragma unroll
      for (int k = 0; k < kFusedChunks; ++k)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (valid(k, v))
            m = maximumf(m, sv[k][v]);
      m = maximumf(m, swizzle_xor16(m));
      m = maximumf(m, shfl_xor32(m));
      if (g == 0)
        wred[0][wave][i] = m;
    }
  }
  __syncthreads();
  if (ok) {
#pragma unroll
    for (int w = 0; w < W; ++w)
      ok &= wshared[w] != 0;
  }
  if (!ok) { // workgroup-uniform; nothing has been stored yet
    for (int r = r0 + wave; r < r0 + nt; r += W) {
      sddmm_row_wave(ro, col, mask, q, kt, scores, r, cols, kdim, region,
                     alpha, beta);
      if constexpr (!SO) {
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        attention_row_softmax(ro, scores, rmax, rsum, r);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        attention_row_output(ro, col, scores, value, out, r, dv);
      }
    }
    return;
  }
  if constexpr (SO) {
    // the scores, already rounded to bf16, as pairs
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k) {
      if (chunk_t0(k) < len_last) { // wave-uniform
        const v2u pr = v2u{pack_bf16x2(sv[k][0], sv[k][1]),
                           pack_bf16x2(sv[k][2], sv[k][3])};
        uint16_t *dst = scores + rbase + chunk_t0(k) + 4 * g;
        if (valid(k, 3)) {
          __builtin_memcpy(dst, &pr, sizeof pr);
        } else {
#pragma unroll
          for (int v = 0; v < 3; ++v)
            if (valid(k, v))
              dst[v] = (uint16_t)(pr[v >> 1] >> (16 * (v & 1)));
        }
      }
    }
    return;
  }
  if constexpr (FLOOR) {
    // the scores' stores and the row outputs' stores, no softmax
    uint32_t x = 0;
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k) {
      pk[k] = v2u{valid(k, 0) ? __float_as_uint(sv[k][0]) : 0u,
                  valid(k, 2) ? __float_as_uint(sv[k][2]) : 0u};
      x ^= pk[k].x ^ pk[k].y;
      uint16_t *dst = scores + rbase + chunk_t0(k) + 4 * g;
      if (valid(k, 3)) {
        __builtin_memcpy(dst, &pk[k], sizeof pk[k]);
      } else {
#pragma unroll
        for (int v = 0; v < 3; ++v)
          if (valid(k, v))
            dst[v] = (uint16_t)(pk[k][v >> 1] >> (16 * (v & 1)));
      }
    }
    if (wave == 0 && g == 0 && i < nt) {
      rmax[r0 + i] = (uint16_t)x;
      rsum[r0 + i] = (uint16_t)(x >> 16);
    }
  } else {
    float m = wred[0][0][i];
#pragma unroll
    for (int w = 1; w < W; ++w)
      m = maximumf(m, wred[0][w][i]);
    // per chunk of entries (a chunk past the last row is skipped whole),
    // each entry's value computed unconditionally and selected afterwards:
    // no branch per entry (adding the zeros leaves the sum's bits as they are)
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k) {
      if (chunk_t0(k) < len_last) { // wave-uniform
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float e = as_stored<uint16_t>(exp_by_exp2(sv[k][v] - m));
          sv[k][v] = valid(k, v) ? e : 0.0f;
          sum += sv[k][v];
        }
      }
    }
    sum += swizzle_xor16(sum);
    sum += shfl_xor32(sum);
    if (g == 0)
      wred[1][wave][i] = sum;
    __syncthreads();
    sum = wred[1][0][i];
#pragma unroll
    for (int w = 1; w < W; ++w)
      sum += wred[1][w][i];
    sum = as_stored<uint16_t>(sum);
    // one correctly rounded reciprocal per row, one multiply per entry
    // (within 1.5 ulp of the quotient before the bf16 rounding)
    const float rsum_i = 1.0f / sum;
    // P rounded to bf16 once, as pairs: the stored scores and the A operand
    // of P V are the same bits
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k) {
      float p[4];
#pragma unroll
      for (int v = 0; v < 4; ++v)
        p[v] = valid(k, v) ? sv[k][v] * rsum_i : 0.0f;
      pk[k] = v2u{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
      uint16_t *dst = scores + rbase + chunk_t0(k) + 4 * g;
      if (valid(k, 3)) {
        __builtin_memcpy(dst, &pk[k], sizeof pk[k]);
      } else {
#pragma unroll
        for (int v = 0; v < 3; ++v)
          if (valid(k, v))
            dst[v] = (uint16_t)(pk[k][v >> 1] >> (16 * (v & 1)));
      }
    }
    if (wave == 0 && g == 0 && i < nt) {
      stv(rmax + r0 + i, m);
      stv(rsum + r0 + i, sum);
    }
  }
  // C. output = P V: P from pk (lane (i, g) holds P[i][t0(k) + 4g + st])
  auto mfma_chunk = [&](int k, const v2u (&b)[4], v4f (&acc)[4])
      __attribute__((always_inline)) {
    if constexpr (FLOOR) {
      if (chunk_t0(k) < len_last) // wave-uniform
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int st = 0; st < 4; ++st)
            acc[n][st] = __uint_as_float(__float_as_uint(acc[n][st]) ^
                                         pk[k][st >> 1] ^ b[n][st & 1]);
      return;
    }
    if (chunk_t0(k) < len_last) { // wave-uniform
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const v2u bn = v2u{bf16_pair(b[0], b[1], n), bf16_pair(b[2], b[3], n)};
        acc[n] = mfma_16x16x16_bf16(pk[k], bn, acc[n]);
      }
    }
  };
  bool nonfinite = false;
  for (int64_t nb = 0; nb < dv; nb += 64) {
    v4f acc[4];
#pragma unroll
    for (int n = 0; n < 4; ++n)
      acc[n] = v4f{0.f, 0.f, 0.f, 0.f};
    if (nb > 0) {
#pragma unroll
      for (int k = 0; k < kFusedChunks; ++k)
        load_v(k, nb, bv[k]);
    } else if constexpr (KB != 1) {
      load_v(2, 0, bv[2]);
      load_v(3, 0, bv[3]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < kFusedChunks; ++k)
      mfma_chunk(k, bv[k], acc);
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
        for (int w = 0; w < W; ++w) {
          if constexpr (FLOOR) // the waves' partial words combine by XOR
            sum = __uint_as_float(__float_as_uint(sum) ^
                                  __float_as_uint(part[w][n][wave][l]));
          else
            sum += part[w][n][wave][l];
        }
        o[n] = sum;
        nf |= !FLOOR && !__builtin_isfinite(sum);
      }
      const int rr = 4 * g + wave;
      if (rr < nt) {
        *reinterpret_cast<v2u *>(out + (int64_t)(r0 + rr) * dv + nb + 4 * i) =
            FLOOR ? v2u{__float_as_uint(o[0]) ^ __float_as_uint(o[1]),
                        __float_as_uint(o[2]) ^ __float_as_uint(o[3])}
                  : v2u{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
        nonfinite |= nf;
      }
      if (__builtin_amdgcn_ballot_w64(nonfinite) != 0 && l == 0)
        v_nonfinite = 1;
    }
    __syncthreads();
  }
  if (v_nonfinite != 0)
    for (int r = r0 + wave; r < r0 + nt; r += W)
      attention_row_output(ro, col, scores, value, out, r, dv);
}

int grid_for(int64_t work, int64_t per_block, const char *what,
             int64_t *grid) {
  *grid = std::max<int64_t>(sw::ceil_div(work, per_block), 1);
  // (every kernel launched with it has at most 1024 work-items a workgroup)
  return sw::check_grid(*grid, 1024, what);
}

} // namespace

namespace sw {

template <typename T>
int launch_sddmm(const int32_t *ro, const int32_t *col, const T *val,
                 const T *lhs, const T *rhs, T *out, int64_t rows,
                 int64_t cols, int64_t nnz, int64_t kdim, int kind,
                 float alpha, float beta, const sw_options &o,
                 hipStream_t st) {
  int64_t grid;
  if (streq(o.sddmm_mapping, "row-tile-mfma") &&
      (kdim == 64 || kdim == 128 || kdim == 256)) {
    const int kb = (int)(kdim / 64);
    if constexpr (sizeof(T) == 4) {
      int rc = grid_for(rows, 16, "SDDMM", &grid);
      if (rc)
        return rc;
      // d of 64 or 128 with 32-bit offsets, and no sample values or an
      // output apart from them: the fused attention kernel's product phase
      // (its 4-entry sample windows may reach a neighbouring tile's entries)
      if ((kdim == 64 || kdim == 128) && nnz >= 4 &&
          narrow_offsets(nnz, 1) && narrow_offsets(cols, kdim) &&
          (val == nullptr || out + nnz <= val || val + nnz <= out)) {
#define SW_SDDMM_FUSED(KB, NS)                                                \
  hipLaunchKernelGGL((attention_tile_fused<KB, kFusedWaves, false, true, NS>),\
                     sw::grid_dim(grid, 64 * kFusedWaves), dim3(64 * kFusedWaves), 0, st, ro, \
                     col, val, lhs, rhs, nullptr, out, nullptr, nullptr,      \
                     nullptr, (int32_t)rows, cols, (int32_t)kdim, (int64_t)0, \
                     alpha, beta, (uint32_t)(nnz - 4), kind)
        if (kb == 1 && val != nullptr)
          SW_SDDMM_FUSED(1, false);
        else if (kb == 1)
          SW_SDDMM_FUSED(1, true);
        else if (val != nullptr)
          SW_SDDMM_FUSED(2, false);
        else
          SW_SDDMM_FUSED(2, true);
#undef SW_SDDMM_FUSED
        return launch_check("SDDMM tile MFMA kernel");
      }
#define SW_SDDMM_TILE(KB)                                                     \
  hipLaunchKernelGGL((sddmm_tile_mfma<KB, kSddmmTileWaves>),                  \
                     sw::grid_dim(grid, 64 * kSddmmTileWaves), dim3(64 * kSddmmTileWaves), 0, st, \
                     ro, col, val, lhs, rhs, out, (int32_t)rows, cols,        \
                     (int32_t)kdim, kind, alpha, beta)
      if (kb == 1)
        SW_SDDMM_TILE(1);
      else if (kb == 2)
        SW_SDDMM_TILE(2);
      else
        SW_SDDMM_TILE(4);
#undef SW_SDDMM_TILE
      return launch_check("SDDMM tile MFMA kernel");
    } else if (aligned16(lhs) && narrow_offsets(kdim, cols) &&
               narrow_offsets(nnz, 1)) {
      // bf16 tiles: a 128-bit lhs load per K step, K^T gathered with 32-bit
      // lane byte offsets
      int rc = grid_for(rows, 16, "SDDMM", &grid);
      if (rc)
        return rc;
      // d of 64 or 128, and no sample values or an output apart from them:
      // the fused attention kernel's product phase, as for fp32
      if ((kdim == 64 || kdim == 128) && nnz >= 4 &&
          (val == nullptr || out + nnz <= val || val + nnz <= out)) {
#define SW_SDDMM_FUSED(KB, NS)                                                \
  hipLaunchKernelGGL((attention_tile_fused_bf16<KB, kFusedWaves, true, NS>),  \
                     sw::grid_dim(grid, 64 * kFusedWaves), dim3(64 * kFusedWaves), 0, st, ro, \
                     col, val, lhs, rhs, nullptr, out, nullptr, nullptr,      \
                     nullptr, (int32_t)rows, cols, (int32_t)kdim, (int64_t)0, \
                     alpha, beta, (uint32_t)(nnz - 4), kind)
        if (kb == 1 && val != nullptr)
          SW_SDDMM_FUSED(1, false);
        else if (kb == 1)
          SW_SDDMM_FUSED(1, true);
        else if (val != nullptr)
          SW_SDDMM_FUSED(2, false);
        else
          SW_SDDMM_FUSED(2, true);
#undef SW_SDDMM_FUSED
        return launch_check("SDDMM tile MFMA kernel");
      }
#define SW_SDDMM_TILE(KB)                                                     \
  hipLaunchKernelGGL((sddmm_tile_mfma_bf16<KB, kSddmmTileWaves>),             \
                     sw::grid_dim(grid, 64 * kSddmmTileWaves), dim3(64 * kSddmmTileWaves), 0, st, \
                     ro, col, val, lhs, rhs, out, (int32_t)rows, cols,        \
                     (int32_t)kdim, kind, alpha, beta)
      if (kb == 1)
        SW_SDDMM_TILE(1);
      else if (kb == 2)
        SW_SDDMM_TILE(2);
      else
        SW_SDDMM_TILE(4);
#undef SW_SDDMM_TILE
      return launch_check("SDDMM tile MFMA kernel");
    }
  }
  if (streq(o.sddmm_mapping, "wave-per-row") ||
      (streq(o.sddmm_mapping, "row-tile-mfma")) ||
      o.sddmm_lanes_per_row == 64) {
    int rc = grid_for(rows, 4, "SDDMM", &grid);
    if (rc)
      return rc;
    hipLaunchKernelGGL(sddmm_wave_per_row<T>, sw::grid_dim(grid, 256), dim3(256),
                       0, st, ro, col, val, lhs, rhs, out, (int32_t)rows, cols,
                       (int32_t)kdim, kind, alpha, beta);
  } else {
    const int64_t B = o.sddmm_block_size;
    int rc = grid_for(rows, B, "SDDMM", &grid);
    if (rc)
      return rc;
    // 16 positions per step where a workgroup of at most 512 threads lets a
    // lane hold 256 registers (configuration 5, fp32: 602 -> 478 us with 256
    // threads); four under the 1024-thread bound.  kdim 64 or 128 and whole
    // waves of at most 256-thread workgroups (one wave per SIMD, so the tile
    // and the per-row steps have 512 registers without spills; bf16 also a
    // 16-byte aligned lhs), with the rhs's bytes within 32 bits (the
    // tile's lane offsets): 64-row matrix-core tiles first
    const bool tiles = (kdim == 64 || kdim == 128) && B % kWave == 0 &&
                       B <= 256 && (sizeof(T) == 4 || aligned16(lhs)) &&
                       (int64_t)sizeof(T) * kdim * cols <= (int64_t)UINT32_MAX;
    if (tiles && kdim == 64)
      hipLaunchKernelGGL((sddmm_thread_per_row<T, 16, 256, 1>),
                         sw::grid_dim(grid, (unsigned)B), dim3((unsigned)B), 0, st, ro,
                         col, val, lhs, rhs, out, (int32_t)rows, cols,
                         (int32_t)kdim, kind, alpha, beta);
    else if (tiles)
      hipLaunchKernelGGL((sddmm_thread_per_row<T, 16, 256, 2>),
                         sw::grid_dim(grid, (unsigned)B), dim3((unsigned)B), 0, st, ro,
                         col, val, lhs, rhs, out, (int32_t)rows, cols,
                         (int32_t)kdim, kind, alpha, beta);
    else if (B <= 512)
      hipLaunchKernelGGL((sddmm_thread_per_row<T, 16, 512>),
                         sw::grid_dim(grid, (unsigned)B), dim3((unsigned)B), 0, st, ro,
                         col, val, lhs, rhs, out, (int32_t)rows, cols,
                         (int32_t)kdim, kind, alpha, beta);
    else
      hipLaunchKernelGGL((sddmm_thread_per_row<T, 4, 1024>),
                         sw::grid_dim(grid, (unsigned)B), dim3((unsigned)B), 0, st, ro,
                         col, val, lhs, rhs, out, (int32_t)rows, cols,
                         (int32_t)kdim, kind, alpha, beta);
  }
  return launch_check("SDDMM kernel");
}

template <typename T>
int launch_row_reduce(const int32_t *ro, const T *val, T *out, int64_t rows,
                      bool is_max, const sw_options &o, hipStream_t st) {
  int64_t grid;
  if (o.sddmm_lanes_per_row == 64) {
    int rc = grid_for(rows, 4, "CSR row reduction", &grid);
    if (rc)
      return rc;
    if (is_max)
      hipLaunchKernelGGL((row_reduce_wave<true, T>), sw::grid_dim(grid, 256),
                         dim3(256), 0, st, ro, val, out, (int32_t)rows);
    else
      hipLaunchKernelGGL((row_reduce_wave<false, T>), sw::grid_dim(grid, 256),
                         dim3(256), 0, st, ro, val, out, (int32_t)rows);
  } else {
    const int64_t B = o.row_reduction_block_size;
    int rc = grid_for(rows, B, "CSR row reduction", &grid);
    if (rc)
      return rc;
    if (is_max)
      hipLaunchKernelGGL((row_reduce_thread<true, T>), sw::grid_dim(grid, (unsigned)B),
                         dim3((unsigned)B), 0, st, ro, val, out, (int32_t)rows);
    else
      hipLaunchKernelGGL((row_reduce_thread<false, T>), sw::grid_dim(grid, (unsigned)B),
                         dim3((unsigned)B), 0, st, ro, val, out, (int32_t)rows);
  }
  return launch_check("CSR row reduction kernel");
}

template <typename T>
int launch_rowwise_map(const int32_t *ro, const T *val, const T *rowv, T *out,
                       int64_t rows, int kind, const sw_options &o,
                       hipStream_t st) {
  int64_t grid;
  if (o.sddmm_lanes_per_row == 64) {
    int rc = grid_for(rows, 4, "CSR row-wise map", &grid);
    if (rc)
      return rc;
    hipLaunchKernelGGL(rowwise_map_wave<T>, sw::grid_dim(grid, 256), dim3(256), 0,
                       st, ro, val, rowv, out, (int32_t)rows, kind);
  } else {
    const int64_t B = o.rowwise_map_block_size;
    int rc = grid_for(rows, B, "CSR row-wise map", &grid);
    if (rc)
      return rc;
#define SW_MAP_THREAD(KIND)                                                   \
  hipLaunchKernelGGL((rowwise_map_thread<T, KIND>), sw::grid_dim(grid, B),   \
                     dim3((unsigned)B), 0, st, ro, val, rowv, out,            \
                     (int32_t)rows)
    switch (kind) {
    case SW_MAP_EXP_SUB:
      SW_MAP_THREAD(SW_MAP_EXP_SUB);
      break;
    case SW_MAP_DIV:
      SW_MAP_THREAD(SW_MAP_DIV);
      break;
    case SW_MAP_SUB:
      SW_MAP_THREAD(SW_MAP_SUB);
      break;
    default:
      SW_MAP_THREAD(SW_MAP_MUL);
      break;
    }
#undef SW_MAP_THREAD
  }
  return launch_check("CSR row-wise map kernel");
}

// ---- entry points (fp32 and bf16 share them) --------------------------------

template <typename T>
int sddmm_entry(const int32_t *row_offsets, const int32_t *column_indices,
                const T *values, const T *lhs, const T *rhs, T *output_values,
                int64_t rows, int64_t cols, int64_t nnz, int64_t kdim,
                int combine, float alpha, float beta, const sw_options *opts,
                void *stream) {
  clear_error();
  sw_options o;
  int rc = resolve_options(opts, &o);
  if (rc)
    return rc;
  if (combine != SW_SDDMM_MUL && combine != SW_SDDMM_AFFINE &&
      combine != SW_SDDMM_DOT)
    return fail(SW_ERR_INVALID_ARGUMENT, "unknown SDDMM combine kind %d",
                combine);
  rc = check_csr(row_offsets, column_indices,
                 combine == SW_SDDMM_DOT ? (const void *)output_values
                                         : (const void *)values,
                 rows, nnz, true);
  if (!rc)
    rc = check_value_alignment(sizeof(T), {values, lhs, rhs, output_values});
  if (rc)
    return rc;
  if (cols < 0 || kdim < 0 || kdim > INT32_MAX)
    return fail(SW_ERR_INVALID_SHAPE, "invalid SDDMM dense shapes");
  if (rows == 0 || nnz == 0)
    return SW_OK;
  if (!output_values || (kdim > 0 && (!lhs || !rhs)))
    return fail(SW_ERR_INVALID_ARGUMENT, "SDDMM operand pointer is null");
  return launch_sddmm<T>(row_offsets, column_indices,
                         combine == SW_SDDMM_DOT ? nullptr : values, lhs, rhs,
                         output_values, rows, cols, nnz, kdim, combine, alpha,
                         beta, o, as_stream(stream));
}

template <typename T>
int row_reduce_entry(const int32_t *row_offsets, const int32_t *column_indices,
                     const T *values, T *output, int64_t rows, int64_t nnz,
                     const char *kind, const sw_options *opts, void *stream) {
  clear_error();
  sw_options o;
  int rc = resolve_options(opts, &o);
  if (rc)
    return rc;
  if (!kind || (!streq(kind, "sum") && !streq(kind, "max")))
    return fail(SW_ERR_INVALID_ARGUMENT,
                "expected CSR row reduction kind 'sum' or 'max', but got '%s'",
                kind ? kind : "(null)");
  rc = check_csr(row_offsets, column_indices, values, rows, nnz, false);
  if (!rc)
    rc = check_value_alignment(sizeof(T), {values, output});
  if (rc)
    return rc;
  if (rows == 0)
    return SW_OK;
  if (!output)
    return fail(SW_ERR_INVALID_ARGUMENT, "output pointer is null");
  return launch_row_reduce<T>(row_offsets, values, output, rows,
                              streq(kind, "max"), o, as_stream(stream));
}

template <typename T>
int rowwise_map_entry(const int32_t *row_offsets,
                      const int32_t *column_indices, const T *values,
                      const T *row_values, T *output_values, int64_t rows,
                      int64_t nnz, int map, const sw_options *opts,
                      void *stream) {
  clear_error();
  sw_options o;
  int rc = resolve_options(opts, &o);
  if (rc)
    return rc;
  if (map < SW_MAP_EXP_SUB || map > SW_MAP_MUL)
    return fail(SW_ERR_INVALID_ARGUMENT, "unknown row-wise map kind %d", map);
  rc = check_csr(row_offsets, column_indices, values, rows, nnz, false);
  if (!rc)
    rc = check_value_alignment(sizeof(T), {values, row_values, output_values});
  if (rc)
    return rc;
  if (rows == 0 || nnz == 0)
    return SW_OK;
  if (!output_values || !row_values)
    return fail(SW_ERR_INVALID_ARGUMENT, "row-wise map pointer is null");
  return launch_rowwise_map<T>(row_offsets, values, row_values, output_values,
                               rows, map, o, as_stream(stream));
}

// The whole chain in one kernel per 16-row tile when the options ask for
// matrix-core tiles and the shapes fit the fused kernel; returns true when it
// was launched (rc holds the launch status).
bool launch_fused_attention(const int32_t *ro, const int32_t *col,
                            const float *mask, const float *q,
                            const float *kt, const float *v, float *scores,
                            float *rmax, float *rsum, float *out,
                            int64_t rows, int64_t cols, int64_t nnz,
                            int64_t d, int64_t dv, float alpha, float beta,
                            hipStream_t st, int *rc) {
  if (!((d == 64 || d == 128) && dv > 0 && dv % 16 == 0 && nnz >= 4 &&
        narrow_offsets(nnz, 1) && narrow_offsets(cols, d) &&
        narrow_offsets(cols, dv)))
    return false;
  int64_t grid;
  *rc = grid_for(rows, 16, "fused attention", &grid);
  if (*rc)
    return true;
  // interleaved output tiles (configuration 5: 25.2 -> 24.0 us)
  const bool il = dv % 64 == 0 && aligned16(v) && aligned16(out);
#define SW_FUSED(KB, IL)                                                      \
  hipLaunchKernelGGL((attention_tile_fused<KB, kFusedWaves, IL, false>),      \
                     sw::grid_dim(grid, 64 * kFusedWaves), dim3(64 * kFusedWaves), 0, st, ro, \
                     col, mask, q, kt, v, scores, rmax, rsum, out,            \
                     (int32_t)rows, cols, (int32_t)d, dv, alpha, beta,        \
                     (uint32_t)(nnz - 4), (int)SW_SDDMM_AFFINE)
  if (d == 64 && il)
    SW_FUSED(1, true);
  else if (d == 64)
    SW_FUSED(1, false);
  else if (il)
    SW_FUSED(2, true);
  else
    SW_FUSED(2, false);
#undef SW_FUSED
  *rc = launch_check("fused attention kernel");
  return true;
}

bool launch_fused_attention(const int32_t *ro, const int32_t *col,
                            const uint16_t *mask, const uint16_t *q,
                            const uint16_t *kt, const uint16_t *v,
                            uint16_t *scores, uint16_t *rmax, uint16_t *rsum,
                            uint16_t *out, int64_t rows, int64_t cols,
                            int64_t nnz, int64_t d, int64_t dv, float alpha,
                            float beta, hipStream_t st, int *rc) {
  if (!((d == 64 || d == 128) && dv > 0 && dv % 64 == 0 && nnz >= 4 &&
        aligned16(q) &&
        (reinterpret_cast<uintptr_t>(v) & 7u) == 0 &&
        (reinterpret_cast<uintptr_t>(out) & 7u) == 0 &&
        narrow_offsets(nnz, 1) && narrow_offsets(cols, d) &&
        narrow_offsets(cols, dv)))
    return false;
  int64_t grid;
  *rc = grid_for(rows, 16, "fused attention", &grid);
  if (*rc)
    return true;
#define SW_FUSED(KB)                                                          \
  hipLaunchKernelGGL((attention_tile_fused_bf16<KB, kFusedWaves, false>),     \
                     sw::grid_dim(grid, 64 * kFusedWaves), dim3(64 * kFusedWaves), 0, st, ro, \
                     col, mask, q, kt, v, scores, rmax, rsum, out,            \
                     (int32_t)rows, cols, (int32_t)d, dv, alpha, beta,        \
                     (uint32_t)(nnz - 4), (int)SW_SDDMM_AFFINE)
  if (d == 64)
    SW_FUSED(1);
  else
    SW_FUSED(2);
#undef SW_FUSED
  *rc = launch_check("fused attention kernel");
  return true;
}

// The tile floor: the fused kernel launch_fused_attention would run for
// these operands, in its FLOOR form; false when the shapes do not take the
// fused kernel.
bool launch_attention_floor(const int32_t *ro, const int32_t *col,
                            const float *mask, const float *q,
                            const float *kt, const float *v, float *scores,
                            float *rmax, float *rsum, float *out,
                            int64_t rows, int64_t cols, int64_t nnz,
                            int64_t d, int64_t dv, hipStream_t st, int *rc) {
  if (!((d == 64 || d == 128) && dv > 0 && dv % 16 == 0 && nnz >= 4 &&
        narrow_offsets(nnz, 1) && narrow_offsets(cols, d) &&
        narrow_offsets(cols, dv)))
    return false;
  int64_t grid;
  *rc = grid_for(rows, 16, "attention tile floor", &grid);
  if (*rc)
    return true;
  const bool il = dv % 64 == 0 && aligned16(v) && aligned16(out);
#define SW_FLOOR(KB, IL)                                                      \
  hipLaunchKernelGGL(                                                         \
      (attention_tile_fused<KB, kFusedWaves, IL, false, false, true>),        \
      sw::grid_dim(grid, 64 * kFusedWaves), dim3(64 * kFusedWaves), 0, st, ro, col, mask, q,  \
      kt, v, scores, rmax, rsum, out, (int32_t)rows, cols, (int32_t)d, dv,    \
      1.0f, 0.0f, (uint32_t)(nnz - 4), (int)SW_SDDMM_AFFINE)
  if (d == 64 && il)
    SW_FLOOR(1, true);
  else if (d == 64)
    SW_FLOOR(1, false);
  else if (il)
    SW_FLOOR(2, true);
  else
    SW_FLOOR(2, false);
#undef SW_FLOOR
  *rc = launch_check("attention tile floor kernel");
  return true;
}

bool launch_attention_floor(const int32_t *ro, const int32_t *col,
                            const uint16_t *mask, const uint16_t *q,
                            const uint16_t *kt, const uint16_t *v,
                            uint16_t *scores, uint16_t *rmax, uint16_t *rsum,
                            uint16_t *out, int64_t rows, int64_t cols,
                            int64_t nnz, int64_t d, int64_t dv,
                            hipStream_t st, int *rc) {
  if (!((d == 64 || d == 128) && dv > 0 && dv % 64 == 0 && nnz >= 4 &&
        aligned16(q) &&
        (reinterpret_cast<uintptr_t>(v) & 7u) == 0 &&
        (reinterpret_cast<uintptr_t>(out) & 7u) == 0 &&
        narrow_offsets(nnz, 1) && narrow_offsets(cols, d) &&
        narrow_offsets(cols, dv)))
    return false;
  int64_t grid;
  *rc = grid_for(rows, 16, "attention tile floor", &grid);
  if (*rc)
    return true;
#define SW_FLOOR(KB)                                                          \
  hipLaunchKernelGGL(                                                         \
      (attention_tile_fused_bf16<KB, kFusedWaves, false, false, true>),       \
      sw::grid_dim(grid, 64 * kFusedWaves), dim3(64 * kFusedWaves), 0, st, ro, col, mask, q,  \
      kt, v, scores, rmax, rsum, out, (int32_t)rows, cols, (int32_t)d, dv,    \
      1.0f, 0.0f, (uint32_t)(nnz - 4), (int)SW_SDDMM_AFFINE)
  if (d == 64)
    SW_FLOOR(1);
  else
    SW_FLOOR(2);
#undef SW_FLOOR
  *rc = launch_check("attention tile floor kernel");
  return true;
}

template <typename T>
int attention_floor_entry(const int32_t *row_offsets,
                          const int32_t *column_indices, const T *mask_values,
                          const T *query, const T *transposed_key,
                          const T *value, T *scores, T *row_maximum,
                          T *row_sum, T *output, int64_t rows, int64_t cols,
                          int64_t nnz, int64_t d, int64_t dv, void *stream) {
  int rc = check_csr(row_offsets, column_indices, mask_values, rows, nnz,
                     true);
  if (!rc)
    rc = check_value_alignment(sizeof(T), {mask_values, query, transposed_key,
                                           value, scores, row_maximum,
                                           row_sum, output});
  if (rc)
    return rc;
  if (cols < 0 || d < 0 || dv < 0 || d > INT32_MAX)
    return fail(SW_ERR_INVALID_SHAPE, "invalid attention shapes");
  if (rows == 0)
    return SW_OK;
  if (!row_maximum || !row_sum || !output || !scores || !query ||
      !transposed_key || !value)
    return fail(SW_ERR_INVALID_ARGUMENT, "attention buffer pointer is null");
  if (!launch_attention_floor(row_offsets, column_indices, mask_values, query,
                              transposed_key, value, scores, row_maximum,
                              row_sum, output, rows, cols, nnz, d, dv,
                              as_stream(stream), &rc))
    return fail(SW_ERR_INVALID_ARGUMENT,
                "the tile floor needs the fused kernel's shapes: d of 64 or "
                "128, dv a multiple of %d, at least 4 entries%s",
                sizeof(T) == 4 ? 16 : 64,
                sizeof(T) == 4 ? "" : ", aligned query, value and output");
  return rc;
}

template <typename T>
int attention_entry(const int32_t *row_offsets, const int32_t *column_indices,
                    const T *mask_values, const T *query,
                    const T *transposed_key, const T *value, T *scores,
                    T *row_maximum, T *row_sum, T *output, int64_t rows,
                    int64_t cols, int64_t nnz, int64_t d, int64_t dv,
                    float alpha, float beta, const sw_options *opts,
                    void *stream) {
  clear_error();
  sw_options o;
  int rc = resolve_options(opts, &o);
  if (rc)
    return rc;
  rc = check_csr(row_offsets, column_indices, mask_values, rows, nnz, true);
  if (!rc)
    rc = check_value_alignment(sizeof(T), {mask_values, query, transposed_key,
                                           value, scores, row_maximum,
                                           row_sum, output});
  if (rc)
    return rc;
  if (cols < 0 || d < 0 || dv < 0 || d > INT32_MAX)
    return fail(SW_ERR_INVALID_SHAPE, "invalid attention shapes");
  if constexpr (std::is_same_v<T, uint16_t>) {
    rc = check_bf16_spmm_mapping(o); // before any launch
    if (rc)
      return rc;
  }
  if (rows == 0)
    return SW_OK;
  if (!row_maximum || !row_sum || (dv > 0 && !output) ||
      (nnz > 0 && (!scores || !query || !transposed_key || (dv > 0 && !value))))
    return fail(SW_ERR_INVALID_ARGUMENT, "attention buffer pointer is null");
  hipStream_t st = as_stream(stream);
  if (nnz > 0 && o.sddmm_lanes_per_row == 64 &&
      streq(o.sddmm_mapping, "row-tile-mfma") &&
      streq(o.spmm_mapping, "row-tile-mfma") &&
      launch_fused_attention(row_offsets, column_indices, mask_values, query,
                             transposed_key, value, scores, row_maximum,
                             row_sum, output, rows, cols, nnz, d, dv, alpha,
                             beta, st, &rc))
    return rc;
  if (nnz > 0) {
    rc = launch_sddmm<T>(row_offsets, column_indices, mask_values, query,
                         transposed_key, scores, rows, cols, nnz, d,
                         SW_SDDMM_AFFINE, alpha, beta, o, st);
    if (rc)
      return rc;
  }
  if (o.sddmm_lanes_per_row == 64) {
    // wave row ops: the four softmax ops run as one kernel
    int64_t grid = std::max<int64_t>(ceil_div(rows, 4), 1);
    rc = check_grid(grid, 256, "attention softmax");
    if (rc)
      return rc;
    hipLaunchKernelGGL(row_softmax_wave<T>, sw::grid_dim(grid, 256), dim3(256), 0,
                       st, row_offsets, scores, row_maximum, row_sum,
                       (int32_t)rows);
    rc = launch_check("attention softmax kernel");
    if (rc)
      return rc;
    if (dv == 0)
      return SW_OK;
    return launch_spmm(row_offsets, column_indices, scores, value, output,
                       rows, cols, nnz, dv, o, "attention output SpMM", st);
  }
  rc = launch_row_reduce<T>(row_offsets, scores, row_maximum, rows, true, o,
                            st);
  if (rc)
    return rc;
  if (nnz > 0) {
    rc = launch_rowwise_map<T>(row_offsets, scores, row_maximum, scores, rows,
                               SW_MAP_EXP_SUB, o, st);
    if (rc)
      return rc;
  }
  rc = launch_row_reduce<T>(row_offsets, scores, row_sum, rows, false, o, st);
  if (rc)
    return rc;
  if (nnz > 0) {
    rc = launch_rowwise_map<T>(row_offsets, scores, row_sum, scores, rows,
                               SW_MAP_DIV, o, st);
    if (rc)
      return rc;
  }
  if (dv == 0)
    return SW_OK;
  return launch_spmm(row_offsets, column_indices, scores, value, output, rows,
                     cols, nnz, dv, o, "attention output SpMM", st);
}

} // namespace sw

extern "C" int sw_sddmm_csr_f32(const int32_t *row_offsets,
                                const int32_t *column_indices,
                                const float *values, const float *lhs,
                                const float *rhs, float *output_values,
                                int64_t rows, int64_t cols, int64_t nnz,
                                int64_t kdim, int combine, float alpha,
                                float beta, const sw_options *opts,
                                void *stream) {
  return sw::sddmm_entry<float>(row_offsets, column_indices, values, lhs, rhs,
                                output_values, rows, cols, nnz, kdim, combine,
                                alpha, beta, opts, stream);
}

extern "C" int sw_sddmm_csr_bf16(const int32_t *row_offsets,
                                 const int32_t *column_indices,
                                 const uint16_t *values, const uint16_t *lhs,
                                 const uint16_t *rhs, uint16_t *output_values,
                                 int64_t rows, int64_t cols, int64_t nnz,
                                 int64_t kdim, int combine, float alpha,
                                 float beta, const sw_options *opts,
                                 void *stream) {
  return sw::sddmm_entry<uint16_t>(row_offsets, column_indices, values, lhs,
                                   rhs, output_values, rows, cols, nnz, kdim,
                                   combine, alpha, beta, opts, stream);
}

extern "C" int sw_csr_row_reduce_f32(const int32_t *row_offsets,
                                     const int32_t *column_indices,
                                     const float *values, float *output,
                                     int64_t rows, int64_t nnz,
                                     const char *kind, const sw_options *opts,
                                     void *stream) {
  return sw::row_reduce_entry<float>(row_offsets, column_indices, values,
                                     output, rows, nnz, kind, opts, stream);
}

extern "C" int sw_csr_row_reduce_bf16(const int32_t *row_offsets,
                                      const int32_t *column_indices,
                                      const uint16_t *values, uint16_t *output,
                                      int64_t rows, int64_t nnz,
                                      const char *kind, const sw_options *opts,
                                      void *stream) {
  return sw::row_reduce_entry<uint16_t>(row_offsets, column_indices, values,
                                        output, rows, nnz, kind, opts, stream);
}

extern "C" int sw_csr_rowwise_map_f32(const int32_t *row_offsets,
                                      const int32_t *column_indices,
                                      const float *values,
                                      const float *row_values,
                                      float *output_values, int64_t rows,
                                      int64_t nnz, int map,
                                      const sw_options *opts, void *stream) {
  return sw::rowwise_map_entry<float>(row_offsets, column_indices, values,
                                      row_values, output_values, rows, nnz,
                                      map, opts, stream);
}

extern "C" int sw_csr_rowwise_map_bf16(const int32_t *row_offsets,
                                       const int32_t *column_indices,
                                       const uint16_t *values,
                                       const uint16_t *row_values,
                                       uint16_t *output_values, int64_t rows,
                                       int64_t nnz, int map,
                                       const sw_options *opts, void *stream) {
  return sw::rowwise_map_entry<uint16_t>(row_offsets, column_indices, values,
                                         row_values, output_values, rows, nnz,
                                         map, opts, stream);
}

extern "C" int sw_sparse_attention_f32(
    const int32_t *row_offsets, const int32_t *column_indices,
    const float *mask_values, const float *query, const float *transposed_key,
    const float *value, float *scores, float *row_maximum, float *row_sum,
    float *output, int64_t rows, int64_t cols, int64_t nnz, int64_t d,
    int64_t dv, float alpha, float beta, const sw_options *opts,
    void *stream) {
  return sw::attention_entry<float>(
      row_offsets, column_indices, mask_values, query, transposed_key, value,
      scores, row_maximum, row_sum, output, rows, cols, nnz, d, dv, alpha,
      beta, opts, stream);
}

extern "C" int sw_attention_tile_floor(
    const int32_t *row_offsets, const int32_t *column_indices,
    const void *mask_values, const void *query, const void *transposed_key,
    const void *value, void *scores, void *row_maximum, void *row_sum,
    void *output, int64_t rows, int64_t cols, int64_t nnz, int64_t d,
    int64_t dv, int value_bytes, void *stream) {
  sw::clear_error();
  if (value_bytes == 4)
    return sw::attention_floor_entry<float>(
        row_offsets, column_indices, static_cast<const float *>(mask_values),
        static_cast<const float *>(query),
        static_cast<const float *>(transposed_key),
        static_cast<const float *>(value), static_cast<float *>(scores),
        static_cast<float *>(row_maximum), static_cast<float *>(row_sum),
        static_cast<float *>(output), rows, cols, nnz, d, dv, stream);
  if (value_bytes == 2)
    return sw::attention_floor_entry<uint16_t>(
        row_offsets, column_indices,
        static_cast<const uint16_t *>(mask_values),
        static_cast<const uint16_t *>(query),
        static_cast<const uint16_t *>(transposed_key),
        static_cast<const uint16_t *>(value), static_cast<uint16_t *>(scores),
        static_cast<uint16_t *>(row_maximum),
        static_cast<uint16_t *>(row_sum), static_cast<uint16_t *>(output),
        rows, cols, nnz, d, dv, stream);
  return sw::fail(SW_ERR_INVALID_ARGUMENT,
                  "tile floor value bytes must be 4 or 2, but got %d",
                  value_bytes);
}

extern "C" int sw_sparse_attention_bf16(
    const int32_t *row_offsets, const int32_t *column_indices,
    const uint16_t *mask_values, const uint16_t *query,
    const uint16_t *transposed_key, const uint16_t *value, uint16_t *scores,
    uint16_t *row_maximum, uint16_t *row_sum, uint16_t *output, int64_t rows,
    int64_t cols, int64_t nnz, int64_t d, int64_t dv, float alpha, float beta,
    const sw_options *opts, void *stream) {
  return sw::attention_entry<uint16_t>(
      row_offsets, column_indices, mask_values, query, transposed_key, value,
      scores, row_maximum, row_sum, output, rows, cols, nnz, d, dv, alpha,
      beta, opts, stream);
}
