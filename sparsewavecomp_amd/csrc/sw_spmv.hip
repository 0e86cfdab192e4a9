// sparsewave.spmv on gfx950: the row mappings (thread, wave, block per row)
// and the position mappings (thread and wave per position), with their
// launchers behind sw_spmv_csr_f32; COO SpMV behind sw_spmv_coo_f32.
//
// Reference kernels (generated IR, not hand-written code):
//   thread-per-row     SparseWaveToGPU.cpp:216-274
//   wave-per-row       SparseWaveToGPU.cpp:276-354, SparseGPUUtils.cpp:34-59,236-245
//   block-per-row      SparseWaveToGPU.cpp:356-487
//   thread-per-position SparsePositionScheduling.cpp:135-316
//   wave-per-position  SparsePositionScheduling.cpp:318-403,
//                      SparsePositionToSCF.cpp:190-271, SparseGPUUtils.cpp:247-292
//   COO thread-per-nonzero SparseWaveToGPU.cpp:154-214
#include "sw_device.h"
#include "sw_internal.h"

using namespace swd;

namespace {

// ---------------------------------------------------------------------------
// sum of val[p] * x[col[p]] over p = p0, p0+stride, ... < e, added to acc in
// position order, with kRowUnroll positions' loads and gathers in flight per
// step (a loop that loads, gathers and multiplies one position at a time
// waits a full memory trip per position).  DEEP > 0 first takes steps of
// DEEP positions while that many remain: a long row handled by one thread
// then needs DEEP times fewer memory trips.
constexpr int kRowUnroll = 4;

// x[c].  NARROW (the host's guarantee that 4 * cols fits 32 bits): the
// wave-uniform base x plus a 32-bit lane byte offset, which the load takes
// directly; otherwise a 64-bit lane address.  On configuration 2 the narrow
// form measured thread-per-row 453 -> 436 us, the position mapping
// 209.1 -> 207.7 us, wave-per-row (16 lanes) 246.3 -> 245.8 us.
template <bool NARROW>
__device__ __forceinline__ float gather(const float *__restrict__ x,
                                        int32_t c) {
  if constexpr (NARROW)
    return *at_bytes(x, 4u * (uint32_t)c);
  else
    return x[c];
}

// Sum of val[q] * x[col[q]] for q = p, p + stride, ... < e.  Every index
// computed here is below e + DEEP * stride <= nnz + 2^14, which the host's
// nnz limit (check_csr) keeps inside int32.
template <bool NARROW, int DEEP = 0>
__device__ __forceinline__ float strided_dot(const int32_t *__restrict__ col,
                                             const float *__restrict__ val,
                                             const float *__restrict__ x,
                                             int32_t p, int32_t e,
                                             int32_t stride, float acc) {
  if constexpr (DEEP > 0) {
    for (; p + (DEEP - 1) * stride < e; p += DEEP * stride) {
      int32_t c[DEEP];
      float v[DEEP], xv[DEEP];
#pragma unroll
      for (int u = 0; u < DEEP; ++u) {
        c[u] = ld_stream(col + p + u * stride);
        v[u] = ld_stream(val + p + u * stride);
      }
#pragma unroll
      for (int u = 0; u < DEEP; ++u)
        xv[u] = gather<NARROW>(x, c[u]);
#pragma unroll
      for (int u = 0; u < DEEP; ++u)
        acc = __builtin_fmaf(v[u], xv[u], acc);
    }
  }
  for (; p + (kRowUnroll - 1) * stride < e; p += kRowUnroll * stride) {
    int32_t c[kRowUnroll];
    float v[kRowUnroll], xv[kRowUnroll];
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u) {
      c[u] = ld_stream(col + p + u * stride);
      v[u] = ld_stream(val + p + u * stride);
    }
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u)
      xv[u] = gather<NARROW>(x, c[u]);
#pragma unroll
    for (int u = 0; u < kRowUnroll; ++u)
      acc = __builtin_fmaf(v[u], xv[u], acc);
  }
  for (; p < e; p += stride)
    acc = __builtin_fmaf(ld_stream(val + p), gather<NARROW>(x, col[p]), acc);
  return acc;
}

// ---------------------------------------------------------------------------
// thread-per-row: one thread accumulates one row sequentially from zero.
// Long rows take steps of kThreadRowDeep positions: the kernel's time is the
// longest rows' chain of memory trips (config 2 has rows of 4096).
constexpr int kThreadRowDeep = 16;
template <bool NARROW>
__global__ __launch_bounds__(1024) void spmv_thread_per_row(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ x,
    float *__restrict__ y, int32_t rows) {
  int64_t r = block_id() * blockDim.x + threadIdx.x;
  if (r >= rows)
    return;
  int32_t s = ro[r], e = ro[r + 1];
  y[r] = strided_dot<NARROW, kThreadRowDeep>(col, val, x, s, e, 1, 0.0f);
}

// ---------------------------------------------------------------------------
// wave-per-row with G lanes per row (G = 64 is the reference's one wave per
// row).  Lane l of a group sums positions start+l, start+l+G, ...; the group
// sum uses DPP / swizzle butterflies; the group's first lane stores.  Lanes
// of long rows take steps of kGroupRowDeep positions (16 lanes per row:
// 276 -> 247 us on configuration 2, 32 lanes: 274 -> 263 us).
constexpr int kGroupRowDeep = 16;
template <int G, bool NARROW>
__global__ __launch_bounds__(1024) void spmv_group_per_row(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ x,
    float *__restrict__ y, int32_t rows) {
  const int groups_per_block = blockDim.x / G;
  int64_t r = block_id() * groups_per_block + threadIdx.x / G;
  const int gl = threadIdx.x & (G - 1);
  float acc = 0.0f;
  if (r < rows) {
    int32_t s = ro[r], e = ro[r + 1];
    acc = strided_dot<NARROW, kGroupRowDeep>(col, val, x, s + gl, e, G,
                                             0.0f);
  }
  // every lane of the wave takes part in the butterfly
  acc = group_sum<G>(acc);
  if (r < rows && gl == 0)
    y[r] = acc;
}

// ---------------------------------------------------------------------------
// block-per-row: the block strides the row, each wave reduces its partial
// sum, partials meet in LDS, wave 0 reduces them and lane 0 stores.
template <bool NARROW>
__global__ __launch_bounds__(1024) void spmv_block_per_row(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ x,
    float *__restrict__ y, int32_t rows) {
  __shared__ float partial[1024 / kWave];
  const int64_t r = block_id();
  const int t = threadIdx.x;
  const int B = blockDim.x;
  if (r >= rows)
    return; // block-uniform: no barrier follows for this block
  const int32_t s = ro[r], e = ro[r + 1];
  if (e - s <= kWave) { // block-uniform
    // A row of at most one wave's positions: only wave 0 holds products,
    // each thread one, and the other waves' partial sums are zeros.  Wave
    // 0 alone gives the same sum -- its butterfly, plus the zeros the full
    // reduction would add (which turns a -0 into +0) -- without the LDS
    // exchange and the barrier.
    if (t >= kWave)
      return;
    const float w = wave_sum(strided_dot<NARROW>(col, val, x, s + t, e, B,
                                                 0.0f));
    if (t == 0)
      y[r] = w + 0.0f;
    return;
  }
  float acc = strided_dot<NARROW>(col, val, x, s + t, e, B, 0.0f);
  // blockDim.x is a multiple of 64 (validated), so every wave is full
  float w = wave_sum(acc);
  const int wave = t / kWave;
  if ((t & (kWave - 1)) == 0)
    partial[wave] = w;
  __syncthreads();
  if (wave == 0) {
    const int waves = B / kWave;
    float v = lane_id() < waves ? partial[lane_id()] : 0.0f;
    v = wave_sum(v);
    if (t == 0)
      y[r] = v;
  }
}

// ---------------------------------------------------------------------------
// Output initialisation of the position mappings
// (SparsePositionScheduling.cpp:31-47): one thread per output element.
// Each thread clears four consecutive elements (one 128-bit store when the
// output is 16-byte aligned).
__global__ __launch_bounds__(1024) void fill_zero_f32(float *__restrict__ y,
                                                      int64_t n) {
  int64_t i = (block_id() * blockDim.x + threadIdx.x) * 4;
  if (i + 4 <= n && (reinterpret_cast<uintptr_t>(y) & 15u) == 0) {
    *reinterpret_cast<v4f *>(y + i) = v4f{0.f, 0.f, 0.f, 0.f};
  } else {
    for (int64_t j = i; j < n && j < i + 4; ++j)
      y[j] = 0.0f;
  }
}


// ---------------------------------------------------------------------------
// Output initialisation of the wide-row SpMM position schedule.  There a row
// is accumulated atomically only when its positions belong to more than one
// wave; every other row receives exactly one plain store from the wave that
// holds it.  So only those rows, and empty rows (which no position reaches),
// need the zero the reference's init kernel writes
// (SparsePositionScheduling.cpp:31-47): one thread per row decides.
// Waves either own aligned chunks of `chunk` positions (chunk > 0) or the
// balanced partition of `units` units of P positions over `waves` waves.
__device__ __forceinline__ int64_t wave_of_position(int64_t p, int64_t chunk,
                                                    int64_t P, int64_t units,
                                                    int64_t waves) {
  if (chunk > 0)
    return p / chunk;
  const int64_t u = p / P;
  const int64_t base = units / waves, rem = units % waves;
  const int64_t big = (base + 1) * rem;
  return u < big ? u / (base + 1) : rem + (u - big) / base;
}

__global__ __launch_bounds__(256) void position_init(
    const int32_t *__restrict__ ro, float *__restrict__ out, int32_t rows,
    int64_t k, int64_t chunk, int64_t P, int64_t units, int64_t waves) {
  const int64_t r = block_id() * blockDim.x + threadIdx.x;
  if (r >= rows)
    return;
  const int32_t s = ro[r], e = ro[r + 1];
  if (s < e && wave_of_position(s, chunk, P, units, waves) ==
                   wave_of_position(e - 1, chunk, P, units, waves))
    return;
  float *o = out + r * k;
  if (k % 4 == 0 && (reinterpret_cast<uintptr_t>(o) & 15u) == 0) {
    for (int64_t c = 0; c < k; c += 4)
      *reinterpret_cast<v4f *>(o + c) = v4f{0.f, 0.f, 0.f, 0.f};
  } else {
    for (int64_t c = 0; c < k; ++c)
      o[c] = 0.0f;
  }
}

// ---------------------------------------------------------------------------
// The rows of a wave's positions: the wave's first and last positions'
// rows found by wave-uniform searches (scalar loads), so that each lane then
// searches only between them -- the same row as a search over all row
// offsets, with a few loads per lane instead of one per halving of rows.
struct WaveRows {
  uint32_t lo, hi; // lane searches run over ro[lo .. hi)
};
__device__ __forceinline__ WaveRows wave_rows(const int32_t *__restrict__ ro,
                                              int32_t rows, int64_t nnz,
                                              int64_t chunk) {
  const int64_t first = (block_id() * blockDim.x +
                         (int64_t)wave_in_group() * kWave) *
                        chunk;
  const int64_t last = std::min(first + (int64_t)kWave * chunk, nnz) - 1;
  const int fr = row_search_uniform(ro, 1u, (uint32_t)rows + 1u,
                                    (int32_t)first);
  const int lr = row_search_gallop(ro, (uint32_t)fr + 1u, (uint32_t)rows + 1u,
                                   (int32_t)last);
  return WaveRows{(uint32_t)fr + 1u, (uint32_t)lr + 2u};
}

// thread-per-position, atomic: worker w handles positions
// [w*chunk, min((w+1)*chunk, nnz)), recovers each position's row by the row
// search and adds val*x atomically (SparsePositionScheduling.cpp:135-194).
// The search runs inside the wave's row range (configuration 2: 2934 ->
// 2628 us; the atomic add per position is the rest).
__global__ __launch_bounds__(1024) void spmv_thread_position_atomic(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ x,
    float *__restrict__ y, int32_t rows, int32_t nnz, int32_t chunk) {
  const int64_t w = block_id() * blockDim.x + threadIdx.x;
  const int64_t b = w * chunk;
  if (((block_id() * blockDim.x + (int64_t)wave_in_group() * kWave) *
       chunk) >= nnz)
    return; // wave-uniform: the whole wave is past the positions
  const WaveRows wr = wave_rows(ro, rows, nnz, chunk);
  if (b >= nnz)
    return;
  const int64_t e = b + chunk < nnz ? b + chunk : nnz;
  for (int64_t p = b; p < e; ++p) {
    const int r = row_search_lane(ro, wr.lo, wr.hi, (int32_t)p);
    unsafeAtomicAdd(y + r, val[p] * x[col[p]]);
  }
}

// thread-per-position, segmented: the chunk's first row comes from the row
// search, later rows from walking the row offsets; a run of equal rows is
// summed locally and added atomically when the row changes
// (SparsePositionScheduling.cpp:196-316).
__global__ __launch_bounds__(1024) void spmv_thread_position_segmented(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ x,
    float *__restrict__ y, int32_t rows, int32_t nnz, int32_t chunk) {
  // (the chunk's own search over all row offsets: the wave-range form of
  // the atomic kernel measured 562 -> 596 us here, configuration 2, chunk 8)
  int64_t w = block_id() * blockDim.x + threadIdx.x;
  int64_t b = w * chunk;
  if (b >= nnz)
    return;
  int64_t e = b + chunk < nnz ? b + chunk : nnz;
  int r = row_search_lane(ro, 1u, (uint32_t)rows + 1u, (int32_t)b);
  int32_t next = ro[r + 1];
  float acc = val[b] * x[col[b]];
  for (int64_t p = b + 1; p < e; ++p) {
    int rr = r;
    while (p >= next) {
      ++rr;
      next = ro[rr + 1];
    }
    float c = val[p] * x[col[p]];
    if (rr == r) {
      acc += c;
    } else {
      unsafeAtomicAdd(y + r, acc);
      r = rr;
      acc = c;
    }
  }
  unsafeAtomicAdd(y + r, acc);
}

// ---------------------------------------------------------------------------
// wave-per-position, Wave64 design.
//
// Positions are grouped in units of P consecutive positions (P = 1 is the
// reference's one position per lane).  There are G = max(ceil(units/B), 1)
// blocks and G*(B/64) waves; wave w owns the balanced partition
// [w*base + min(w, rem), ...) of the units (SparsePositionToSCF.cpp:190-223)
// and lane l the unit begin+l.  The wave finds the rows of its first and last
// position with wave-uniform searches (scalar loads), each lane then finds the row of
// its first position inside that narrow range, walks its P positions
// (col/val read with 128-bit loads when P >= 4) and
//   - stores rows that start and end inside the lane directly,
//   - keeps the partial of its first row (head) and of its last row (tail).
// One segmented scan over the tails joins rows that continue across lanes;
// a lane whose first row continues from its left neighbour picks up that
// neighbour's scanned tail ("carry"), and every other row segment ends with
// one atomic add.  The output is zeroed first, as in the reference.
template <int P, bool VEC>
__global__ __launch_bounds__(1024) void spmv_wave_position(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ x,
    float *__restrict__ y, int32_t rows, int32_t nnz, int64_t units,
    int64_t wave_count) {
  const int lane = lane_id();
  const int64_t wave =
      block_id() * (blockDim.x / kWave) + wave_in_group();
  const uint64_t base = (uint64_t)units / (uint64_t)wave_count;
  const uint64_t rem = (uint64_t)units % (uint64_t)wave_count;
  const uint64_t wv = (uint64_t)wave;
  const uint64_t ub = wv * base + (wv < rem ? wv : rem);
  const uint64_t ue = ub + base + (wv < rem ? 1u : 0u);
  const int64_t wbeg = (int64_t)ub * P;
  const int64_t wend = (int64_t)ue * P < nnz ? (int64_t)ue * P : nnz;
  if (wbeg >= wend)
    return; // wave-uniform: the whole wave leaves

  const int64_t u = (int64_t)ub + lane;
  const bool active = (uint64_t)u < ue && u * P < nnz;
  const int32_t p0 = active ? (int32_t)(u * P) : 0;
  const int32_t pe = active ? (int32_t)((u * P + P) < nnz ? u * P + P : nnz) : 0;

  // Issue the lane's column/value loads and x gathers first; the row
  // searches below use scalar loads and overlap with them.  The products are
  // formed in the walk, so nothing waits on the gathers before the searches.
  float vv[P], xg[P];
#pragma unroll
  for (int q = 0; q < P; ++q) {
    vv[q] = 0.0f;
    xg[q] = 0.0f;
  }
  if (active) {
    bool full = false;
    if constexpr (VEC && P >= 4) {
      full = pe - p0 == P;
      if (full) {
#pragma unroll
        for (int q = 0; q < P; q += 4) {
          // values non-temporal, columns plain: the same speed as plain
          // loads for both (209.8 us on configuration 2 at P = 8) with 14%
          // less L2-to-fabric traffic (x stays in L2 longer: hit rate 82.5%
          // against 79.2%); non-temporal columns as well measured 218 us.
          // Both as a uniform base plus a 32-bit byte offset (VEC implies
          // 4 * nnz fits): 207.4 -> 206.9 us
          const uint32_t bo = 4u * (uint32_t)(p0 + q);
          v4i c = ld_stream(at_bytes(reinterpret_cast<const v4i *>(col), bo));
          v4f v =
              ld_nontemporal(at_bytes(reinterpret_cast<const v4f *>(val), bo));
          vv[q + 0] = v.x;
          vv[q + 1] = v.y;
          vv[q + 2] = v.z;
          vv[q + 3] = v.w;
          // the host takes VEC only when 4 * cols fits 32 bits
          xg[q + 0] = gather<true>(x, c.x);
          xg[q + 1] = gather<true>(x, c.y);
          xg[q + 2] = gather<true>(x, c.z);
          xg[q + 3] = gather<true>(x, c.w);
        }
      }
    }
    if (!full) {
#pragma unroll
      for (int q = 0; q < P; ++q)
        if (p0 + q < pe) {
          vv[q] = ld_stream(val + p0 + q);
          xg[q] = x[ld_stream(col + p0 + q)];
        }
    }
  }

  const int first_row =
      row_search_uniform(ro, 1u, (uint32_t)rows + 1u, (int32_t)wbeg);
  const int last_row = row_search_gallop(ro, (uint32_t)first_row + 1u,
                                         (uint32_t)rows + 1u,
                                         (int32_t)(wend - 1));

  // Row boundaries ro[first_row+1 .. first_row+64] staged in LDS (one
  // coalesced load per wave) serve the lanes' row lookups whenever the wave
  // spans at most 64 rows; otherwise lanes search the row offsets directly.
  __shared__ int32_t window[1024 / kWave][kWave];
  int32_t *win = window[wave_in_group()];
  const int span = last_row - first_row; // wave-uniform
  const bool use_win = span < kWave;
  if (use_win) {
    const int j = first_row + 1 + lane;
    win[lane] = j <= first_row + 1 + span ? ro[j] : INT32_MAX;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  int lrow = 0, row = 0, closed = 0;
  float head = 0.0f, acc = 0.0f;
  if (active) {
    int32_t next;
    if (use_win) {
      // count of window boundaries <= p0, over entries [0, span]
      int lo = 0, hi = span; // the answer lies in [0, span]
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
          if (closed == 0)
            head = acc;
          else
            y[row] = acc; // row began and ended inside this lane
          ++closed;
          acc = 0.0f;
          ++row;
          next = use_win ? win[row - first_row] : ro[row + 1];
        }
        acc = __builtin_fmaf(vv[q], xg[q], acc);
      }
    }
  }

  // segmented scan over the lanes' open tails
  const int key = active ? row : -1;
  const float scanned = wave_segmented_scan(key, active ? acc : 0.0f);
  const int prev_key = shfl_up1_i(key, INT32_MIN);
  const float prev_scanned = shfl_up1_f(scanned, 0.0f);
  const int next_lrow = shfl_down1_i(active ? lrow : -2, -2);
  // Segment emissions are fire-and-forget atomic adds into the zeroed
  // output.  Measured on configuration 2 (P = 4, 64-thread blocks, 206.7 us
  // as written): plain stores for the rows a wave holds whole with atomic
  // adds only for the two rows it may share, 402 us with the waves in
  // XCD-contiguous order (stores and atomics then meet in nearly every
  // 128-byte line of the output); all-atomic in that order 229 us.
  if (active) {
    if (closed > 0) {
      float h = head + (prev_key == lrow ? prev_scanned : 0.0f);
      unsafeAtomicAdd(y + lrow, h);
    }
    if (next_lrow != row)
      unsafeAtomicAdd(y + row, scanned);
  }
}

// The values and gathered x of one lane's P positions q0 .. q0 + P - 1 that
// lie in [lb_all, le_all) (zeros elsewhere); 128-bit column / value loads
// when the whole group lies inside the arrays.
template <int P, bool VEC>
__device__ __forceinline__ void owner_step_loads(
    const int32_t *__restrict__ col, const float *__restrict__ val,
    const float *__restrict__ x, int32_t q0, int32_t lb_all, int32_t le_all,
    int32_t nnz, float (&vv)[P], float (&xg)[P]) {
  const int32_t lb = std::max(q0, lb_all);
  const int32_t le = std::min(q0 + P, le_all);
#pragma unroll
  for (int q = 0; q < P; ++q) {
    vv[q] = 0.0f;
    xg[q] = 0.0f;
  }
  if (lb >= le)
    return;
  if constexpr (VEC && P >= 4) {
    if (q0 + P <= nnz) {
#pragma unroll
      for (int q = 0; q < P; q += 4) {
        const uint32_t bo = 4u * (uint32_t)(q0 + q);
        const v4i c =
            ld_stream(at_bytes(reinterpret_cast<const v4i *>(col), bo));
        const v4f v =
            ld_nontemporal(at_bytes(reinterpret_cast<const v4f *>(val), bo));
        const int32_t p = q0 + q;
        vv[q + 0] = v.x;
        vv[q + 1] = v.y;
        vv[q + 2] = v.z;
        vv[q + 3] = v.w;
        if (p + 0 >= lb && p + 0 < le) xg[q + 0] = gather<true>(x, c.x);
        if (p + 1 >= lb && p + 1 < le) xg[q + 1] = gather<true>(x, c.y);
        if (p + 2 >= lb && p + 2 < le) xg[q + 2] = gather<true>(x, c.z);
        if (p + 3 >= lb && p + 3 < le) xg[q + 3] = gather<true>(x, c.w);
      }
      return;
    }
  }
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const int32_t p = q0 + q;
    if (p >= lb && p < le) {
      vv[q] = ld_stream(val + p);
      xg[q] = x[ld_stream(col + p)];
    }
  }
}

// Rows r_lo .. r_hi - 1 of the SpMV by one wave: their positions
// [ro[r_lo], ro[r_hi]) in steps of 64 * P, lane l taking P consecutive
// positions; a lane finds the row of its first position in an LDS window
// of 64 row ends (win: the wave's 64-entry slice), walks its positions
// storing the rows that begin and end inside it, and the DPP segmented scan
// joins the rows that cross lanes; a row still open at the end of a step is
// carried, wave-uniform, into the next step's lane 0; rows with no entries
// are stored as zero by a pass over the rows.  Every row is stored once,
// by a plain store, with its sum formed in a fixed order.  Every lane of the
// wave calls it with the same rows.
template <int P, bool VEC>
__device__ __forceinline__ void owner_rows(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ x,
    float *__restrict__ y, int r_lo, int r_hi, int32_t nnz, int32_t *win) {
  const int lane = lane_id();
  if (r_lo >= r_hi)
    return; // no rows
  // positions of the owned rows, kept inside [0, nnz]
  const int32_t p_beg = std::min(std::max(ro[r_lo], 0), nnz);
  const int32_t p_end = std::min(std::max(ro[r_hi], p_beg), nnz);

  constexpr int32_t kStep = kWave * P;
  const int32_t a0 = VEC ? (p_beg & ~3) : p_beg;
  int r_cur = r_lo;          // row of the step's first position
  float carry = 0.0f;        // partial of r_cur from earlier steps
  for (int32_t s0 = a0; s0 < p_end; s0 += kStep) {
    const int32_t q0 = s0 + lane * P; // lane's first position
    const int32_t lb = std::max(q0, p_beg);
    const int32_t le = std::min(q0 + P, p_end);
    const bool active = lb < le;
    float va[P], xa[P];
    owner_step_loads<P, VEC>(col, val, x, q0, p_beg, p_end, nnz, va, xa);
    // row ends of rows r_cur .. r_cur + 63 (INT32_MAX past the wave's rows)
    const int jw = r_cur + 1 + lane;
    const int32_t wv = jw <= r_hi ? ro[jw] : INT32_MAX;
    win[lane] = wv;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int lrow = 0, row = 0, closed = 0;
    float head = 0.0f, acc = 0.0f;
    int32_t next = 0;
    if (active) {
      // number of window row ends <= lb; 64 means lb lies past the window
      int lo = 0, hi = kWave;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (win[mid] <= lb)
          lo = mid + 1;
        else
          hi = mid;
      }
      // (the minimum keeps rows inside the wave's range whatever the row
      // offsets hold; for a valid CSR operand it never binds)
      if (lo < kWave) {
        lrow = std::min(r_cur + lo, r_hi - 1);
        next = win[lrow - r_cur];
      } else {
        lrow = std::min(row_search_lane(ro, (uint32_t)r_cur + kWave + 1u,
                                        (uint32_t)r_hi + 1u, lb),
                        r_hi - 1);
        next = ro[lrow + 1];
      }
      row = lrow;
      // lane 0 of a later step continues the row carried from the last
      if (lane == 0)
        acc = carry;
#pragma unroll
      for (int q = 0; q < P; ++q) {
        const int32_t p = q0 + q;
        if (p >= lb && p < le) {
          while (p >= next && row < r_hi - 1) {
            if (closed == 0)
              head = acc;
            else
              y[row] = acc; // began and ended inside this lane
            ++closed;
            acc = 0.0f;
            ++row;
            next = row - r_cur < kWave ? win[row - r_cur] : ro[row + 1];
          }
          acc = __builtin_fmaf(va[q], xa[q], acc);
        }
      }
    }
    // every lane's window reads done before the next step rewrites it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int key = active ? row : -1;
    const float scanned = wave_segmented_scan(key, active ? acc : 0.0f);
    const int prev_key = shfl_up1_i(key, INT32_MIN);
    const float prev_scanned = shfl_up1_f(scanned, 0.0f);
    const int next_lrow = shfl_down1_i(active ? lrow : -2, -2);
    const int32_t step_end = std::min(s0 + kStep, p_end);
    if (active) {
      if (closed > 0)
        y[lrow] = head + (prev_key == lrow ? prev_scanned : 0.0f);
      // the tail row ends in this step unless it reaches past step_end
      if (next_lrow != row && next <= step_end)
        y[row] = scanned;
    }
    // a row open past the step end is held by lane 63 (the step is full)
    const int last_row = __builtin_amdgcn_readlane(row, kWave - 1);
    const int32_t last_next = __builtin_amdgcn_readlane(next, kWave - 1);
    const bool open = s0 + kStep < p_end && last_next > s0 + kStep;
    carry = open ? __int_as_float(__builtin_amdgcn_readlane(
                       __float_as_int(scanned), kWave - 1))
                 : 0.0f;
    // the next step's first row: lane 63's last row when that row is open,
    // else the row holding the next position (after it, usually right after)
    if (s0 + kStep < p_end)
      r_cur = open ? last_row
                   : std::min(row_search_gallop(ro, (uint32_t)last_row + 1u,
                                                (uint32_t)r_hi + 1u,
                                                s0 + kStep),
                              r_hi - 1);
  }
  // rows with no entries, which no position reaches, are zero (r_hi <= rows,
  // so ro[r + 1] exists)
  for (int r = r_lo + lane; r < r_hi; r += kWave)
    if (ro[r] == ro[r + 1])
      y[r] = 0.0f;
}

// ---------------------------------------------------------------------------
// wave-per-row-balanced: row-owner SpMV (Wave64 extension).
//
// The nonzeros are cut into chunks of C = 64 * P * S positions, and wave w
// owns the rows whose first position lies in chunk w (ro[r] in
// [wC, (w+1)C); rows beginning at or past the last chunk's start belong to
// the last wave).  So every output row has exactly one writer, which stores
// it with a plain store: no zero fill and no atomics, and the work stays
// balanced by nonzeros (a wave's rows hold C positions give or take the row
// that straddles each chunk end).  Waves run in XCD-contiguous order, so the
// short row ranges that neighbouring waves store share one XCD's L2.
//
// A wave finds its first row (a wave-uniform binary search) and the first
// row of the next chunk (a gallop from there), then walks its positions
// [ro[r_lo], ro[r_hi]) in steps of 64 * P: lane l takes P consecutive
// positions, finds the row of its first position in an LDS window of 64 row
// ends, and walks them as the position kernel does -- rows that begin and end
// inside the lane are stored directly, a lane's first and last rows are
// joined across lanes by the DPP segmented scan.  A row still open at the
// end of a step is carried, wave-uniform, into the next step's lane 0.
// Rows with no entries, which no position reaches, are stored as zero by a
// pass over the wave's rows.
//
// Every sum is formed in a fixed order (a lane's positions in sequence, the
// scan's fixed DPP steps, the carry), so repeated calls give bit-identical
// outputs, which the atomic position mappings do not.  It costs time: on
// configuration 2 (P = 4, S = 4) 235 us against the position kernel's
// 207 us; S = 1 248 us, S = 2 240 us; loading each step's values one step
// ahead measured no faster (237 us).  A wave's rows run to the end of the
// row that straddles its chunk end, so the few waves holding the start of a
// row of thousands of entries finish last.
template <int P, bool VEC>
__global__ __launch_bounds__(256) void spmv_row_owner(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ x,
    float *__restrict__ y, int32_t rows, int32_t nnz, int64_t chunk,
    int64_t waves) {
  const int64_t wave =
      xcd_contiguous(block_id(), grid_blocks()) * (blockDim.x / kWave) +
      wave_in_group();
  if (wave >= waves)
    return; // wave-uniform
  const int r_lo =
      wave == 0 ? 0
                : row_search_uniform(ro, 0u, (uint32_t)rows + 1u,
                                     (int32_t)(wave * chunk - 1)) + 1;
  const int r_hi =
      wave == waves - 1
          ? rows
          : row_search_gallop(ro, (uint32_t)r_lo, (uint32_t)rows + 1u,
                              (int32_t)((wave + 1) * chunk - 1)) + 1;
  __shared__ int32_t window[256 / kWave][kWave];
  owner_rows<P, VEC>(ro, col, val, x, y, r_lo, r_hi, nnz,
                     window[wave_in_group()]);
}

// ---------------------------------------------------------------------------
// thread-per-row with whole-wave workgroups: the reference's launch (one
// thread per row); a wave whose rows are very uneven takes its 64
// consecutive rows together through owner_rows -- the rows' positions
// spread evenly over the lanes, so a row of thousands of entries no longer
// holds its wave for hundreds of dependent steps.  Each row is stored once,
// its sum formed in a fixed order (in such waves not the reference's
// sequential order: within the fp32 bound).
template <int P, bool VEC, bool NARROW>
__global__ __launch_bounds__(1024) void spmv_thread_per_row_waves(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ x,
    float *__restrict__ y, int32_t rows, int32_t nnz) {
  const int64_t r0 = block_id() * blockDim.x +
                     (int64_t)wave_in_group() * kWave;
  if (r0 >= rows)
    return; // wave-uniform
  const int r_hi = (int)std::min<int64_t>(r0 + kWave, rows);
  // A wave whose longest row takes a thread at most kWalkFactor times the
  // steps of the shared walk (64 P positions a step) sums each row in its
  // own lane, as the reference does: the walk pays off only where one row
  // holds most of the wave's positions (longest row above 8x the wave's
  // mean at P = 4).  Factor 1 / 2 / 4: configuration 2 254.7 / 268.9 /
  // 301.7 us, the harness's skewed/32 matrix 21.3 / 9.3 / 9.2 us, skewed/256
  // 126.4 / 78.5 / 78.5 us, uniform rows (configuration 1, uniform/32,
  // uniform/256) no different; the walk always: uniform/256 138 us against
  // 50 us one row per lane.
  const int64_t r = r0 + lane_id();
  const int nt = r_hi - (int)r0; // rows of this wave, 1 .. 64
  const int32_t s = ro[r0 + std::min<int64_t>(lane_id(), nt - 1)];
  const int32_t e = r < rows ? ro[r + 1] : s;
  // the wave's positions from its first and last lanes, and one ballot:
  // does a row need more than kWalkFactor times the walk's steps?
  constexpr int kWalkFactor = 2;
  const int32_t total = __builtin_amdgcn_readlane(e, nt - 1) -
                        __builtin_amdgcn_readlane(s, 0);
  const int32_t steps = (total + kWave * P - 1) / (kWave * P);
  if (__builtin_amdgcn_ballot_w64(e - s > kThreadRowDeep * kWalkFactor *
                                              steps) == 0) {
    if (r < rows)
      y[r] = strided_dot<NARROW, kThreadRowDeep>(col, val, x, s, e, 1, 0.0f);
    return;
  }
  __shared__ int32_t window[1024 / kWave][kWave];
  owner_rows<P, VEC>(ro, col, val, x, y, (int)r0, r_hi, nnz,
                     window[wave_in_group()]);
}

// ---------------------------------------------------------------------------
// Gather floor (a diagnostic with no reference counterpart): the part of a
// CSR SpMV that no row schedule avoids -- every column index and value read
// once with 128-bit loads and every x[col] gathered once -- without the row
// structure.  Lane l of wave w owns positions [8u, 8u + 8), u = 64w + l, and
// each wave writes the sum of its products to partial[w].  Its time bounds
// any SpMV schedule that reads col/val and gathers x once per nonzero.
constexpr int kFloorUnit = 8;

__global__ __launch_bounds__(64) void spmv_gather_floor(
    const int32_t *__restrict__ col, const float *__restrict__ val,
    const float *__restrict__ x, float *__restrict__ partial, int64_t nnz,
    bool vec) {
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t p0 = u * kFloorUnit;
  float acc = 0.0f;
  if (vec && p0 + kFloorUnit <= nnz) {
#pragma unroll
    for (int q = 0; q < kFloorUnit; q += 4) {
      const v4i c = ld_stream(reinterpret_cast<const v4i *>(col + p0 + q));
      const v4f v = ld_stream(reinterpret_cast<const v4f *>(val + p0 + q));
      acc = __builtin_fmaf(v.x, x[c.x], acc);
      acc = __builtin_fmaf(v.y, x[c.y], acc);
      acc = __builtin_fmaf(v.z, x[c.z], acc);
      acc = __builtin_fmaf(v.w, x[c.w], acc);
    }
  } else {
    for (int64_t p = p0; p < p0 + kFloorUnit && p < nnz; ++p)
      acc = __builtin_fmaf(val[p], x[col[p]], acc);
  }
  acc = group_sum<kWave>(acc);
  if (threadIdx.x == 0)
    partial[blockIdx.x] = acc;
}

// ---------------------------------------------------------------------------
// batch row recovery (sw_csr_row_at_position)
__global__ __launch_bounds__(256) void csr_row_at_position_kernel(
    const int32_t *__restrict__ ro, int32_t rows,
    const int64_t *__restrict__ pos, int32_t *__restrict__ out,
    int64_t count) {
  int64_t i = block_id() * blockDim.x + threadIdx.x;
  if (i < count)
    out[i] = row_search_lane(ro, 1u, (uint32_t)rows + 1u, (int32_t)pos[i]);
}

// ---------------------------------------------------------------------------
// sparsewave.coo_spmv (SparseWaveOps.td:54-88): parallel row-index,
// column-index and value arrays, entries in any order, coordinates may
// repeat; the output is zeroed first, then accumulated.
//
// thread-per-nonzero: the reference's COO lowering
// (ThreadPerNonzeroCOOSpMVPattern, SparseWaveToGPU.cpp:154-214), one thread
// and one atomic add of val*x[col] per stored entry.
__global__ __launch_bounds__(1024) void coo_thread_per_nonzero(
    const int32_t *__restrict__ ri, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ x,
    float *__restrict__ y, int64_t nnz) {
  const int64_t p = block_id() * blockDim.x + threadIdx.x;
  if (p < nnz)
    unsafeAtomicAdd(y + ld_nontemporal(ri + p),
                    ld_nontemporal(val + p) * x[ld_nontemporal(col + p)]);
}

// Run-segmented COO (Wave64 extension, taken under the position mapping):
// grid lane u takes entries [u*P, u*P+P).  Runs of equal adjacent row
// indices are summed in registers; a run that closes inside the lane is added
// atomically; the lane's last run is carried across lanes by a segmented scan
// keyed on run numbers (a ballot prefix count of run starts, which is
// monotone even when row indices are not), so a row-sorted matrix costs about
// one atomic per row per wave instead of one per entry.  Unsorted input stays
// correct: a row split over several runs gets one atomic per run.
template <int P, bool VEC>
__global__ __launch_bounds__(1024) void coo_run_segmented(
    const int32_t *__restrict__ ri, const int32_t *__restrict__ col,
    const float *__restrict__ val, const float *__restrict__ x,
    float *__restrict__ y, int64_t nnz) {
  const int64_t u = block_id() * blockDim.x + threadIdx.x;
  const int64_t p0 = u * P;
  const bool active = p0 < nnz;
  const int n = active ? (int)(nnz - p0 < P ? nnz - p0 : P) : 0;
  int32_t rr[P];
  float prod[P];
#pragma unroll
  for (int q = 0; q < P; ++q) {
    rr[q] = 0;
    prod[q] = 0.0f;
  }
  bool full = false;
  if constexpr (VEC && P >= 4) {
    full = n == P;
    if (full) {
#pragma unroll
      for (int q = 0; q < P; q += 4) {
        // row and column indices plain, values non-temporal: 222 us on
        // configuration 2 as COO, against 233 us with all three
        // non-temporal and 247 us with all three plain
        v4i r = ld_stream(reinterpret_cast<const v4i *>(ri + p0 + q));
        v4i c = ld_stream(reinterpret_cast<const v4i *>(col + p0 + q));
        v4f v = ld_nontemporal(reinterpret_cast<const v4f *>(val + p0 + q));
        rr[q + 0] = r.x;
        rr[q + 1] = r.y;
        rr[q + 2] = r.z;
        rr[q + 3] = r.w;
        // the host takes VEC only when 4 * cols fits 32 bits
        prod[q + 0] = v.x * gather<true>(x, c.x);
        prod[q + 1] = v.y * gather<true>(x, c.y);
        prod[q + 2] = v.z * gather<true>(x, c.z);
        prod[q + 3] = v.w * gather<true>(x, c.w);
      }
    }
  }
  if (!full) {
#pragma unroll
    for (int q = 0; q < P; ++q)
      if (q < n) {
        rr[q] = ld_stream(ri + p0 + q);
        prod[q] = ld_nontemporal(val + p0 + q) * x[ld_stream(col + p0 + q)];
      }
  }
  int hk = -1, tk = -1, closed = 0;
  float head = 0.0f, acc = 0.0f;
  if (active) {
    hk = tk = rr[0];
#pragma unroll
    for (int q = 0; q < P; ++q)
      if (q < n) {
        if (rr[q] != tk) {
          if (closed == 0)
            head = acc;
          else
            unsafeAtomicAdd(y + tk, acc);
          ++closed;
          acc = 0.0f;
          tk = rr[q];
        }
        acc += prod[q];
      }
  }
  // A lane's last run continues the previous lane's last run exactly when
  // the lane holds a single run of the same row.
  const int prev_tk = shfl_up1_i(active ? tk : -1, -1);
  const bool starts = !(active && closed == 0 && tk == prev_tk);
  const uint64_t m = ballot(starts);
  const int run = (int)__builtin_amdgcn_mbcnt_hi(
                      (uint32_t)(m >> 32),
                      __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u)) +
                  (starts ? 1 : 0);
  const float scanned = wave_segmented_scan(run, active ? acc : 0.0f);
  const float prev_scanned = shfl_up1_f(scanned, 0.0f);
  const int next_hk = shfl_down1_i(active ? hk : -2, -2);
  if (active) {
    if (closed > 0)
      unsafeAtomicAdd(y + hk, head + (prev_tk == hk ? prev_scanned : 0.0f));
    if (next_hk != tk)
      unsafeAtomicAdd(y + tk, scanned);
  }
}

template <int P, bool VEC>
void launch_coo_runs(int64_t grid, int64_t B, hipStream_t st,
                     const int32_t *ri, const int32_t *col, const float *val,
                     const float *x, float *y, int64_t nnz) {
  hipLaunchKernelGGL((coo_run_segmented<P, VEC>), sw::grid_dim(grid, B),
                     dim3((unsigned)B), 0, st, ri, col, val, x, y, nnz);
}

template <int G>
void launch_group(dim3 grid, dim3 block, hipStream_t st, const int32_t *ro,
                  const int32_t *col, const float *val, const float *x,
                  float *y, int32_t rows, bool narrow) {
  if (narrow)
    hipLaunchKernelGGL((spmv_group_per_row<G, true>), grid, block, 0, st, ro,
                       col, val, x, y, rows);
  else
    hipLaunchKernelGGL((spmv_group_per_row<G, false>), grid, block, 0, st, ro,
                       col, val, x, y, rows);
}

template <int P, bool VEC>
void launch_row_owner(dim3 grid, dim3 block, hipStream_t st,
                      const int32_t *ro, const int32_t *col, const float *val,
                      const float *x, float *y, int32_t rows, int32_t nnz,
                      int64_t chunk, int64_t waves) {
  hipLaunchKernelGGL((spmv_row_owner<P, VEC>), grid, block, 0, st, ro, col,
                     val, x, y, rows, nnz, chunk, waves);
}

// Steps of 64 * P positions in one wave's chunk of the row-owner SpMV
// (configuration 2, P = 4: 1 step 248 us, 2 steps 240 us, 4 steps 235 us).
constexpr int64_t kRowOwnerSteps = 4;

template <int P, bool VEC>
void launch_wave_position(dim3 grid, dim3 block, hipStream_t st,
                          const int32_t *ro, const int32_t *col,
                          const float *val, const float *x, float *y,
                          int32_t rows, int32_t nnz, int64_t units,
                          int64_t waves) {
  hipLaunchKernelGGL((spmv_wave_position<P, VEC>), grid, block, 0, st, ro,
                     col, val, x, y, rows, nnz, units, waves);
}

} // namespace

namespace sw {

int launch_fill_zero(float *y, int64_t n, int64_t block, hipStream_t st) {
  if (n <= 0)
    return SW_OK;
  // a memory-bound fill: full 256-lane workgroups whatever the compute
  // kernel's block size (64-lane groups measured 5.2 us for 4 MB)
  block = std::max<int64_t>(block, 256);
  int64_t grid = ceil_div(ceil_div(n, 4), block);
  int rc = check_grid(grid, block, "output initialisation");
  if (rc)
    return rc;
  hipLaunchKernelGGL(fill_zero_f32, grid_dim(grid, block), dim3((unsigned)block),
                     0, st, y, n);
  return launch_check("output initialisation kernel");
}

int launch_position_init(const int32_t *ro, float *out, int64_t rows,
                         int64_t k, int64_t chunk, int64_t P, int64_t units,
                         int64_t waves, hipStream_t st) {
  if (rows <= 0 || k <= 0)
    return SW_OK;
  int64_t grid = ceil_div(rows, 256);
  int rc = check_grid(grid, 256, "output initialisation");
  if (rc)
    return rc;
  hipLaunchKernelGGL(position_init, grid_dim(grid, 256), dim3(256), 0, st,
                     ro, out, (int32_t)rows, k, chunk, P,
                     std::max<int64_t>(units, 1), std::max<int64_t>(waves, 1));
  return launch_check("position output initialisation kernel");
}

int launch_spmv(const int32_t *ro, const int32_t *col, const float *val,
                const float *x, float *y, int64_t rows, int64_t cols,
                int64_t nnz, const sw_options &o, hipStream_t st) {
  const int64_t B = o.spmv_block_size;
  const int32_t n = (int32_t)rows;
  const bool narrow = narrow_offsets(cols, 1);
  if (streq(o.spmv_mapping, "thread-per-row")) {
    int64_t grid = std::max<int64_t>(ceil_div(rows, B), 1);
    int rc = check_grid(grid, B, "thread-per-row SpMV");
    if (rc)
      return rc;
    dim3 g = grid_dim(grid, B), b((unsigned)B);
    // whole-wave workgroups: uneven waves take their 64 rows together
    // (configuration 2, 256-thread blocks: 438 -> 269 us)
    if (B % kWave == 0) {
      const bool vec = aligned16(col) && aligned16(val) && narrow &&
                       narrow_offsets(nnz, 1);
      if (vec)
        hipLaunchKernelGGL((spmv_thread_per_row_waves<4, true, true>), g, b,
                           0, st, ro, col, val, x, y, n, (int32_t)nnz);
      else if (narrow)
        hipLaunchKernelGGL((spmv_thread_per_row_waves<4, false, true>), g, b,
                           0, st, ro, col, val, x, y, n, (int32_t)nnz);
      else
        hipLaunchKernelGGL((spmv_thread_per_row_waves<4, false, false>), g, b,
                           0, st, ro, col, val, x, y, n, (int32_t)nnz);
      return launch_check("thread-per-row SpMV kernel");
    }
    if (narrow)
      hipLaunchKernelGGL(spmv_thread_per_row<true>, g, b, 0, st, ro, col, val,
                         x, y, n);
    else
      hipLaunchKernelGGL(spmv_thread_per_row<false>, g, b, 0, st, ro, col, val,
                         x, y, n);
    return launch_check("thread-per-row SpMV kernel");
  }
  if (streq(o.spmv_mapping, "wave-per-row")) {
    const int64_t G = o.spmv_lanes_per_row;
    int64_t grid = std::max<int64_t>(ceil_div(rows, B / G), 1);
    int rc = check_grid(grid, B, "wave-per-row SpMV");
    if (rc)
      return rc;
    dim3 g = grid_dim(grid, B), b((unsigned)B);
    switch (G) {
    case 1: launch_group<1>(g, b, st, ro, col, val, x, y, n, narrow); break;
    case 2: launch_group<2>(g, b, st, ro, col, val, x, y, n, narrow); break;
    case 4: launch_group<4>(g, b, st, ro, col, val, x, y, n, narrow); break;
    case 8: launch_group<8>(g, b, st, ro, col, val, x, y, n, narrow); break;
    case 16: launch_group<16>(g, b, st, ro, col, val, x, y, n, narrow); break;
    case 32: launch_group<32>(g, b, st, ro, col, val, x, y, n, narrow); break;
    default: launch_group<64>(g, b, st, ro, col, val, x, y, n, narrow); break;
    }
    return launch_check("wave-per-row SpMV kernel");
  }
  if (streq(o.spmv_mapping, "block-per-row")) {
    int64_t grid = std::max<int64_t>(rows, 1);
    int rc = check_grid(grid, B, "block-per-row SpMV");
    if (rc)
      return rc;
    dim3 g = grid_dim(grid, B), b((unsigned)B);
    if (narrow)
      hipLaunchKernelGGL(spmv_block_per_row<true>, g, b, 0, st, ro, col, val,
                         x, y, n);
    else
      hipLaunchKernelGGL(spmv_block_per_row<false>, g, b, 0, st, ro, col, val,
                         x, y, n);
    return launch_check("block-per-row SpMV kernel");
  }
  int rc;
  if (streq(o.spmv_mapping, "thread-per-position")) {
    // every contribution is atomic: zero the whole output first
    rc = launch_fill_zero(y, rows, o.spmv_block_size, st);
    if (rc)
      return rc;
    if (nnz == 0)
      return SW_OK;
    const int64_t chunk = o.spmv_position_chunk_size;
    int64_t workers = ceil_div(nnz, chunk);
    int64_t grid = std::max<int64_t>(ceil_div(workers, B), 1);
    rc = check_grid(grid, B, "thread-per-position SpMV");
    if (rc)
      return rc;
    if (streq(o.spmv_position_reduction, "segmented"))
      hipLaunchKernelGGL(spmv_thread_position_segmented, grid_dim(grid, B),
                         dim3((unsigned)B), 0, st, ro, col, val, x, y, n,
                         (int32_t)nnz, (int32_t)std::min<int64_t>(chunk, nnz));
    else
      hipLaunchKernelGGL(spmv_thread_position_atomic, grid_dim(grid, B),
                         dim3((unsigned)B), 0, st, ro, col, val, x, y, n,
                         (int32_t)nnz, (int32_t)std::min<int64_t>(chunk, nnz));
    return launch_check("thread-per-position SpMV kernel");
  }
  if (streq(o.spmv_mapping, "wave-per-row-balanced")) {
    if (nnz == 0) // every row is empty
      return launch_fill_zero(y, rows, B, st);
    const int64_t P = o.spmv_positions_per_lane;
    const int64_t chunk = kWave * P * kRowOwnerSteps;
    const int64_t waves = ceil_div(nnz, chunk);
    // the kernel is compiled for at most 256 threads per workgroup
    const int64_t OB = std::min<int64_t>(B, 256);
    const int64_t grid = ceil_div(waves, OB / kWave);
    rc = check_grid(grid, OB, "wave-per-row-balanced SpMV");
    if (rc)
      return rc;
    const bool vec = aligned16(col) && aligned16(val) && narrow &&
                     narrow_offsets(nnz, 1);
    dim3 g = grid_dim(grid, OB), b((unsigned)OB);
    const int32_t z = (int32_t)nnz;
    switch (P) {
    case 1: launch_row_owner<1, false>(g, b, st, ro, col, val, x, y, n, z, chunk, waves); break;
    case 2: launch_row_owner<2, false>(g, b, st, ro, col, val, x, y, n, z, chunk, waves); break;
    case 4:
      if (vec) launch_row_owner<4, true>(g, b, st, ro, col, val, x, y, n, z, chunk, waves);
      else launch_row_owner<4, false>(g, b, st, ro, col, val, x, y, n, z, chunk, waves);
      break;
    case 8:
      if (vec) launch_row_owner<8, true>(g, b, st, ro, col, val, x, y, n, z, chunk, waves);
      else launch_row_owner<8, false>(g, b, st, ro, col, val, x, y, n, z, chunk, waves);
      break;
    default:
      if (vec) launch_row_owner<16, true>(g, b, st, ro, col, val, x, y, n, z, chunk, waves);
      else launch_row_owner<16, false>(g, b, st, ro, col, val, x, y, n, z, chunk, waves);
      break;
    }
    return launch_check("wave-per-row-balanced SpMV kernel");
  }
  // wave-per-position
  const int64_t P = o.spmv_positions_per_lane;
  const int64_t units = ceil_div(nnz, P);
  const int64_t grid = std::max<int64_t>(ceil_div(units, B), 1);
  rc = check_grid(grid, B, "wave-per-position SpMV");
  if (rc)
    return rc;
  const int64_t waves = grid * (B / 64);
  rc = launch_fill_zero(y, rows, o.spmv_block_size, st);
  if (rc)
    return rc;
  if (nnz == 0)
    return SW_OK;
  const bool vec = aligned16(col) && aligned16(val) && narrow &&
                   narrow_offsets(nnz, 1);
  dim3 g = grid_dim(grid, B), b((unsigned)B);
  const int32_t z = (int32_t)nnz;
  switch (P) {
  case 1: launch_wave_position<1, false>(g, b, st, ro, col, val, x, y, n, z, units, waves); break;
  case 2: launch_wave_position<2, false>(g, b, st, ro, col, val, x, y, n, z, units, waves); break;
  case 4:
    if (vec) launch_wave_position<4, true>(g, b, st, ro, col, val, x, y, n, z, units, waves);
    else launch_wave_position<4, false>(g, b, st, ro, col, val, x, y, n, z, units, waves);
    break;
  case 8:
    if (vec) launch_wave_position<8, true>(g, b, st, ro, col, val, x, y, n, z, units, waves);
    else launch_wave_position<8, false>(g, b, st, ro, col, val, x, y, n, z, units, waves);
    break;
  default:
    if (vec) launch_wave_position<16, true>(g, b, st, ro, col, val, x, y, n, z, units, waves);
    else launch_wave_position<16, false>(g, b, st, ro, col, val, x, y, n, z, units, waves);
    break;
  }
  return launch_check("wave-per-position SpMV kernel");
}

int launch_spmv_coo(const int32_t *ri, const int32_t *col, const float *val,
                    const float *x, float *y, int64_t rows, int64_t cols,
                    int64_t nnz, const sw_options &o, hipStream_t st) {
  const int64_t B = o.spmv_block_size;
  int rc = launch_fill_zero(y, rows, B, st);
  if (rc || nnz == 0)
    return rc;
  if (streq(o.spmv_mapping, "wave-per-position")) {
    const int64_t P = o.spmv_positions_per_lane;
    const int64_t grid = std::max<int64_t>(ceil_div(ceil_div(nnz, P), B), 1);
    rc = check_grid(grid, B, "run-segmented COO SpMV");
    if (rc)
      return rc;
    const bool vec = aligned16(ri) && aligned16(col) && aligned16(val) &&
                     narrow_offsets(cols, 1);
    switch (P) {
    case 1: launch_coo_runs<1, false>(grid, B, st, ri, col, val, x, y, nnz); break;
    case 2: launch_coo_runs<2, false>(grid, B, st, ri, col, val, x, y, nnz); break;
    case 4:
      if (vec) launch_coo_runs<4, true>(grid, B, st, ri, col, val, x, y, nnz);
      else launch_coo_runs<4, false>(grid, B, st, ri, col, val, x, y, nnz);
      break;
    case 8:
      if (vec) launch_coo_runs<8, true>(grid, B, st, ri, col, val, x, y, nnz);
      else launch_coo_runs<8, false>(grid, B, st, ri, col, val, x, y, nnz);
      break;
    default:
      if (vec) launch_coo_runs<16, true>(grid, B, st, ri, col, val, x, y, nnz);
      else launch_coo_runs<16, false>(grid, B, st, ri, col, val, x, y, nnz);
      break;
    }
    return launch_check("run-segmented COO SpMV kernel");
  }
  const int64_t grid = std::max<int64_t>(ceil_div(nnz, B), 1);
  rc = check_grid(grid, B, "thread-per-nonzero COO SpMV");
  if (rc)
    return rc;
  hipLaunchKernelGGL(coo_thread_per_nonzero, grid_dim(grid, B),
                     dim3((unsigned)B), 0, st, ri, col, val, x, y, nnz);
  return launch_check("thread-per-nonzero COO SpMV kernel");
}

} // namespace sw

extern "C" int sw_spmv_csr_f32(const int32_t *row_offsets,
                               const int32_t *column_indices,
                               const float *values, const float *vector,
                               float *output, int64_t rows, int64_t cols,
                               int64_t nnz, const sw_options *opts,
                               void *stream) {
  sw::clear_error();
  sw_options o;
  int rc = sw::resolve_options(opts, &o);
  if (rc)
    return rc;
  rc = sw::check_csr(row_offsets, column_indices, values, rows, nnz, true);
  if (!rc)
    rc = sw::check_value_alignment(sizeof(float), {values, vector, output});
  if (rc)
    return rc;
  if (cols < 0)
    return sw::fail(SW_ERR_INVALID_SHAPE, "expected non-negative columns");
  if (rows == 0)
    return SW_OK;
  if (!output || (nnz > 0 && cols > 0 && !vector))
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "vector or output pointer is null");
  return sw::launch_spmv(row_offsets, column_indices, values, vector, output,
                         rows, cols, nnz, o, sw::as_stream(stream));
}

extern "C" int sw_spmv_gather_floor_f32(const int32_t *column_indices,
                                        const float *values,
                                        const float *vector, float *partial,
                                        int64_t nnz, void *stream) {
  sw::clear_error();
  if (nnz < 0)
    return sw::fail(SW_ERR_INVALID_SHAPE, "expected non-negative nnz");
  if (nnz == 0)
    return SW_OK;
  if (!column_indices || !values || !vector || !partial)
    return sw::fail(SW_ERR_INVALID_ARGUMENT,
                    "column index, value, vector or partial pointer is null");
  const int64_t grid = sw::ceil_div(sw::ceil_div(nnz, kFloorUnit), kWave);
  int rc = sw::check_flat_grid(grid, kWave, "gather floor");
  if (rc)
    return rc;
  const bool vec = sw::aligned16(column_indices) && sw::aligned16(values);
  hipLaunchKernelGGL(spmv_gather_floor, dim3((unsigned)grid), dim3(kWave), 0,
                     sw::as_stream(stream), column_indices, values, vector,
                     partial, nnz, vec);
  return sw::launch_check("gather floor kernel");
}

extern "C" int sw_spmv_coo_f32(const int32_t *row_indices,
                               const int32_t *column_indices,
                               const float *values, const float *vector,
                               float *output, int64_t rows, int64_t cols,
                               int64_t nnz, const sw_options *opts,
                               void *stream) {
  sw::clear_error();
  sw_options o;
  int rc = sw::resolve_options(opts, &o);
  if (rc)
    return rc;
  if (rows < 0 || cols < 0 || nnz < 0)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "expected non-negative rows, columns and nnz");
  if (rows > INT32_MAX)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "i32 COO row indices cannot address %lld rows",
                    (long long)rows);
  rc = sw::check_value_alignment(sizeof(float), {values, vector, output});
  if (rc)
    return rc;
  if (rows == 0)
    return SW_OK;
  if (!output)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "output pointer is null");
  if (nnz > 0 && (!row_indices || !column_indices || !values || !vector))
    return sw::fail(SW_ERR_INVALID_ARGUMENT,
                    "row index, column index, value or vector pointer is null");
  return sw::launch_spmv_coo(row_indices, column_indices, values, vector,
                             output, rows, cols, nnz, o,
                             sw::as_stream(stream));
}

extern "C" int sw_csr_row_at_position(const int32_t *row_offsets, int64_t rows,
                                      const int64_t *positions,
                                      int32_t *out_rows, int64_t count,
                                      void *stream) {
  sw::clear_error();
  if (rows < 0 || count < 0 || rows > INT32_MAX - 1)
    return sw::fail(SW_ERR_INVALID_SHAPE, "invalid rows or count");
  if (count == 0)
    return SW_OK;
  if (!row_offsets || !positions || !out_rows)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "null pointer");
  int64_t grid = sw::ceil_div(count, 256);
  int rc = sw::check_grid(grid, 256, "row recovery");
  if (rc)
    return rc;
  hipLaunchKernelGGL(csr_row_at_position_kernel, sw::grid_dim(grid, 256),
                     dim3(256), 0, sw::as_stream(stream), row_offsets,
                     (int32_t)rows, positions, out_rows, count);
  return sw::launch_check("row recovery kernel");
}
