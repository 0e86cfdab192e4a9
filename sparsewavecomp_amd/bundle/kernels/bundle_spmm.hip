// Fixed-shape SpMM entry point for an lrrt bundle (gfx950, Wave64).
//
// Bare-pointer kernel ABI in sparsewave.spmm operand order
// (rowOffsets, columnIndices, values, rhs, output: five 8-byte global
// pointers, kernarg 40 bytes; tools/sparsewave-bundle/sparsewave_bundle_ir.py:11-17
// in the reference), shapes baked in at compile time:
//   SW_ROWS  output rows (= launch n)
//   SW_K     rhs / output columns (= the tile size: one tile per row)
// Mapping wave-per-row-tile with 64-thread blocks: the runtime launches
// ceil_div(n, 64/64) * 64 work-items, so block b is row b.  Lanes stride the
// row's positions (four in flight per step), each reads the value once and
// SW_K rhs columns (128-bit loads when SW_K is a multiple of 4), the 64
// partial sums of every column meet in a DPP/swizzle butterfly and lane 0
// stores the row.
#include "../../csrc/sw_device.h"

#ifndef SW_ROWS
#error "SW_ROWS must be defined"
#endif
#ifndef SW_K
#error "SW_K must be defined"
#endif

using namespace swd;

extern "C" __global__ __launch_bounds__(64) void sparsewave_spmm_wave_per_row_tile(
    const int32_t *__restrict__ rowOffsets,
    const int32_t *__restrict__ columnIndices,
    const float *__restrict__ values, const float *__restrict__ rhs,
    float *__restrict__ output) {
  constexpr int K = SW_K;
  const int row = blockIdx.x;
  if (row >= SW_ROWS)
    return;
  const int l = __builtin_amdgcn_workitem_id_x();
  float acc[K];
#pragma unroll
  for (int c = 0; c < K; ++c)
    acc[c] = 0.0f;
  const int32_t s = rowOffsets[row], e = rowOffsets[row + 1];
  // one position's value and rhs row, added to the lane's partials
  auto add = [&](float v, const float *b) __attribute__((always_inline)) {
    if constexpr (K % 4 == 0) {
#pragma unroll
      for (int c = 0; c < K; c += 4) {
        const v4f b4 = *reinterpret_cast<const v4f *>(b + c);
        acc[c] = __builtin_fmaf(v, b4.x, acc[c]);
        acc[c + 1] = __builtin_fmaf(v, b4.y, acc[c + 1]);
        acc[c + 2] = __builtin_fmaf(v, b4.z, acc[c + 2]);
        acc[c + 3] = __builtin_fmaf(v, b4.w, acc[c + 3]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < K; ++c)
        acc[c] = __builtin_fmaf(v, b[c], acc[c]);
    }
  };
  // four of the lane's positions in flight per step, added in order
  constexpr int U = 4;
  int32_t p = s + l;
  for (; p + (U - 1) * kWave < e; p += U * kWave) {
    float v[U];
    const float *b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      v[u] = ld_stream(values + p + u * kWave);
      b[u] = rhs + (int64_t)ld_stream(columnIndices + p + u * kWave) * K;
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      add(v[u], b[u]);
  }
  for (; p < e; p += kWave)
    add(ld_stream(values + p),
        rhs + (int64_t)ld_stream(columnIndices + p) * K);
#pragma unroll
  for (int c = 0; c < K; ++c)
    acc[c] = group_sum<kWave>(acc[c]);
  if (l == 0) {
#pragma unroll
    for (int c = 0; c < K; ++c)
      output[(int64_t)row * K + c] = acc[c];
  }
}
