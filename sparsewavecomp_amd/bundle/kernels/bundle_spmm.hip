// Fixed-shape SpMM entry point for an lrrt bundle (gfx950, Wave64).
//
// Bare-pointer kernel ABI in sparsewave.spmm operand order
// (rowOffsets, columnIndices, values, rhs, output: five 8-byte global
// pointers, kernarg 40 bytes; tools/sparsewave-bundle/sparsewave_bundle_ir.py:11-17
// in the reference), shapes baked in at compile time:
//   SW_ROWS  output rows (= launch n)
//   SW_K     rhs / output columns (= the tile size: one tile per row)
// Mapping wave-per-row-tile with 64-thread blocks: the runtime launches
// ceil_div(n, 64/64) * 64 work-items, one wave per output row.  Each wave
// runs the library's row-tile unit (sw_spmm_tile.h, the code behind
// sw_spmm_csr_f32 with spmm-mapping=wave-per-row-tile): rows in
// XCD-contiguous order, four positions per lane in flight, 128-bit RHS loads
// and a non-temporal 128-bit output store when K is a multiple of 4 and the
// rhs and output are 16-byte aligned (checked per launch, wave-uniform).
#include "../../csrc/sw_spmm_tile.h"

#ifndef SW_ROWS
#error "SW_ROWS must be defined"
#endif
#ifndef SW_K
#error "SW_K must be defined"
#endif

using namespace swd;

namespace {

constexpr int next_pow2_k(int v) {
  int p = 1;
  while (p < v)
    p <<= 1;
  return p;
}

constexpr int kVecCL = next_pow2_k((SW_K + 3) / 4); // column lanes, V = 4
constexpr int kScalarCL = next_pow2_k(SW_K);       // column lanes, V = 1

} // namespace

extern "C" __global__ __launch_bounds__(64) void sparsewave_spmm_wave_per_row_tile(
    const int32_t *__restrict__ rowOffsets,
    const int32_t *__restrict__ columnIndices,
    const float *__restrict__ values, const float *__restrict__ rhs,
    float *__restrict__ output) {
  // the grid is SW_ROWS blocks (launch n = rows); gridDim is not used, since
  // reading it would add hidden kernel arguments the 40-byte ABI lacks
  const int64_t unit = xcd_contiguous(blockIdx.x, SW_ROWS);
  const int gl = __builtin_amdgcn_workitem_id_x();
  const bool vec = SW_K % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(rhs) |
                     reinterpret_cast<uintptr_t>(output)) & 15u) == 0;
  if (vec)
    spmm_row_tile_unit<4, kVecCL, 64, float>(rowOffsets, columnIndices,
                                             values, rhs, output, SW_ROWS,
                                             SW_K, SW_K, 1, unit, gl);
  else
    spmm_row_tile_unit<1, kScalarCL, 64, float>(rowOffsets, columnIndices,
                                                values, rhs, output, SW_ROWS,
                                                SW_K, SW_K, 1, unit, gl);
}
