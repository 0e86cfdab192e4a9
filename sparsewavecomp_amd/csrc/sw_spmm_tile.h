// The wave-per-row-tile SpMM work unit, shared by the library's kernel
// (sw_spmm.hip, spmm_row_tile) and the lrrt bundle's fixed-shape entry point
// (bundle/kernels/bundle_spmm.hip), so that a bundle runs the library's
// code.  Kernel of WavePerRowTileSpMMPattern, SparseWaveToGPU.cpp:1057-1256
// in the reference.
#pragma once

#include "sw_device.h"

namespace swd {

// A group of G lanes owns one (row, tile) work unit; G = 64 is the
// reference's wave per row tile, smaller G packs 64/G units into a wave for
// short rows.  Inside the group, CL "column lanes" each own V consecutive
// output columns of the tile (V = 4 uses 128-bit RHS loads) and PL = G/CL
// "position lanes" stride the row.  Each position lane reads val[p] and
// col[p] once and reuses them for all of its columns; the partial sums are
// reduced across the PL position lanes with xor shuffles, and the first
// position lane stores its V outputs (one contiguous T-column store per
// group).  Full and tail tiles share the code; tail columns are masked.
// positions per lane in flight in the row-tile loop (4: K=4 490 us, K=64
// 1377 us; 8: 494 us and 1456 us on configuration 3)
constexpr int kTileUnroll = 4;

// One group's (row, tile) unit `unit`; gl is the lane's index in its group.
// Every lane of the wave must call it (the reduction crosses the group).
template <int V, int CL, int G, typename T>
__device__ __forceinline__ void spmm_row_tile_unit(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const T *__restrict__ val, const T *__restrict__ rhs,
    T *__restrict__ out, int64_t rows, int64_t k, int32_t tile,
    int64_t tiles_per_row, int64_t unit, int gl) {
  constexpr int PL = G / CL;
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
      int32_t p = s + pl;
      // kTileUnroll positions per lane in flight: their loads and rhs
      // gathers are issued before the first product (rows longer than the
      // group carry most of the nonzeros of a skewed matrix)
      for (; p + (kTileUnroll - 1) * PL < e; p += kTileUnroll * PL) {
        float v[kTileUnroll];
        int64_t c[kTileUnroll];
#pragma unroll
        for (int u = 0; u < kTileUnroll; ++u) {
          v[u] = tof(ld_stream(val + p + u * PL));
          c[u] = ld_stream(col + p + u * PL);
        }
        v4f b[kTileUnroll];
#pragma unroll
        for (int u = 0; u < kTileUnroll; ++u)
          b[u] = ld4(rhs + c[u] * k + cb);
#pragma unroll
        for (int u = 0; u < kTileUnroll; ++u) {
          acc[0] = __builtin_fmaf(v[u], b[u].x, acc[0]);
          if constexpr (V == 4) {
            acc[1] = __builtin_fmaf(v[u], b[u].y, acc[1]);
            acc[2] = __builtin_fmaf(v[u], b[u].z, acc[2]);
            acc[3] = __builtin_fmaf(v[u], b[u].w, acc[3]);
          }
        }
      }
      for (; p < e; p += PL) {
        const float v = tof(ld_stream(val + p));
        const int64_t c = ld_stream(col + p);
        const v4f b = ld4(rhs + c * k + cb);
        acc[0] = __builtin_fmaf(v, b.x, acc[0]);
        if constexpr (V == 4) {
          acc[1] = __builtin_fmaf(v, b.y, acc[1]);
          acc[2] = __builtin_fmaf(v, b.z, acc[2]);
          acc[3] = __builtin_fmaf(v, b.w, acc[3]);
        }
      }
    } else {
      for (int32_t p = s + pl; p < e; p += PL) {
        const float v = tof(ld_stream(val + p));
        const int64_t c = ld_stream(col + p);
        const T *b = rhs + c * k + cb;
#pragma unroll
        for (int i = 0; i < V; ++i)
          if (cb + i < cend)
            acc[i] = __builtin_fmaf(v, ldv(b + i), acc[i]);
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
    T *o = out + r * k + cb;
    // non-temporal: the output is not re-read and should not displace RHS
    // rows from L2
    if (V == 4 && cb + 4 <= cend) {
      st4_nt(o, v4f{acc[0], acc[V > 1 ? 1 : 0], acc[V > 2 ? 2 : 0],
                    acc[V > 3 ? 3 : 0]});
    } else {
#pragma unroll
      for (int i = 0; i < V; ++i)
        if (cb + i < cend)
          st1_nt(o + i, acc[i]);
    }
  }
}

} // namespace swd
