// A wave's 64 consecutive rows of an SDDMM as one matrix-core tile (fp32, or
// bf16 elements with fp32 arithmetic).
//
// Shared by the library's thread-per-row SDDMM (sw_attention.hip: one
// work-item per row, so each wave holds 64 consecutive rows) and the lrrt
// attention bundle's scores kernel (bundle/kernels/bundle_attention.hip,
// whose manifest fixes the same launch).  When every row's column list is
// a prefix of the tile's last row's -- true for block masks, causal
// diagonal blocks included, whose blocks line up with the 64-row tiles --
// the tile's entries are the dense products of its lhs rows with the rhs
// columns of the last row's entries, 16 entries (a chunk) at a time:
//   S^T = K_chunk Q^T with v_mfma_f32_16x16x4_f32 (fp32) or
//   v_mfma_f32_16x16x32_bf16 (bf16: lane group g supplies K elements
//   32 s + 8 g .. 32 s + 8 g + 7 of step s in both operands),
// the gathered rhs columns as the A operand and four 16-row lhs tiles as B
// operands, so that lane (i, g) holds row 16 R + i's dot products at
// entries t0 + 4g .. t0 + 4g + 3 (both products leave that layout).  A bf16
// result is rounded to bf16 once, as it is stored.  The next chunk's rhs
// gathers and sample values are in flight over a chunk's products; each
// buffer is named (a buffer indexed by a run-time variable becomes indexed
// register moves behind a wait for every load).
//
// The structure check reads every column index of the tile once: each row
// against the last row's columns, which the wave stages in its LDS slice,
// 8 rows' loads per batch, every load from a clamped valid position.  A tile
// that fails it, or whose last row has more than kTileCols entries, stores
// nothing and the function returns false; the caller computes those rows
// another way.  Sums are formed by the matrix cores (the dot's order
// differs from a sequential loop's, within the fp32 bound).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "sw_device.h"

namespace sw_tile64 {

using swd::v2u;
using swd::v4f;
using swd::v4u;

constexpr int kTileCols = 512; // the last row's entries held in LDS
constexpr int kCheckRows = 8;  // rows whose columns one check batch loads

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Rows r0 .. r0 + 63 (those below `rows`) of
//   out[p] = combine(sample[p] (0 without samples), lhs row . rhs col)
// with kdim = 64 KB; T is float or uint16_t (bf16 bits; lhs then 16-byte
// aligned); lcol is this wave's LDS slice of kTileCols entries.  Every lane
// of the wave calls it with the same r0.  SAMPLES: sample is not null (a
// compile-time flag: a run-time test beside each sample load became a
// branch around it, which split the chunk's batch of loads: 78 -> 90 us
// on configuration 5's bundle).
template <typename T, int KB, bool SAMPLES, typename Combine>
__device__ __forceinline__ bool sddmm_tile64(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col,
    const T *sample, const T *__restrict__ lhs, const T *__restrict__ rhs,
    T *out, int64_t rows, int64_t cols, int64_t r0, int32_t *lcol,
    Combine combine) {
  constexpr bool kF32 = std::is_same_v<T, float>;
  static_assert(kF32 || std::is_same_v<T, uint16_t>, "fp32 or bf16 bits");
  constexpr int kdim = 64 * KB;
  // MFMA steps per chunk and the operand registers of one step
  constexpr int S = kF32 ? 16 * KB : 2 * KB;
  using Op = std::conditional_t<kF32, float, v4u>;
  const int l = __lane_id();
  const int i = l & 15, g = l >> 4;
  const int nt = rows - r0 < 64 ? (int)(rows - r0) : 64; // >= 1
  const int64_t rr = r0 + (l < nt ? l : nt - 1);
  const int32_t rb = ro[rr];
  const int32_t rlen = l < nt ? ro[rr + 1] - rb : 0;
  const int32_t bl = __builtin_amdgcn_readlane(rb, nt - 1);
  const int32_t len_last = __builtin_amdgcn_readlane(rlen, nt - 1);
  if (len_last > kTileCols)
    return false;
  if (len_last == 0) {
    // an empty last row: a prefix tile only when every row is empty (and
    // bl may then be the arrays' end, so nothing is loaded)
    return __builtin_amdgcn_ballot_w64(rlen > 0) == 0;
  }
  {
    // entries past the last row's end repeat its final column, so that a
    // chunk's lanes read valid columns without a check
    const int span = (len_last + 15) & ~15;
    for (int t = l; t < span; t += 64)
      lcol[t] = col[bl + (t < len_last ? t : len_last - 1)];
    wave_sync();
    // every load unconditional, from a clamped valid position (a row's last
    // entry, or the last row's first for an empty row), so that no branch
    // splits a batch; the compare then selects the entries in range
    bool mine = rlen <= len_last;
    for (int i0 = 0; i0 < nt; i0 += kCheckRows) {
      int32_t x[kCheckRows][kTileCols / 64];
#pragma unroll
      for (int j = 0; j < kCheckRows; ++j) {
        const int row = i0 + j < nt ? i0 + j : nt - 1;
        const int32_t b = __builtin_amdgcn_readlane(rb, row);
        const int32_t n = __builtin_amdgcn_readlane(rlen, row);
#pragma unroll
        for (int u = 0; u < kTileCols / 64; ++u) {
          const int t = l + 64 * u;
          x[j][u] = col[n > 0 ? b + (t < n ? t : n - 1) : bl];
        }
      }
#pragma unroll
      for (int j = 0; j < kCheckRows; ++j) {
        const int row = i0 + j < nt ? i0 + j : nt - 1;
        const int32_t n = __builtin_amdgcn_readlane(rlen, row);
#pragma unroll
        for (int u = 0; u < kTileCols / 64; ++u) {
          const int t = l + 64 * u;
          mine &= !(t < n && t < len_last) || x[j][u] == lcol[t];
        }
      }
    }
    if (__builtin_amdgcn_ballot_w64(!mine) != 0)
      return false;
  }
  // row 16 R + i's first position and length, each 16-row tile's longest
  // row, and its lhs rows (B operand of step st: elements 64 kb + 16 g + st
  // in fp32, elements 32 st + 8 g .. + 7 in bf16)
  int32_t rbR[4], lenR[4], maxR[4];
  Op qb[4][S];
#pragma unroll
  for (int R = 0; R < 4; ++R) {
    const int src = 16 * R + i;
    rbR[R] = __builtin_amdgcn_ds_bpermute(src << 2, rb);
    lenR[R] = __builtin_amdgcn_ds_bpermute(src << 2, rlen);
    int m = lenR[R];
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int other = __builtin_amdgcn_ds_bpermute((l ^ o) << 2, m);
      m = other > m ? other : m;
    }
    maxR[R] = __builtin_amdgcn_readlane(m, 16 * R);
    const int64_t qr = r0 + src < rows ? r0 + src : rows - 1;
    if constexpr (kF32) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          v4f v;
          __builtin_memcpy(&v, lhs + qr * kdim + 64 * kb + 16 * g + 4 * u,
                           sizeof v);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            qb[R][16 * kb + 4 * u + e] = v[e];
        }
    } else {
#pragma unroll
      for (int st = 0; st < S; ++st)
        qb[R][st] = *reinterpret_cast<const v4u *>(lhs + qr * kdim +
                                                   32 * st + 8 * g);
    }
  }
  // one chunk's rhs gathers (A operand of step st: rhs[64 kb + 16 g + st]
  // at the column of entry t0 + i in fp32; rhs[32 st + 8 g + e], e = 0..7,
  // as four bf16 pairs in bf16) and the samples of the entries its lanes
  // store, each from a clamped valid position (selected afterwards)
  auto load = [&](int t0, Op (&a)[S], float (&mv)[4][4])
      __attribute__((always_inline)) {
    const int64_t c = lcol[t0 + i];
    if constexpr (kF32) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int st = 0; st < 16; ++st)
          a[16 * kb + st] = rhs[(int64_t)(64 * kb + 16 * g + st) * cols + c];
    } else {
#pragma unroll
      for (int st = 0; st < S; ++st) {
        uint32_t x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          x[e] = rhs[(int64_t)(32 * st + 8 * g + e) * cols + c];
        a[st] = v4u{x[0] | (x[1] << 16), x[2] | (x[3] << 16),
                    x[4] | (x[5] << 16), x[6] | (x[7] << 16)};
      }
    }
#pragma unroll
    for (int R = 0; R < 4; ++R)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int t = t0 + 4 * g + v;
        const int32_t p = lenR[R] > 0
                              ? rbR[R] + (t < lenR[R] ? t : lenR[R] - 1)
                              : bl;
        mv[R][v] = SAMPLES ? swd::tof(sample[p]) : 0.0f;
      }
  };
  // a chunk's products and its entries' stores (one 16-byte store when the
  // lane's four entries are all in its row)
  auto compute = [&](int t0, const Op (&a)[S], const float (&mv)[4][4])
      __attribute__((always_inline)) {
#pragma unroll
    for (int R = 0; R < 4; ++R) {
      if (t0 >= maxR[R]) // wave-uniform
        continue;
      v4f acc;
      if constexpr (kF32) {
        // two independent chains of products (even and odd steps)
        v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < S; st += 2) {
          acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[st], qb[R][st], acc0,
                                                      0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(
              a[st + 1], qb[R][st + 1], acc1, 0, 0, 0);
        }
        acc = acc0 + acc1;
      } else {
        acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < S; ++st)
          acc = swd::mfma_16x16x32_bf16(a[st], qb[R][st], acc);
      }
      v4f sc;
#pragma unroll
      for (int v = 0; v < 4; ++v)
        sc[v] = combine(mv[R][v], acc[v]);
      const int t = t0 + 4 * g;
      T *dst = out + rbR[R] + t;
      if (t + 3 < lenR[R]) {
        if constexpr (kF32) {
          __builtin_memcpy(dst, &sc, sizeof sc);
        } else {
          const v2u pr = {swd::pack_bf16x2(sc[0], sc[1]),
                          swd::pack_bf16x2(sc[2], sc[3])};
          __builtin_memcpy(dst, &pr, sizeof pr);
        }
      } else {
#pragma unroll
        for (int v = 0; v < 3; ++v)
          if (t + v < lenR[R])
            swd::stv(dst + v, sc[v]);
      }
    }
  };
  // chunks in pairs, each buffer named: the next chunk's loads fly over a
  // chunk's products
  Op a0[S], a1[S];
  float m0[4][4], m1[4][4];
  load(0, a0, m0);
  for (int t0 = 0; t0 < len_last; t0 += 32) {
    if (t0 + 16 < len_last)
      load(t0 + 16, a1, m1);
    compute(t0, a0, m0);
    if (t0 + 16 >= len_last)
      break;
    if (t0 + 32 < len_last)
      load(t0 + 32, a0, m0);
    compute(t0 + 16, a1, m1);
  }
  return true;
}

} // namespace sw_tile64
