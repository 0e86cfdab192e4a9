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
// result is rounded to bf16 once, as it is stored.  The next two chunks'
// rhs gathers and sample values are in flight over a chunk's products; each
// buffer is named (a buffer indexed by a run-time variable becomes indexed
// register moves behind a wait for every load).
//
// The structure check reads every column index of the tile once: each row
// against the last row's columns, which the wave stages in its LDS slice,
// 16 rows' 16-byte loads per batch, every load from a valid window.  A tile
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
using swd::v4i;
using swd::v4u;

constexpr int kTileCols = 512; // the last row's entries held in LDS
constexpr int kCheckRows = 32; // rows whose columns one check batch loads

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Rows r0 .. r0 + 63 (those below `rows`) of
//   out[p] = combine(sample[p] (0 without samples), lhs row . rhs col)
// with kdim = 64 KB; T is float or uint16_t (bf16 bits; lhs then 16-byte
// aligned); lcol is this wave's LDS slice of kTileCols entries.  Every lane
// of the wave calls it with the same r0.  The caller guarantees that
// sizeof(T) kdim cols fits 32 bits, and a tile whose positions end past
// 2^32 / 4 takes the rows' own path: every gather, sample load and store
// takes a wave-uniform base (scalar registers) and a 32-bit lane byte
// offset, the form the memory instructions take directly, so no lane
// computes a 64-bit address (with 64-bit addresses the address registers of
// three chunks in flight pushed the wave to reuse the registers of loads
// still in flight, a full wait every three chunks).  SAMPLES: sample is not null (a
// compile-time flag: a run-time test beside each sample load became a
// branch around it, which split the chunk's batch of loads: 78 -> 90 us
// on configuration 5's bundle).  WIDE: each row group's four samples of a
// lane as one element-aligned window (16 bytes fp32, 8 bytes bf16) instead
// of four loads (thread-per-row SDDMM in 256-thread workgroups, four tile
// waves per CU: 69.5 -> 64.7 us on configuration 5; the bundle's one wave
// per CU: 48.2 -> 50.4 us, so it keeps the four loads).
template <typename T, int KB, bool SAMPLES, bool WIDE, typename Combine>
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
  const int32_t rb = ro[rr], re = ro[rr + 1]; // one trip: no load is guarded
  const int32_t rlen = l < nt ? re - rb : 0;
  const int32_t bl = __builtin_amdgcn_readlane(rb, nt - 1);
  const int32_t len_last = __builtin_amdgcn_readlane(rlen, nt - 1);
  const int64_t te = (int64_t)bl + len_last; // the end of the tile's positions
  if (len_last > kTileCols ||
      (int64_t)bl + len_last > (int64_t)(UINT32_MAX / 4))
    return false;
  if (len_last == 0) {
    // an empty last row: a prefix tile only when every row is empty (and
    // bl may then be the arrays' end, so nothing is loaded)
    return __builtin_amdgcn_ballot_w64(rlen > 0) == 0;
  }
  {
    // entries past the last row's end repeat its final column, so that a
    // chunk's lanes read valid columns without a check; one batch of
    // clamped loads for all kTileCols slots (a loop up to the row's end
    // waited for each load before its store)
    {
      int32_t y[kTileCols / 64];
#pragma unroll
      for (int u = 0; u < kTileCols / 64; ++u) {
        const int t = l + 64 * u;
        y[u] = *swd::at_bytes(
            col, 4u * (uint32_t)(bl + (t < len_last ? t : len_last - 1)));
      }
#pragma unroll
      for (int u = 0; u < kTileCols / 64; ++u)
        lcol[l + 64 * u] = y[u];
    }
    wave_sync();
    // Every row but the last against the last row's columns, kCheckRows
    // rows per batch: lane l compares entries t = 4l .. 4l + 3 and
    // 256 + 4l .. + 3 of each row, read as two element-aligned 16-byte
    // loads (one wave per CU, as both callers launch it, keeps only its own
    // loads in flight: 4-byte loads, 8 rows per batch, made this check half
    // of the tile's time).  Every load is unconditional: the window of
    // entry t of a row starting at b is read from min(b + t, te - 4), te
    // the end of the tile's positions, so it lies inside the tile; entries
    // past a row's end read the next rows' columns and are compared with
    // nothing.  A window holding a compared entry is never moved: a row
    // before the last ends at or before the last row's start bl, so its
    // window starts at b + t < bl <= te - 4 when the last row holds at
    // least four entries (a tile whose last row holds fewer takes the rows'
    // own path).
    if (len_last < 4)
      return false;
    bool mine = rlen <= len_last;
    for (int i0 = 0; i0 < nt - 1; i0 += kCheckRows) {
      v4i x[kCheckRows][2];
#pragma unroll
      for (int j = 0; j < kCheckRows; ++j) {
        const int row = i0 + j < nt - 1 ? i0 + j : nt - 1;
        const int64_t b = __builtin_amdgcn_readlane(rb, row);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int64_t w = std::min<int64_t>(b + 4 * l + 256 * u, te - 4);
          __builtin_memcpy(&x[j][u], swd::at_bytes(col, 4u * (uint32_t)w),
                           sizeof(v4i));
        }
      }
      // the batch's loads stay together (the scheduler otherwise moves each
      // next to its compare, a wait between every few loads)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < kCheckRows; ++j) {
        const int row = i0 + j < nt - 1 ? i0 + j : nt - 1;
        const int32_t n = __builtin_amdgcn_readlane(rlen, row);
        const int32_t lim = n < len_last ? n : len_last; // wave-uniform
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int t = 4 * l + 256 * u;
          v4i ref;
          __builtin_memcpy(&ref, lcol + t, sizeof ref);
#pragma unroll
          for (int m = 0; m < 4; ++m)
            mine &= !(t + m < lim) || x[j][u][m] == ref[m];
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
  const __amdgpu_buffer_rsrc_t krs =
      swd::buffer_rsrc(rhs, (uint32_t)(sizeof(T) * kdim * cols));
  auto load = [&](int t0, Op (&a)[S], float (&mv)[4][4])
      __attribute__((always_inline)) {
    const uint32_t c = lcol[t0 + i];
    // buffer loads over rhs: the lane's rows (16 g, or 8 g in bf16) and
    // column c as its offset, rhs row 64 kb + st (32 st + e) as the
    // wave-uniform offset, so that one lane offset serves every step (as
    // global loads each step's row base took a 64-bit lane address)
    if constexpr (kF32) {
      const uint32_t ko = 4u * (16u * g * (uint32_t)cols + c);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int st = 0; st < 16; ++st)
          a[16 * kb + st] = swd::buffer_load_f32(
              krs, ko, 4u * (uint32_t)(64 * kb + st) * (uint32_t)cols);
    } else {
      const uint32_t ko = 2u * (8u * g * (uint32_t)cols + c);
#pragma unroll
      for (int st = 0; st < S; ++st) {
        uint32_t x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          x[e] = __builtin_amdgcn_raw_buffer_load_b16(
              krs, (int)ko, (int)(2u * (uint32_t)(32 * st + e) * (uint32_t)cols),
              0);
        a[st] = v4u{x[0] | (x[1] << 16), x[2] | (x[3] << 16),
                    x[4] | (x[5] << 16), x[6] | (x[7] << 16)};
      }
    }
    if constexpr (SAMPLES && WIDE) {
      // the window of entries t0 + 4g .. + 3 of row 16 R + i read from
      // min(e, te - 4), e its first position: only the last row's can move
      // (by d = 1..3; a row before the last ends at or before bl <= te - 4),
      // and then entry v sits in element v + d
#pragma unroll
      for (int R = 0; R < 4; ++R) {
        const uint32_t e = (uint32_t)(rbR[R] + t0 + 4 * g);
        const uint32_t w = std::min(e, (uint32_t)(te - 4));
        const uint32_t d = e - w;
        float x[4];
        if constexpr (kF32) {
          v4f y;
          __builtin_memcpy(&y, swd::at_bytes(sample, 4u * w), sizeof y);
          x[0] = y.x, x[1] = y.y, x[2] = y.z, x[3] = y.w;
        } else {
          v2u y;
          __builtin_memcpy(&y, swd::at_bytes(sample, 2u * w), sizeof y);
          x[0] = swd::tof((uint16_t)(y.x & 0xFFFFu));
          x[1] = swd::tof((uint16_t)(y.x >> 16));
          x[2] = swd::tof((uint16_t)(y.y & 0xFFFFu));
          x[3] = swd::tof((uint16_t)(y.y >> 16));
        }
        mv[R][0] = d == 0 ? x[0] : d == 1 ? x[1] : d == 2 ? x[2] : x[3];
        mv[R][1] = d == 0 ? x[1] : d == 1 ? x[2] : x[3];
        mv[R][2] = d == 0 ? x[2] : x[3];
        mv[R][3] = x[3];
      }
    } else {
#pragma unroll
      for (int R = 0; R < 4; ++R)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int t = t0 + 4 * g + v;
          const int32_t p = lenR[R] > 0
                                ? rbR[R] + (t < lenR[R] ? t : lenR[R] - 1)
                                : bl;
          mv[R][v] = SAMPLES ? swd::tof(*swd::at_bytes(
                                   sample, (uint32_t)(sizeof(T) * p)))
                             : 0.0f;
        }
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
      T *dst = swd::at_bytes(out, (uint32_t)(sizeof(T) * (rbR[R] + t)));
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
  // three chunks in flight, each buffer named: the loads of chunks j + 1
  // and j + 2 fly over chunk j's products.  Every chunk's loads are issued
  // unconditionally -- those of the (at most two) chunks past the last
  // repeat the last chunk's -- so that the compiler's wait before a chunk's
  // products counts the later chunks' loads as outstanding; a load inside a
  // branch made it wait for them too.
  const int nch = (len_last + 15) >> 4; // >= 1
  auto t_of = [&](int j) __attribute__((always_inline)) {
    return 16 * (j < nch ? j : nch - 1);
  };
  Op a0[S], a1[S], a2[S];
  float m0[4][4], m1[4][4], m2[4][4];
  load(t_of(0), a0, m0);
  load(t_of(1), a1, m1);
  for (int j = 0;; j += 3) {
    load(t_of(j + 2), a2, m2);
    compute(16 * j, a0, m0);
    if (j + 1 >= nch)
      break;
    load(t_of(j + 3), a0, m0);
    compute(16 * (j + 1), a1, m1);
    if (j + 2 >= nch)
      break;
    load(t_of(j + 4), a1, m1);
    compute(16 * (j + 2), a2, m2);
    if (j + 3 >= nch)
      break;
  }
  return true;
}

} // namespace sw_tile64
