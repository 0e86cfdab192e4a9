// sparsewave.bsr_spmm on gfx950 behind sw_bsr_spmm_f32 / sw_bsr_spmm_bf16.
//
// Reference kernel: ThreadPerOutputBSRSpMMPattern
// (lib/Dialect/SparseWave/Transforms/SparseWaveToGPU.cpp:560-665), blocks
// row-major [nnzb][b][b] (SparseWaveOps.td:133-137), shape rules of the
// verifier (lib/Dialect/SparseWave/IR/SparseWaveOps.cpp:144-207, 340-372).
//
// The MI355X path for 16 x 16 blocks runs each block product on the matrix
// cores, accumulating in fp32 registers across the block row's blocks:
//   fp32, k % 4 == 0: a wave owns a 16 x 64 output strip (four tiles with
//     interleaved columns, 128-bit RHS loads and output stores) and issues
//     v_mfma_f32_16x16x4_f32 four times per block and tile;
//   bf16 with a bf16 output, k % 8 == 0: a wave owns a 16 x 128 output strip
//     (eight tiles with interleaved columns, 128-bit RHS loads) and issues
//     v_mfma_f32_16x16x16_bf16 once per block and tile;
//   otherwise a workgroup of four waves owns one block row and 128 output
//     columns, each wave two 16 x 16 tiles, issuing
//     fp32: v_mfma_f32_16x16x4_f32 four times per block and tile,
//     bf16: v_mfma_f32_16x16x16_bf16 once per block and tile.
#include "sw_device.h"
#include "sw_internal.h"

#include <algorithm>

using namespace swd;

namespace {

// thread-per-output for any block size: one thread per output element,
// the products added in block and column order.  BS = 16: the block size
// known, a block's 16 values and rhs rows requested together.  ROW (k and
// the workgroup size multiples of 64): a wave's outputs lie in one row, whose
// index is put in a scalar register, so that the block values and column
// indices are scalar loads shared by the wave.
template <typename T, typename TO, int BS, bool ROW>
__global__ __launch_bounds__(1024) void bsr_thread_per_output(
    const int32_t *__restrict__ bro, const int32_t *__restrict__ bcol,
    const T *__restrict__ bval, const T *__restrict__ rhs,
    TO *__restrict__ out, int64_t rows, int64_t k, int32_t b_any) {
  const int32_t b = BS > 0 ? BS : b_any;
  int64_t e = block_id() * blockDim.x + threadIdx.x;
  if (e >= rows * k)
    return;
  int64_t r = e / k, c = e - r * k;
  if constexpr (ROW) // rows < 2^31
    r = __builtin_amdgcn_readfirstlane((int32_t)r);
  int64_t br = r / b, lr = r - br * b;
  float acc = 0.0f;
  for (int32_t bp = bro[br]; bp < bro[br + 1]; ++bp) {
    const T *blk = bval + (int64_t)bp * b * b + lr * b;
    int64_t rb = (int64_t)bcol[bp] * b;
    if constexpr (BS > 0) {
      float a[BS], x[BS];
#pragma unroll
      for (int lc = 0; lc < BS; ++lc) {
        a[lc] = tof(blk[lc]);
        x[lc] = tof(rhs[(rb + lc) * k + c]);
      }
#pragma unroll
      for (int lc = 0; lc < BS; ++lc)
        acc = __builtin_fmaf(a[lc], x[lc], acc);
    } else {
      for (int32_t lc = 0; lc < b; ++lc)
        acc = __builtin_fmaf(tof(blk[lc]), tof(rhs[(rb + lc) * k + c]), acc);
    }
  }
  stv(out + e, acc);
}

// MFMA operand layouts (one 16 x 16 x K step, wave64, lane l):
//   A[i][k] with i = l % 16, k from the lane group g = l / 16,
//   B[k][j] with j = l % 16, same k,
//   D[4*g + v][l % 16] in accumulator register v.
// The k order inside a block is a free choice as long as A and B agree;
// fp32 uses k = 4*g + s at step s so that one 128-bit load gives a lane its
// four A values.
// Block rows are visited XCD-aware: workgroups are dispatched to the eight
// XCDs round-robin, so workgroup w runs block row
// (w % 8) * (nbr / 8) + w / 8 and each XCD walks a contiguous range of block
// rows, keeping the RHS tiles of a banded matrix in its own L2.
__device__ __forceinline__ int xcd_block_row(int w, int nbr) {
  constexpr int kXcds = 8;
  if (nbr % kXcds != 0)
    return w;
  return (w % kXcds) * (nbr / kXcds) + w / kXcds;
}

// Blocks are processed in batches of NB: the batch's column indices arrive
// with one load (lane j holds block j's column, broadcast by v_readlane),
// then every A and B operand of the batch is requested before the first
// MFMA, so a block row waits for two memory latencies per batch instead of
// two per block.
template <int NB>
__global__ __launch_bounds__(256) void bsr16_mfma_f32(
    const int32_t *__restrict__ bro, const int32_t *__restrict__ bcol,
    const float *__restrict__ bval, const float *__restrict__ rhs,
    float *__restrict__ out, int64_t k, int nbr) {
  const int br = xcd_block_row(blockIdx.x, nbr);
  const int wave = wave_in_group();
  const int l = lane_id();
  const int i = l & 15, g = l >> 4;
  const int64_t n0 = (int64_t)blockIdx.y * 128 + wave * 32;
  const int64_t c0 = n0 + i, c1 = n0 + 16 + i;
  const bool ok0 = c0 < k, ok1 = c1 < k;
  v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  const int32_t s = bro[br], e = bro[br + 1];
  for (int32_t b0 = s; b0 < e; b0 += NB) {
    const int nb = e - b0 < NB ? e - b0 : NB; // wave-uniform
    const int bcl = l < nb ? bcol[b0 + l] : 0;
    v4f a[NB];
    float bv0[NB][4], bv1[NB][4];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (j < nb) {
        const int64_t bc = __builtin_amdgcn_readlane(bcl, j);
        a[j] = ld_stream(reinterpret_cast<const v4f *>(
            bval + (int64_t)(b0 + j) * 256 + i * 16 + g * 4));
        const float *brow = rhs + (bc * 16 + g * 4) * k;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          bv0[j][st] = ok0 ? brow[st * k + c0] : 0.0f;
          bv1[j][st] = ok1 ? brow[st * k + c1] : 0.0f;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (j < nb) {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j][st], bv0[j][st],
                                                      acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j][st], bv1[j][st],
                                                      acc1, 0, 0, 0);
        }
      }
    }
  }
  // non-temporal stores: the output is not re-read, so it should not
  // displace RHS tiles from the caches
  float *o = out + ((int64_t)br * 16 + g * 4) * k;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    if (ok0)
      __builtin_nontemporal_store(acc0[v], o + v * k + c0);
    if (ok1)
      __builtin_nontemporal_store(acc1[v], o + v * k + c1);
  }
}

template <int NB, typename TO>
__global__ __launch_bounds__(256) void bsr16_mfma_bf16(
    const int32_t *__restrict__ bro, const int32_t *__restrict__ bcol,
    const uint16_t *__restrict__ bval, const uint16_t *__restrict__ rhs,
    TO *__restrict__ out, int64_t k, int nbr) {
  const int br = xcd_block_row(blockIdx.x, nbr);
  const int wave = wave_in_group();
  const int l = lane_id();
  const int i = l & 15, g = l >> 4;
  const int64_t n0 = (int64_t)blockIdx.y * 128 + wave * 32;
  const int64_t c0 = n0 + i, c1 = n0 + 16 + i;
  const bool ok0 = c0 < k, ok1 = c1 < k;
  v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  const int32_t s = bro[br], e = bro[br + 1];
  for (int32_t b0 = s; b0 < e; b0 += NB) {
    const int nb = e - b0 < NB ? e - b0 : NB;
    const int bcl = l < nb ? bcol[b0 + l] : 0;
    v4s a[NB], bv0[NB], bv1[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (j < nb) {
        const int64_t bc = __builtin_amdgcn_readlane(bcl, j);
        // A[i][4g .. 4g+3]: 8 contiguous bytes of the row-major block
        a[j] = *reinterpret_cast<const v4s *>(bval + (int64_t)(b0 + j) * 256 +
                                              i * 16 + g * 4);
        const uint16_t *brow = rhs + (bc * 16 + g * 4) * k;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          bv0[j][st] = ok0 ? (short)brow[st * k + c0] : (short)0;
          bv1[j][st] = ok1 ? (short)brow[st * k + c1] : (short)0;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (j < nb) {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a[j], bv0[j], acc0, 0,
                                                         0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a[j], bv1[j], acc1, 0,
                                                         0, 0);
      }
    }
  }
  // non-temporal stores: the output is not re-read, so it should not
  // displace RHS tiles from the caches
  TO *o = out + ((int64_t)br * 16 + g * 4) * k;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    if (ok0)
      st1_nt(o + v * k + c0, acc0[v]);
    if (ok1)
      st1_nt(o + v * k + c1, acc1[v]);
  }
}

// Column-interleaved bf16 kernel (k % 8 == 0, rhs and output 16-byte
// aligned).  A workgroup owns one block row and a 128-column strip as eight
// 16 x 16 tiles whose columns interleave -- tile t's MFMA column j is strip
// column 8j + t -- so one 128-bit load of an RHS row gives a lane its eight
// columns' values, one per tile: per block a lane issues one 64-bit A load
// and four 128-bit B loads (the block's 16 x 128 RHS slab in four wave
// instructions), then eight v_mfma_f32_16x16x16_bf16.  The B operand of tile
// t is element t of the four loaded rows (lane group g: rows 4g .. 4g+3).
// The block row's blocks are split over the SPL waves of the workgroup
// (wave w takes blocks w NB .. w NB + NB - 1, then every NB SPL-th batch),
// which shortens each wave's chain of memory trips; the waves' partial
// tiles are summed in LDS by wave 0.  Each lane ends with eight consecutive
// columns of four output rows: one 128-bit (bf16) or two 128-bit (fp32)
// stores per row.  Workgroups run in XCD-contiguous block-row order.
//
// FLOOR (the slab-floor diagnostic, sw_bsr_slab_floor): the same grid, block
// order, loads, LDS reduction and stores, with the matrix-core products
// replaced by an XOR of every 32-bit word the lane loads; every output
// element of the lane's region then holds that XOR (truncated to 16 bits for
// a bf16 output).  Its time is the floor of the kernel's memory trips.
template <int NB, int SPL, typename TO, bool FLOOR = false>
__global__ __launch_bounds__(64 * SPL) void bsr16_mfma_bf16_x8(
    const int32_t *__restrict__ bro, const int32_t *__restrict__ bcol,
    const uint16_t *__restrict__ bval, const uint16_t *__restrict__ rhs,
    TO *__restrict__ out, int64_t k, int nbr) {
  __shared__ float red[SPL > 1 ? SPL - 1 : 1][8][4][kWave];
  const int64_t br = xcd_contiguous(blockIdx.x, gridDim.x);
  const int sp = wave_in_group();
  const int l = lane_id();
  const int j = l & 15, g = l >> 4;
  const int64_t cb = (int64_t)blockIdx.y * 128 + 8 * j;
  const bool ok = cb < k; // k % 8 == 0: all eight columns or none
  v4f acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t)
    acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  const int32_t s = bro[br], e = bro[br + 1];
  for (int32_t b0 = s + sp * NB; b0 < e; b0 += NB * SPL) {
    const int nb = e - b0 < NB ? e - b0 : NB; // wave-uniform
    const int bcl = l < nb ? bcol[b0 + l] : 0;
    v2u a[NB];
    v4u q[NB][4];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (u < nb) {
        const int64_t bc = __builtin_amdgcn_readlane(bcl, u);
        // A[j][4g .. 4g+3] of block b0 + u: 8 contiguous bytes
        a[u] = ld_stream(reinterpret_cast<const v2u *>(
            bval + (int64_t)(b0 + u) * 256 + j * 16 + g * 4));
        const uint16_t *brow = rhs + (bc * 16 + g * 4) * k + cb;
#pragma unroll
        for (int st = 0; st < 4; ++st)
          q[u][st] = ok ? *reinterpret_cast<const v4u *>(brow + st * k)
                        : v4u{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (u < nb) {
        if constexpr (FLOOR) {
          uint32_t x = a[u].x ^ a[u].y;
#pragma unroll
          for (int st = 0; st < 4; ++st)
            x ^= q[u][st].x ^ q[u][st].y ^ q[u][st].z ^ q[u][st].w;
          acc[0].x = __uint_as_float(__float_as_uint(acc[0].x) ^ x);
          continue;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          // element t of the four rows (dword t / 2, half t % 2), paired by
          // byte permutes
          const int d = t >> 1;
          const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
          const v2u bt = v2u{
              __builtin_amdgcn_perm(q[u][1][d], q[u][0][d], sel),
              __builtin_amdgcn_perm(q[u][3][d], q[u][2][d], sel)};
          acc[t] = mfma_16x16x16_bf16(a[u], bt, acc[t]);
        }
      }
    }
  }
  if constexpr (FLOOR) {
    // the XOR of the waves' words, in every element the lane stores
    if constexpr (SPL > 1) {
      if (sp > 0)
        red[sp - 1][0][0][l] = acc[0].x;
      __syncthreads();
      if (sp > 0)
        return; // after the only barrier
      uint32_t x = __float_as_uint(acc[0].x);
#pragma unroll
      for (int w = 0; w < SPL - 1; ++w)
        x ^= __float_as_uint(red[w][0][0][l]);
      acc[0].x = __uint_as_float(x);
    }
    const uint32_t x = __float_as_uint(acc[0].x);
    if (ok) {
      TO *o = out + (br * 16 + g * 4) * k + cb;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if constexpr (sizeof(TO) == 2) {
          const uint32_t h = (x & 0xFFFFu) | (x << 16);
          __builtin_nontemporal_store(v4u{h, h, h, h},
                                      reinterpret_cast<v4u *>(o + v * k));
        } else {
          const float f = __uint_as_float(x);
          st4_nt(o + v * k, v4f{f, f, f, f});
          st4_nt(o + v * k + 4, v4f{f, f, f, f});
        }
      }
    }
    return;
  }
  if constexpr (SPL > 1) {
    if (sp > 0)
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          red[sp - 1][t][v][l] = acc[t][v];
    __syncthreads();
    if (sp > 0)
      return; // after the only barrier
#pragma unroll
    for (int w = 0; w < SPL - 1; ++w)
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          acc[t][v] += red[w][t][v][l];
  }
  if (ok) {
    TO *o = out + (br * 16 + g * 4) * k + cb;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if constexpr (sizeof(TO) == 2) {
        __builtin_nontemporal_store(
            v4u{pack_bf16x2(acc[0][v], acc[1][v]),
                pack_bf16x2(acc[2][v], acc[3][v]),
                pack_bf16x2(acc[4][v], acc[5][v]),
                pack_bf16x2(acc[6][v], acc[7][v])},
            reinterpret_cast<v4u *>(o + v * k));
      } else {
        st4_nt(o + v * k, v4f{acc[0][v], acc[1][v], acc[2][v], acc[3][v]});
        st4_nt(o + v * k + 4, v4f{acc[4][v], acc[5][v], acc[6][v], acc[7][v]});
      }
    }
  }
}

// Column-interleaved fp32 variant (k % 4 == 0, 16-byte aligned operands): a
// wave owns a 16 x 64 output strip as four 16 x 16 MFMA tiles whose columns
// interleave -- tile t's MFMA column j is output column 4j + t of the strip --
// so one 128-bit load of an RHS row gives a lane its B values for all four
// tiles, and one 128-bit store writes its four results of an output row.
// Per block and strip a lane issues one A load and four B loads instead of
// one A load and sixteen scalar B loads.
//
// A workgroup covers one block row and up to kF32Strips strips; SPL waves per
// strip split the block row's blocks (wave sp takes batches sp, sp + SPL, ...)
// so that more loads are in flight per block row, and the SPL partial tiles
// are summed through LDS by wave 0 of each strip.
constexpr int kF32Strips = 2;

// FLOOR: the slab-floor diagnostic, as for the bf16 kernel above.
template <int NB, int SPL, bool FLOOR = false>
__global__ __launch_bounds__(64 * kF32Strips * SPL) void bsr16_mfma_f32_x4(
    const int32_t *__restrict__ bro, const int32_t *__restrict__ bcol,
    const float *__restrict__ bval, const float *__restrict__ rhs,
    float *__restrict__ out, int64_t k, int nbr) {
  __shared__ float red[kF32Strips][SPL > 1 ? SPL - 1 : 1][4][4][kWave];
  const int br = xcd_block_row(blockIdx.x, nbr);
  const int strips = blockDim.x / (kWave * SPL);
  const int wv = wave_in_group();
  const int strip = wv % strips, sp = wv / strips;
  const int l = lane_id();
  const int i = l & 15, g = l >> 4;
  const int64_t cb = ((int64_t)blockIdx.y * strips + strip) * 64 + 4 * i;
  const bool ok = cb < k; // k % 4 == 0: all four columns or none
  v4f acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  const int32_t s = bro[br], e = bro[br + 1];
  for (int32_t b0 = s + sp * NB; b0 < e; b0 += NB * SPL) {
    const int nb = e - b0 < NB ? e - b0 : NB; // wave-uniform
    const int bcl = l < nb ? bcol[b0 + l] : 0;
    v4f a[NB], bv[NB][4];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (j < nb) {
        const int64_t bc = __builtin_amdgcn_readlane(bcl, j);
        a[j] = ld_stream(reinterpret_cast<const v4f *>(
            bval + (int64_t)(b0 + j) * 256 + i * 16 + g * 4));
        const float *brow = rhs + (bc * 16 + g * 4) * k + cb;
#pragma unroll
        for (int st = 0; st < 4; ++st)
          bv[j][st] = ok ? *reinterpret_cast<const v4f *>(brow + st * k)
                         : v4f{0.f, 0.f, 0.f, 0.f};
      }
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (j < nb) {
        if constexpr (FLOOR) {
          uint32_t x = 0;
#pragma unroll
          for (int st = 0; st < 4; ++st)
            x ^= __float_as_uint(a[j][st]) ^ __float_as_uint(bv[j][st].x) ^
                 __float_as_uint(bv[j][st].y) ^ __float_as_uint(bv[j][st].z) ^
                 __float_as_uint(bv[j][st].w);
          acc[0].x = __uint_as_float(__float_as_uint(acc[0].x) ^ x);
          continue;
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j][st], bv[j][st].x,
                                                        acc[0], 0, 0, 0);
          acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j][st], bv[j][st].y,
                                                        acc[1], 0, 0, 0);
          acc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j][st], bv[j][st].z,
                                                        acc[2], 0, 0, 0);
          acc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j][st], bv[j][st].w,
                                                        acc[3], 0, 0, 0);
        }
      }
    }
  }
  if constexpr (FLOOR) {
    if constexpr (SPL > 1) {
      if (sp > 0)
        red[strip][sp - 1][0][0][l] = acc[0].x;
      __syncthreads();
      if (sp > 0)
        return;
      uint32_t x = __float_as_uint(acc[0].x);
#pragma unroll
      for (int w = 0; w < SPL - 1; ++w)
        x ^= __float_as_uint(red[strip][w][0][0][l]);
      acc[0].x = __uint_as_float(x);
    }
    if (ok) {
      float *o = out + ((int64_t)br * 16 + g * 4) * k + cb;
      const float f = acc[0].x;
#pragma unroll
      for (int v = 0; v < 4; ++v)
        __builtin_nontemporal_store(v4f{f, f, f, f},
                                    reinterpret_cast<v4f *>(o + v * k));
    }
    return;
  }
  if constexpr (SPL > 1) {
    if (sp > 0) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          red[strip][sp - 1][t][v][l] = acc[t][v];
    }
    __syncthreads();
    if (sp > 0)
      return;
#pragma unroll
    for (int w = 0; w < SPL - 1; ++w)
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          acc[t][v] += red[strip][w][t][v][l];
  }
  if (ok) {
    float *o = out + ((int64_t)br * 16 + g * 4) * k + cb;
#pragma unroll
    for (int v = 0; v < 4; ++v)
      __builtin_nontemporal_store(v4f{acc[0][v], acc[1][v], acc[2][v],
                                      acc[3][v]},
                                  reinterpret_cast<v4f *>(o + v * k));
  }
}

// fp32 x4 kernel shape: blocks per batch and waves per strip. Configuration
// 4, two strips per workgroup: 1 wave x 4-block batches 134.0 us, 2 x 2
// 127.5 us, 2 x 1 128.3 us, 2 x 4 144.2 us, 4 x 2 130.3 us, 4 x 1 124.0 us.
constexpr int kF32Batch = 1;
constexpr int kF32Split = 4;

int check_bsr(const int32_t *bro, const int32_t *bcol, const void *bval,
              const void *rhs, const void *out, int64_t rows, int64_t cols,
              int64_t nnzb, int64_t k, int64_t b) {
  if (b < 1)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "BSR block size must be positive, but got %lld",
                    (long long)b);
  if (rows < 0 || cols < 0 || nnzb < 0 || k < 0)
    return sw::fail(SW_ERR_INVALID_SHAPE, "negative BSR shape");
  if (rows % b != 0 || cols % b != 0)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "BSR matrix dimensions %lld x %lld must be divisible by "
                    "block size %lld",
                    (long long)rows, (long long)cols, (long long)b);
  if (nnzb * b * b > (int64_t)INT32_MAX * 16)
    return sw::fail(SW_ERR_INVALID_SHAPE, "too many BSR blocks");
  if (rows / b > INT32_MAX - 1)
    return sw::fail(SW_ERR_INVALID_SHAPE, "too many BSR block rows");
  if (!bro)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "block row offsets pointer is null");
  if (rows > 0 && k > 0 && !out)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "output pointer is null");
  if (nnzb > 0 && (!bcol || !bval || (k > 0 && !rhs)))
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "BSR operand pointer is null");
  return SW_OK;
}

// bf16 x8 kernel shape: blocks per batch and waves per block row.
// Configuration 4 (bf16 output), one wave per block row: batches of
// 1 / 2 / 4 / 8 blocks 63.2 / 62.1 / 69.9 / 113.6 us (94 VGPRs at 2, 142 at
// 4); the block row split over waves: 2 waves x 2-block batches 60.8 us,
// 2 x 1 58.3 us, 4 x 1 56.6 us, 4 x 2 62.8 us, 8 x 1 98.2 us.
constexpr int kBf16Batch = 1;
constexpr int kBf16Split = 4;

template <typename T, typename TO>
int launch_bsr(const int32_t *bro, const int32_t *bcol, const T *bval,
               const T *rhs, TO *out, int64_t rows, int64_t nnzb, int64_t k,
               int64_t b, const sw_options &o, hipStream_t st, bool mfma_ok) {
  (void)nnzb;
  if (rows == 0 || k == 0)
    return SW_OK;
  const int nbr = (int)(rows / 16);
  // The matrix-core kernels index block rows by blockIdx.x alone (y holds
  // the column strips), so their x must stay within one grid dimension's
  // 2^32 - 1 work-items (512-work-item workgroups: about 8.4 million block
  // rows); past it the thread-per-output kernel below, whose launch folds,
  // computes the product.
  mfma_ok = mfma_ok && nbr <= sw::grid_row(512);
  if constexpr (sizeof(T) == 4) {
    // fp32 with k % 4 == 0 takes the column-interleaved kernel (measured on
    // configuration 4: 167 us against 189 us for the one-column-per-lane
    // kernel below, before the block row was split over waves)
    if (mfma_ok && k % 4 == 0 && sw::aligned16(rhs) && sw::aligned16(out)) {
      const int64_t strips =
          std::min<int64_t>(kF32Strips, sw::ceil_div(k, 64));
      const int64_t gy = sw::ceil_div(k, 64 * strips);
      if (gy > 65535)
        return sw::fail(SW_ERR_INVALID_SHAPE, "rhs has too many columns");
      const int rc = sw::check_flat_grid(nbr, 64 * strips * kF32Split,
                                         "BSR MFMA kernel");
      if (rc)
        return rc;
      hipLaunchKernelGGL((bsr16_mfma_f32_x4<kF32Batch, kF32Split>),
                         dim3((unsigned)nbr, (unsigned)gy),
                         dim3((unsigned)(64 * strips * kF32Split)), 0, st, bro,
                         bcol, bval, rhs, out, k, nbr);
      return sw::launch_check("BSR MFMA kernel");
    }
  } else {
    // k % 8 == 0: eight interleaved tiles per workgroup, 128-bit RHS loads
    // (configuration 4: bf16 output 57.1 us against 69.8 us for the two-tile
    // kernel below; fp32 output 74.3 against 73.7 us)
    {
      if (mfma_ok && k % 8 == 0 && sw::aligned16(rhs) && sw::aligned16(out)) {
        const int64_t gy = sw::ceil_div(k, 128);
        if (gy > 65535)
          return sw::fail(SW_ERR_INVALID_SHAPE, "rhs has too many columns");
        const int rc =
            sw::check_flat_grid(nbr, 64 * kBf16Split, "BSR MFMA kernel");
        if (rc)
          return rc;
        hipLaunchKernelGGL((bsr16_mfma_bf16_x8<kBf16Batch, kBf16Split, TO>),
                           dim3((unsigned)nbr, (unsigned)gy),
                           dim3(64 * kBf16Split), 0, st, bro, bcol, bval,
                           rhs, out, k, nbr);
        return sw::launch_check("BSR MFMA kernel");
      }
    }
  }
  if (mfma_ok) {
    int64_t gy = sw::ceil_div(k, 128);
    if (gy > 65535)
      return sw::fail(SW_ERR_INVALID_SHAPE, "rhs has too many columns");
    const int rc = sw::check_flat_grid(nbr, 256, "BSR MFMA kernel");
    if (rc)
      return rc;
    dim3 grid((unsigned)nbr, (unsigned)gy);
    if constexpr (sizeof(T) == 4)
      hipLaunchKernelGGL(bsr16_mfma_f32<8>, grid, dim3(256), 0, st, bro, bcol,
                         bval, rhs, out, k, nbr);
    else
      hipLaunchKernelGGL((bsr16_mfma_bf16<8, TO>), grid, dim3(256), 0, st, bro,
                         bcol, bval, rhs, out, k, nbr);
    return sw::launch_check("BSR MFMA kernel");
  }
  const int64_t B = o.spmm_block_size;
  int64_t grid = std::max<int64_t>(sw::ceil_div(rows * k, B), 1);
  int rc = sw::check_grid(grid, B, "BSR SpMM");
  if (rc)
    return rc;
  const bool row = k % 64 == 0 && B % 64 == 0 && rows <= INT32_MAX;
#define SW_BSR_TPO(BS, ROW)                                                   \
  hipLaunchKernelGGL((bsr_thread_per_output<T, TO, BS, ROW>),                 \
                     sw::grid_dim(grid, B), dim3((unsigned)B), 0, st, bro,   \
                     bcol, bval, rhs, out, rows, k, (int32_t)b)
  if (b == 16 && row)
    SW_BSR_TPO(16, true);
  else if (b == 16)
    SW_BSR_TPO(16, false);
  else if (row)
    SW_BSR_TPO(0, true);
  else
    SW_BSR_TPO(0, false);
#undef SW_BSR_TPO
  return sw::launch_check("thread-per-output BSR SpMM kernel");
}

template <typename T, typename TO>
int bsr_entry(const int32_t *block_row_offsets,
              const int32_t *block_column_indices, const T *block_values,
              const T *rhs, TO *output, int64_t rows, int64_t cols,
              int64_t nnzb, int64_t k, int64_t block_size,
              const sw_options *opts, void *stream) {
  sw::clear_error();
  sw_options o;
  int rc = sw::resolve_options(opts, &o);
  if (rc)
    return rc;
  rc = check_bsr(block_row_offsets, block_column_indices, block_values, rhs,
                 output, rows, cols, nnzb, k, block_size);
  if (rc)
    return rc;
  rc = sw::check_value_alignment(sizeof(T), {block_values, rhs});
  if (!rc)
    rc = sw::check_value_alignment(sizeof(TO), {output});
  if (rc)
    return rc;
  // the MFMA kernels read A rows of a block as 16-byte (fp32) or 8-byte
  // (bf16) vectors
  const bool mfma = o.bsr_use_mfma && block_size == 16 &&
                    (reinterpret_cast<uintptr_t>(block_values) &
                     (4 * sizeof(T) - 1)) == 0;
  return launch_bsr<T, TO>(block_row_offsets, block_column_indices,
                           block_values, rhs, output, rows, nnzb, k,
                           block_size, o, sw::as_stream(stream), mfma);
}

// The slab floor: the MFMA kernel launch_bsr would run for these operands,
// in its FLOOR form.
template <typename T, typename TO>
int launch_slab_floor(const int32_t *bro, const int32_t *bcol, const T *bval,
                      const T *rhs, TO *out, int64_t rows, int64_t k,
                      hipStream_t st) {
  if (rows == 0 || k == 0)
    return SW_OK;
  const int nbr = (int)(rows / 16);
  if constexpr (sizeof(T) == 4) {
    const int64_t strips = std::min<int64_t>(kF32Strips, sw::ceil_div(k, 64));
    const int64_t gy = sw::ceil_div(k, 64 * strips);
    if (gy > 65535)
      return sw::fail(SW_ERR_INVALID_SHAPE, "rhs has too many columns");
    const int rc = sw::check_flat_grid(nbr, 64 * strips * kF32Split,
                                       "BSR slab floor kernel");
    if (rc)
      return rc;
    hipLaunchKernelGGL((bsr16_mfma_f32_x4<kF32Batch, kF32Split, true>),
                       dim3((unsigned)nbr, (unsigned)gy),
                       dim3((unsigned)(64 * strips * kF32Split)), 0, st, bro,
                       bcol, bval, rhs, out, k, nbr);
  } else {
    const int64_t gy = sw::ceil_div(k, 128);
    if (gy > 65535)
      return sw::fail(SW_ERR_INVALID_SHAPE, "rhs has too many columns");
    const int rc =
        sw::check_flat_grid(nbr, 64 * kBf16Split, "BSR slab floor kernel");
    if (rc)
      return rc;
    hipLaunchKernelGGL((bsr16_mfma_bf16_x8<kBf16Batch, kBf16Split, TO, true>),
                       dim3((unsigned)nbr, (unsigned)gy), dim3(64 * kBf16Split),
                       0, st, bro, bcol, bval, rhs, out, k, nbr);
  }
  return sw::launch_check("BSR slab floor kernel");
}

} // namespace

extern "C" int sw_bsr_slab_floor(const int32_t *block_row_offsets,
                                 const int32_t *block_column_indices,
                                 const void *block_values, const void *rhs,
                                 void *output, int64_t rows, int64_t cols,
                                 int64_t nnzb, int64_t k, int value_bytes,
                                 int output_bytes, void *stream) {
  sw::clear_error();
  int rc = check_bsr(block_row_offsets, block_column_indices, block_values,
                     rhs, output, rows, cols, nnzb, k, 16);
  if (rc)
    return rc;
  const bool f32 = value_bytes == 4 && output_bytes == 4;
  const bool b16 = value_bytes == 2 && (output_bytes == 2 || output_bytes == 4);
  if (!f32 && !b16)
    return sw::fail(SW_ERR_INVALID_ARGUMENT,
                    "slab floor value / output bytes must be 4 / 4, 2 / 2 or "
                    "2 / 4, but got %d / %d", value_bytes, output_bytes);
  // the floor runs where the MFMA kernels run: 16-byte aligned rhs and
  // output, block values aligned to four elements, k % 4 (fp32) or k % 8
  const uintptr_t va = reinterpret_cast<uintptr_t>(block_values);
  if (k % (f32 ? 4 : 8) != 0 || !sw::aligned16(rhs) ||
      !sw::aligned16(output) || (va & (4u * value_bytes - 1)) != 0)
    return sw::fail(SW_ERR_INVALID_ARGUMENT,
                    "the slab floor needs the MFMA kernels' shapes: k a "
                    "multiple of %d, 16-byte aligned rhs and output, block "
                    "values aligned to %d bytes", f32 ? 4 : 8,
                    4 * value_bytes);
  hipStream_t st = sw::as_stream(stream);
  if (f32)
    return launch_slab_floor<float, float>(
        block_row_offsets, block_column_indices,
        static_cast<const float *>(block_values),
        static_cast<const float *>(rhs), static_cast<float *>(output), rows,
        k, st);
  if (output_bytes == 2)
    return launch_slab_floor<uint16_t, uint16_t>(
        block_row_offsets, block_column_indices,
        static_cast<const uint16_t *>(block_values),
        static_cast<const uint16_t *>(rhs), static_cast<uint16_t *>(output),
        rows, k, st);
  return launch_slab_floor<uint16_t, float>(
      block_row_offsets, block_column_indices,
      static_cast<const uint16_t *>(block_values),
      static_cast<const uint16_t *>(rhs), static_cast<float *>(output), rows,
      k, st);
}

extern "C" int sw_bsr_spmm_f32(const int32_t *block_row_offsets,
                               const int32_t *block_column_indices,
                               const float *block_values, const float *rhs,
                               float *output, int64_t rows, int64_t cols,
                               int64_t nnzb, int64_t k, int64_t block_size,
                               const sw_options *opts, void *stream) {
  return bsr_entry<float, float>(block_row_offsets, block_column_indices,
                                 block_values, rhs, output, rows, cols, nnzb,
                                 k, block_size, opts, stream);
}

extern "C" int sw_bsr_spmm_bf16(const int32_t *block_row_offsets,
                                const int32_t *block_column_indices,
                                const uint16_t *block_values,
                                const uint16_t *rhs, uint16_t *output,
                                int64_t rows, int64_t cols, int64_t nnzb,
                                int64_t k, int64_t block_size,
                                const sw_options *opts, void *stream) {
  return bsr_entry<uint16_t, uint16_t>(block_row_offsets,
                                       block_column_indices, block_values, rhs,
                                       output, rows, cols, nnzb, k, block_size,
                                       opts, stream);
}

extern "C" int sw_bsr_spmm_bf16_f32out(const int32_t *block_row_offsets,
                                       const int32_t *block_column_indices,
                                       const uint16_t *block_values,
                                       const uint16_t *rhs, float *output,
                                       int64_t rows, int64_t cols,
                                       int64_t nnzb, int64_t k,
                                       int64_t block_size,
                                       const sw_options *opts, void *stream) {
  return bsr_entry<uint16_t, float>(block_row_offsets, block_column_indices,
                                    block_values, rhs, output, rows, cols,
                                    nnzb, k, block_size, opts, stream);
}
