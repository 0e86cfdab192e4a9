// Device-side building blocks for gfx950 (CDNA4, Wave64).
//
// Cross-lane work uses DPP (row_shr, quad_perm, row_mirror, row_bcast) and
// ds_swizzle, which move data through the VALU without LDS memory, and
// v_readlane for wave-uniform results.  Streaming CSR and BSR arrays are
// read with plain loads (ld_stream); the non-temporal hint is kept where it
// measured no slower: the values of the position and COO SpMV kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

namespace swd {

constexpr int kWave = 64;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ int lane_id() { return __lane_id(); }
// The workgroup's index in the launch and the launch's workgroup count: a
// 1-D launch of more than 2^32 - 1 work-items is folded into an (x, y) grid
// (one dimension's work-item count is 32 bits), numbered row by row; the
// last row's surplus workgroups return from their kernel's index checks.
// Both values are wave-uniform (scalar registers).
__device__ __forceinline__ int64_t block_id() {
  return (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
}
__device__ __forceinline__ int64_t grid_blocks() {
  return (int64_t)gridDim.x * gridDim.y;
}
// The wave's index in its workgroup, in a scalar register: it is the same in
// every lane, but as threadIdx.x / 64 the compiler keeps it per lane and
// makes every test and product on it a vector instruction.
__device__ __forceinline__ int wave_in_group() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
}

// ---- DPP --------------------------------------------------------------
// DPP control codes (GFX9 encoding).
constexpr int kQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kRowShr1 = 0x111;
constexpr int kRowShr2 = 0x112;
constexpr int kRowShr4 = 0x114;
constexpr int kRowShr8 = 0x118;
constexpr int kRowMirror = 0x140;      // lane i <- 15 - i within a row of 16
constexpr int kRowHalfMirror = 0x141;  // lane i <- 7 - i within 8 lanes
constexpr int kRowBcast15 = 0x142;     // lane 15 of row r -> row r+1
constexpr int kRowBcast31 = 0x143;     // lane 31 -> rows 2 and 3

// Lanes whose DPP source is invalid (or masked off) keep `old`.
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ __forceinline__ int dpp_i(int old, int src) {
  return __builtin_amdgcn_update_dpp(old, src, CTRL, ROW_MASK, BANK_MASK,
                                     false);
}
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float old, float src) {
  return __int_as_float(dpp_i<CTRL, ROW_MASK, BANK_MASK>(__float_as_int(old),
                                                         __float_as_int(src)));
}

// ds_swizzle bit mode: lane i reads lane ((i & and) | or) ^ xor within 32.
__device__ __forceinline__ float swizzle_xor16(float v) {
  return __int_as_float(
      __builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (0x10 << 10)));
}

__device__ __forceinline__ float shfl_xor32(float v) {
  // lane ^ 32: ds_bpermute with a byte address
  int src = (lane_id() ^ 32) << 2;
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(v)));
}

// Sum over aligned groups of G lanes (G a power of two <= 64); every lane of
// a group receives the group sum.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 2) v += dpp_f<kQuadXor1>(0.0f, v);
  if constexpr (G >= 4) v += dpp_f<kQuadXor2>(0.0f, v);
  if constexpr (G >= 8) v += dpp_f<kRowHalfMirror>(0.0f, v);
  if constexpr (G >= 16) v += dpp_f<kRowMirror>(0.0f, v);
  if constexpr (G >= 32) v += swizzle_xor16(v);
  if constexpr (G >= 64) v += shfl_xor32(v);
  return v;
}

// Whole-wave sum, returned wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<kQuadXor1>(0.0f, v);
  v += dpp_f<kQuadXor2>(0.0f, v);
  v += dpp_f<kRowHalfMirror>(0.0f, v);
  v += dpp_f<kRowMirror>(0.0f, v);
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}

// Inclusive segmented scan over the wave: lane l adds the running value of
// lane l - k whenever both carry the same key.  Keys must be non-decreasing
// over the lanes that matter (CSR rows are), which makes the combine
// associative, so the Hillis-Steele row_shr steps followed by the two
// row_bcast steps give the segmented prefix sum.
__device__ __forceinline__ float wave_segmented_scan(int key, float v) {
  constexpr int kNoKey = INT32_MIN;
  int k;
  float s;
  k = dpp_i<kRowShr1>(kNoKey, key);
  s = dpp_f<kRowShr1>(0.0f, v);
  v += (k == key) ? s : 0.0f;
  k = dpp_i<kRowShr2>(kNoKey, key);
  s = dpp_f<kRowShr2>(0.0f, v);
  v += (k == key) ? s : 0.0f;
  k = dpp_i<kRowShr4>(kNoKey, key);
  s = dpp_f<kRowShr4>(0.0f, v);
  v += (k == key) ? s : 0.0f;
  k = dpp_i<kRowShr8>(kNoKey, key);
  s = dpp_f<kRowShr8>(0.0f, v);
  v += (k == key) ? s : 0.0f;
  k = dpp_i<kRowBcast15, 0xA>(kNoKey, key);
  s = dpp_f<kRowBcast15, 0xA>(0.0f, v);
  v += (k == key) ? s : 0.0f;
  k = dpp_i<kRowBcast31, 0xC>(kNoKey, key);
  s = dpp_f<kRowBcast31, 0xC>(0.0f, v);
  v += (k == key) ? s : 0.0f;
  return v;
}

// XCD-contiguous workgroup order.  Workgroups are dispatched to the eight
// XCDs round-robin (workgroup b to XCD b % 8); this maps b to a position so
// that each XCD works through one contiguous range of the n workgroups' work,
// and neighbouring work items share that XCD's L2.  A bijection on [0, n).
__device__ __forceinline__ int64_t xcd_contiguous(int64_t b, int64_t n) {
  constexpr int64_t kXcds = 8;
  const int64_t q = n / kXcds, r = n % kXcds;
  const int64_t x = b % kXcds, i = b / kXcds;
  return x * q + (x < r ? x : r) + i;
}

// Shift by one lane up / down across the whole wave (ds_bpermute).
__device__ __forceinline__ int shfl_up1_i(int v, int fill) {
  int l = lane_id();
  int r = __builtin_amdgcn_ds_bpermute((l - 1) << 2, v);
  return l == 0 ? fill : r;
}
__device__ __forceinline__ float shfl_up1_f(float v, float fill) {
  return __int_as_float(shfl_up1_i(__float_as_int(v), __float_as_int(fill)));
}
__device__ __forceinline__ int shfl_down1_i(int v, int fill) {
  int l = lane_id();
  int r = __builtin_amdgcn_ds_bpermute((l + 1) << 2, v);
  return l == kWave - 1 ? fill : r;
}

__device__ __forceinline__ uint64_t ballot(bool p) {
  return __builtin_amdgcn_ballot_w64(p);
}

// ---- softmax arithmetic -----------------------------------------------------
// exp(x) as the hardware base-2 exponential of x log2 e (v_exp_f32), used by
// the fused attention kernels and the lrrt bundle's exponentials: rounding
// the product adds at most 2^-24 |x log2 e| ln 2 relative error (1.2e-6 at
// x = -20, beside v_exp_f32's own ulp), 2 vector instructions instead of
// the library expf's 13 (range reduction, ldexp and range checks).  A
// softmax's arguments are x = s - max <= 0, so nothing overflows; -inf gives
// 0 and NaN stays NaN, as with expf.  Unlike expf, v_exp_f32 flushes a
// result below 2^-126 to zero: for x < -87.3 the exponential is 0 where expf
// gives a subnormal, an absolute error below 2^-126 in each probability (the
// row sum is at least 1).
__device__ __forceinline__ float exp_by_exp2(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

// ---- loads ---------------------------------------------------------------
// Operands streamed once per launch (CSR columns and values, BSR blocks).
// A plain load: with the non-temporal hint the CSR SpMV/SpMM and BSR kernels
// measured 1-13% slower on MI355X (config-2 thread-per-row 825 -> 714 us,
// wave-per-row 297 -> 270 us, BSR fp32 148 -> 133 us without it).
template <typename T>
__device__ __forceinline__ T ld_stream(const T *p) {
  return *p;
}

// Non-temporal load: used for the values of the position SpMV and the COO
// SpMV, where it measured no slower and keeps x longer in L2.
template <typename T>
__device__ __forceinline__ T ld_nontemporal(const T *p) {
  return __builtin_nontemporal_load(p);
}

// ---- bf16 storage ----------------------------------------------------------
// bf16 operands travel as raw 16-bit patterns (uint16_t).  Kernels compute in
// fp32: widening is exact, and every stored bf16 result is rounded to nearest
// even once (v_cvt_pk_bf16_f32; NaN stays NaN, overflow rounds to inf).
__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
// bf16(lo) in bits 0..15, bf16(hi) in bits 16..31
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}
// fp32 value of an element stored as T (float, or bf16 bits as uint16_t)
__device__ __forceinline__ float tof(float v) { return v; }
__device__ __forceinline__ float tof(uint16_t v) { return bf16_to_f32(v); }
template <typename T>
__device__ __forceinline__ float ldv(const T *p) {
  return tof(*p);
}
__device__ __forceinline__ void stv(float *p, float v) { *p = v; }
__device__ __forceinline__ void stv(uint16_t *p, float v) {
  *p = f32_to_bf16(v);
}
// Four consecutive elements as fp32 (16-byte aligned floats, 8-byte aligned
// bf16), and their non-temporal store.
__device__ __forceinline__ v4f ld4(const float *p) {
  return *reinterpret_cast<const v4f *>(p);
}
__device__ __forceinline__ v4f ld4(const uint16_t *p) {
  const v2u w = *reinterpret_cast<const v2u *>(p);
  return v4f{bf16_to_f32(w.x & 0xFFFFu), bf16_to_f32(w.x >> 16),
             bf16_to_f32(w.y & 0xFFFFu), bf16_to_f32(w.y >> 16)};
}
__device__ __forceinline__ void st4_nt(float *p, v4f v) {
  __builtin_nontemporal_store(v, reinterpret_cast<v4f *>(p));
}
__device__ __forceinline__ void st4_nt(uint16_t *p, v4f v) {
  __builtin_nontemporal_store(v2u{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)},
                              reinterpret_cast<v2u *>(p));
}
template <typename T>
__device__ __forceinline__ void st1_nt(T *p, float v) {
  if constexpr (sizeof(T) == 4)
    __builtin_nontemporal_store(v, reinterpret_cast<float *>(p));
  else
    __builtin_nontemporal_store(f32_to_bf16(v), reinterpret_cast<uint16_t *>(p));
}

// ---- bf16 matrix-core products ------------------------------------------------
// D += A B over one 16 x 16 tile, fp32 accumulation.  Operand registers hold
// bf16 pairs, element 2e in the low half of dword e.  Lane l supplies row (A)
// or column (B) l % 16 of the operand and a block of K elements picked by
// l / 16 -- the same K elements in A and in B, so any assignment of logical
// K indices to (l / 16, element) works as long as both operands use it.  The
// result is D[4 (l / 16) + v][l % 16] in accumulator register v.
__device__ __forceinline__ v4f mfma_16x16x32_bf16(v4u a, v4u b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
      __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
      0);
}
__device__ __forceinline__ v4f mfma_16x16x16_bf16(v2u a, v2u b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
      __builtin_bit_cast(v4s, a), __builtin_bit_cast(v4s, b), c, 0, 0, 0);
}
// Element n (0..3) of two 4-element bf16 vectors, each held as two dwords, as
// one bf16 pair with a's in the low half: one byte permute (v_perm_b32 picks
// bytes of {hi: db, lo: da}).
__device__ __forceinline__ uint32_t bf16_pair(v2u a, v2u b, int n) {
  const uint32_t da = (n & 2) ? a.y : a.x, db = (n & 2) ? b.y : b.x;
  return __builtin_amdgcn_perm(db, da, (n & 1) ? 0x07060302u : 0x05040100u);
}

// Raw buffer descriptor (stride 0) over the n bytes at the wave-uniform p.
// A buffer load adds a 32-bit lane offset and a wave-uniform SGPR offset to
// the descriptor's base, so a lane's address costs no vector instruction.
// Word 3 is the gfx9-family format word of a raw 32-bit buffer.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *p,
                                                              uint32_t n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)n,
                                           0x00020000);
}

// the float at byte lane_off + uniform_off of the buffer (lane_off < n, the
// descriptor's size, or the load reads zero)
__device__ __forceinline__ float buffer_load_f32(__amdgpu_buffer_rsrc_t r,
                                                 uint32_t lane_off,
                                                 uint32_t uniform_off) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)lane_off,
                                                  (int)uniform_off, 0));
}

// p advanced by b bytes.  With p wave-uniform this is the form the global
// memory instructions take directly (base in SGPRs, one 32-bit VGPR offset),
// so a lane's address costs no 64-bit arithmetic; the caller guarantees that
// the byte offset fits 32 bits.
template <typename T>
__device__ __forceinline__ T *at_bytes(T *p, uint32_t b) {
  using B = std::conditional_t<std::is_const_v<T>, const char, char>;
  return reinterpret_cast<T *>(reinterpret_cast<B *>(p) + b);
}

// ---- CSR row recovery -------------------------------------------------------
// All variants return (first j in [lo, hi) with ro[j] > pos) - 1, or hi - 1
// when there is none, i.e. the upper-bound search of the reference
// (SparsePositionToSCF.cpp:225-271) restricted to a range known to hold the
// answer.  For sorted row offsets the result is identical to the full search.

// Per-lane binary search.
__device__ __forceinline__ int row_search_lane(const int32_t *__restrict__ ro,
                                               uint32_t lo, uint32_t hi,
                                               int32_t pos) {
  while (lo < hi) {
    uint32_t mid = lo + ((hi - lo) >> 1);
    if (ro[mid] <= pos)
      lo = mid + 1;
    else
      hi = mid;
  }
  return (int)lo - 1;
}

// Wave-uniform binary search: every lane follows the same path, so the
// probes compile to scalar loads through the scalar data cache and cost no
// vector-memory (TA/TCP) throughput, which the x gathers saturate.
__device__ __forceinline__ int row_search_uniform(const int32_t *__restrict__ ro,
                                                  uint32_t lo, uint32_t hi,
                                                  int32_t pos) {
  lo = __builtin_amdgcn_readfirstlane(lo);
  hi = __builtin_amdgcn_readfirstlane(hi);
  pos = __builtin_amdgcn_readfirstlane(pos);
  while (lo < hi) {
    uint32_t mid = lo + ((hi - lo) >> 1);
    if (ro[mid] <= pos)
      lo = mid + 1;
    else
      hi = mid;
  }
  return (int)lo - 1;
}

// Wave-uniform galloping search for an answer expected close to `lo`:
// probes lo, lo+1, lo+3, lo+7, ... then bisects the last gap.
__device__ __forceinline__ int row_search_gallop(const int32_t *__restrict__ ro,
                                                 uint32_t lo, uint32_t hi,
                                                 int32_t pos) {
  lo = __builtin_amdgcn_readfirstlane(lo);
  hi = __builtin_amdgcn_readfirstlane(hi);
  pos = __builtin_amdgcn_readfirstlane(pos);
  uint32_t probe = lo, step = 1;
  while (probe < hi && ro[probe] <= pos) {
    lo = probe + 1;
    probe = lo + step;
    step <<= 1;
  }
  if (probe < hi)
    hi = probe + 1; // ro[probe] > pos: the answer is at most probe
  return row_search_uniform(ro, lo, hi, pos);
}

// ---- 16-row tiles with shared column structure ------------------------------
// Rows r0 .. r0+nt-1 (nt <= 16) form an MFMA tile when every row's column
// list is a prefix of the tile's last row's list -- true for block masks and
// for causal diagonal blocks, where later rows extend earlier ones.  Then the
// tile's dense products over the last row's columns give every stored entry.
// The check reads every column index of the tile once.
//
// tile_prefix_ok_block splits the rows over the W waves of the workgroup
// (wave w checks rows w, w+W, ...) and combines their verdicts in LDS; every
// thread of the workgroup must call it (it has a barrier).
__device__ __forceinline__ bool tile_prefix_ok_block(
    const int32_t *__restrict__ ro, const int32_t *__restrict__ col, int r0,
    int nt, int *verdict /* __shared__ int[1] */) {
  const int lane = lane_id();
  const int wave = wave_in_group();
  const int waves = blockDim.x / kWave;
  if (threadIdx.x == 0)
    *verdict = 1;
  __syncthreads();
  // lanes 0..nt hold ro[r0 .. r0+nt]: one load instead of a chain (loads
  // here are unconditional from clamped, valid addresses: a guarded load
  // becomes a branch that waits for it on the spot)
  const int32_t my_ro = ro[r0 + (lane < nt ? lane : nt)];
  const int32_t base_last = __builtin_amdgcn_readlane(my_ro, nt - 1);
  const int32_t len_last = __builtin_amdgcn_readlane(my_ro, nt) - base_last;
  bool ok = true;
  for (int i = wave; i < nt - 1; i += waves) {
    const int32_t b = __builtin_amdgcn_readlane(my_ro, i);
    const int32_t len = __builtin_amdgcn_readlane(my_ro, i + 1) - b;
    if (len > len_last) {
      ok = false;
      break; // wave-uniform
    }
    for (int32_t t0 = 0; t0 < len; t0 += 4 * kWave) { // wave-uniform
      int32_t x[4], y[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int32_t t = std::min(t0 + u * kWave + lane, len - 1);
        x[u] = col[b + t];
        y[u] = col[base_last + t];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
        ok &= x[u] == y[u]; // clamped lanes compare the last entry again
    }
  }
  if (__builtin_amdgcn_ballot_w64(!ok) != 0 && lane == 0)
    *verdict = 0;
  __syncthreads();
  return *verdict != 0;
}


} // namespace swd
