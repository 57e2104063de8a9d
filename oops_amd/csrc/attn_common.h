// Shared device-side building blocks of the gfx950 attention kernels.
//
// Tile geometry used by every kernel: one wavefront owns a 32 x 32 score
// tile computed with 32x32 MFMA.  In the "query-column" layout a lane owns
// one query (lane % 32) and 16 keys; lane half g = lane / 32 holds keys
// kappa(g, j) = (j / 4) * 8 + g * 4 + (j % 4), j = 0..15, which is exactly
// the row set of the MFMA 32x32 accumulator.  The same index map turns an
// accumulator straight into the k-operand of the next MFMA, so P never
// leaves registers.  Tiles staged in LDS are stored with their key (or
// query) positions permuted so each lane reads its 8 or 16 operands with one
// or two 16-byte LDS reads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/oops_amd.h"

namespace oops {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();
constexpr int kWave = 64;

__device__ __forceinline__ int kappa(int g, int j) { return ((j >> 2) << 3) | (g << 2) | (j & 3); }

// 32-key position map used for bias / mask / LSE tiles: lane half g reads
// positions g*16 .. g*16+15, which hold keys kappa(g, 0..15).
__device__ __forceinline__ int perm32(int key) {
  return (((key >> 2) & 1) << 4) | (((key >> 3) & 3) << 2) | (key & 3);
}
// 32-key position map for the k-operand of a 32x32x16 MFMA: MFMA m (keys
// 16m..16m+15) reads positions 16m + g*8 .. +7, which hold kappa(g, 8m+0..7).
__device__ __forceinline__ int perm16(int key) {
  return (key & 0x13) | (((key >> 2) & 1) << 3) | (((key >> 3) & 1) << 2);
}

// ---------------------------------------------------------------- elements
template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kVec = 1;    // operands per lane per MFMA
  static constexpr int kKStep = 2;  // k extent of one MFMA
  using Frag = float;
  static __device__ __forceinline__ float to_f(float x) { return x; }
  static __device__ __forceinline__ float from_f(float x) { return x; }
  static __device__ __forceinline__ f32x16 mma(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};
template <> struct Elem<__bf16> {
  static constexpr int kVec = 8;
  static constexpr int kKStep = 16;
  using Frag = bf16x8;
  static __device__ __forceinline__ float to_f(__bf16 x) { return (float)x; }
  static __device__ __forceinline__ __bf16 from_f(float x) { return (__bf16)x; }
  static __device__ __forceinline__ f32x16 mma(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Elem<_Float16> {
  static constexpr int kVec = 8;
  static constexpr int kKStep = 16;
  using Frag = f16x8;
  static __device__ __forceinline__ float to_f(_Float16 x) { return (float)x; }
  static __device__ __forceinline__ _Float16 from_f(float x) { return (_Float16)x; }
  static __device__ __forceinline__ f32x16 mma(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Pack 8 fp32 values into a 16-bit k-operand fragment.
template <typename T>
__device__ __forceinline__ typename Elem<T>::Frag pack8(const float* x) {
  typename Elem<T>::Frag f;
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = (T)x[i];
  return f;
}

// 16 bytes of a row: elements col .. col+16/sizeof(T)-1, zero past `limit`.
template <typename T>
__device__ __forceinline__ uint4 load16(const T* row, int col, int limit, bool vec) {
  constexpr int n = 16 / sizeof(T);
  if (vec && col + n <= limit) return *reinterpret_cast<const uint4*>(row + col);
  union {
    uint4 u;
    T e[n];
  } r;
#pragma unroll
  for (int i = 0; i < n; ++i) r.e[i] = (col + i < limit) ? row[col + i] : (T)0.0f;
  return r.u;
}

// Store the elements of a 16-byte chunk one by one (destination not 16-byte aligned).
template <typename T>
__device__ __forceinline__ void store_elems(T* dst, uint4 u) {
  const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
  for (int i = 0; i < (int)(16 / sizeof(T)); ++i) dst[i] = e[i];
}

// ---------------------------------------------------------------- geometry
struct Sample {
  int64_t G, Lq, Lk;
  int64_t q_off, q_sg, q_sh, q_si;
  int64_t k_off, k_sg, k_sh, k_si;
  int64_t v_off, v_sg, v_sh, v_si;
  int64_t o_off, o_sg, o_sh, o_si;
  int64_t do_off, do_sg, do_sh, do_si;
  int64_t b_off, b_sg, b_sh, b_si;
  int64_t m_off, m_sg, m_si;
  int64_t l_off;
  int64_t db_off, db_sg, db_sh, db_si;
  int64_t bias_mode, r0, r1, r2, r3;
};
static_assert(sizeof(Sample) == OOPS_TABLE_WIDTH * sizeof(int64_t), "table layout");

// Grid decomposition shared by host and device: every sample contributes
// G * H * ceil(L / block) * splits tiles; samples are concatenated in table
// order.  `uniform` (all samples the same tile count) skips the scan.
template <typename Count>
__device__ __forceinline__ int find_sample(int64_t& tile, const Sample* table, int num_samples,
                                           int64_t uniform, Count count) {
  if (uniform > 0) {
    const int s = (int)(tile / uniform);
    tile -= (int64_t)s * uniform;
    return s;
  }
  for (int s = 0; s < num_samples; ++s) {
    const int64_t c = count(table[s]);
    if (tile < c) return s;
    tile -= c;
  }
  return -1;
}

__device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace oops
