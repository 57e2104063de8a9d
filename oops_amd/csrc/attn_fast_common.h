// Helpers shared by the 16-bit fast-path kernels (forward and backward).
#pragma once

#include "attn_kernels.h"

namespace oops {
namespace fast {

// packed pair of 16-bit values and the v_dot2 row-sum on it
template <typename T> struct Pair;
template <> struct Pair<__bf16> {
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float dot(v2 a, v2 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
};
template <> struct Pair<_Float16> {
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float dot(v2 a, v2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }
};

constexpr int kMaxKeyTiles = 256;       // Lk <= 16384 on the fast paths
constexpr float kLazyRescale = 8.0f;    // running-max slack (log2 units)
constexpr uint32_t kOut = 0x80000000u;  // a buffer offset past every resource

// max / sum of x over both 32-lane halves, in every lane
__device__ __forceinline__ float max_halves(float x) {
  const int xi = __builtin_bit_cast(int, x);
  const auto r = __builtin_amdgcn_permlane32_swap(xi, xi, false, false);
  return fmaxf(__builtin_bit_cast(float, (int)r[0]), __builtin_bit_cast(float, (int)r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const int xi = __builtin_bit_cast(int, x);
  const auto r = __builtin_amdgcn_permlane32_swap(xi, xi, false, false);
  return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
}

__device__ __forceinline__ uint4 buffer_load16_s(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Identity k-operand carrying weight w: MFMA c of a 32-wide tile adds the
// 16 entries 16c .. 16c+15 of the other operand's k axis, each times w.
template <typename T>
__device__ __forceinline__ void identity_frags(typename Elem<T>::Frag (&id)[2], float w, int lane) {
  const int lq = lane & 31, g2 = lane >> 5;
  const T wt = (T)w;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) id[c][j] = (lq == 16 * c + g2 * 8 + j) ? wt : (T)0.0f;
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::Frag lds_frag(const T* p) {
  return __builtin_bit_cast(typename Elem<T>::Frag, *reinterpret_cast<const uint4*>(p));
}

// Store accumulator values acc[4q'..4q'+3] (head-dim d0 .. d0+3, contiguous
// for a 32x32 accumulator: rows kappa(g, 4q'+0..3)) as one 8-byte write.
template <typename T>
__device__ __forceinline__ void store4(T* row, int d0, float x0, float x1, float x2, float x3) {
  typedef T v4 __attribute__((ext_vector_type(4)));
  v4 v;
  v[0] = (T)x0;
  v[1] = (T)x1;
  v[2] = (T)x2;
  v[3] = (T)x3;
  *reinterpret_cast<v4*>(row + d0) = v;
}

}  // namespace fast
}  // namespace oops
