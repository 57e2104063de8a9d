// Helpers shared by the 16-bit fast-path kernels (forward and backward).
#pragma once
#include <type_traits>

#include "attn_kernels.h"

// Minimum workgroups per CU the fast kernels are compiled for (VGPR budget:
// 512 / (4 x this) registers per lane).
#ifndef OOPS_FWD_OCC
#define OOPS_FWD_OCC 2
#endif
#ifndef OOPS_DQ_OCC
#define OOPS_DQ_OCC 2
#endif
#ifndef OOPS_DKV_OCC
#define OOPS_DKV_OCC 2
#endif
#ifndef OOPS_DBIAS_OCC
#define OOPS_DBIAS_OCC 2
#endif
// Groups (rows) per workgroup of the dK/dV kernel with a row-shared bias: 1 or 2.
#ifndef OOPS_DKV_ROWS
#define OOPS_DKV_ROWS 1
#endif

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

// A value every lane of the wave holds (e.g. read from one LDS word) moved to
// scalar registers, so branches on it are uniform scalar branches.
__device__ __forceinline__ uint64_t uniform64(uint64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint4 buffer_load16_s(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Packed pairs p[2q], p[2q+1] of a lane's tokens (or channels) 8q + 4g .. 8q + 4g + 3 (q = 0..3, g = lane / 32) are
// traded between the two 32-lane halves with v_permlane32_swap: afterwards the lower half holds
// tokens 0..15 and the upper half tokens 16..31, lo = the first 8 and hi = the next 8 (one 32-byte
// run per lane).  Every lane of the wave must execute it.
__device__ __forceinline__ void trade16(const uint32_t (&p)[8], uint4& lo, uint4& hi) {
  const auto x0 = __builtin_amdgcn_permlane32_swap(p[0], p[4], false, false);
  const auto x1 = __builtin_amdgcn_permlane32_swap(p[1], p[5], false, false);
  const auto x2 = __builtin_amdgcn_permlane32_swap(p[2], p[6], false, false);
  const auto x3 = __builtin_amdgcn_permlane32_swap(p[3], p[7], false, false);
  lo = make_uint4(x0[0], x1[0], x0[1], x1[1]);
  hi = make_uint4(x2[0], x3[0], x2[1], x3[1]);
}

// Identity k-operand carrying weight w: MFMA c of a 32-wide tile adds the
// 16 entries 16c .. 16c+15 of the other operand's k axis, each times w.
template <typename T>
__device__ __forceinline__ void identity_frags(typename Elem<T>::Frag (&id)[2], float w, int lane) {
  // element j of fragment c holds the weight when lq == 16 c + 8 g2 + j: the
  // weight's 16 bits shifted into place within the dword that holds j
  const int lq = lane & 31, g2 = lane >> 5;
  const uint32_t wb = __builtin_bit_cast(uint16_t, (T)w);
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int j = lq - 16 * c - 8 * g2;  // in 0..7 for the one fragment that holds the weight
    const uint32_t v = wb << ((j & 1) * 16);
    uint32_t u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) u[k] = (j >> 1) == k ? v : 0u;
    id[c] = __builtin_bit_cast(typename Elem<T>::Frag, make_uint4(u[0], u[1], u[2], u[3]));
  }
}

// The identity MFMA that adds the bias multiplies every bias element of a
// 16-key chunk by the zeros of the other keys' columns, so a non-finite bias
// element (an additive -inf mask) would make the whole chunk NaN.  Bias
// elements whose exponent is all ones (+-inf, NaN) are therefore read as the
// largest finite value of their sign: -max times the weight 1/scale still
// gives a logit of -inf or below -1e38, so such a key's P is exactly 0, as
// with -inf.  (A NaN or +inf bias element, which makes the whole row NaN in
// float arithmetic, reads as +-max.)
template <typename T>
__device__ __forceinline__ uint32_t finite2(uint32_t d) {
  static_assert(std::is_same_v<T, __bf16> || std::is_same_v<T, _Float16>, "16-bit elements");
  constexpr uint32_t kExp = std::is_same_v<T, __bf16> ? 0x7F80u : 0x7C00u;  // exponent field
  constexpr uint32_t kMax = std::is_same_v<T, __bf16> ? 0x7F7Fu : 0x7BFFu;  // largest finite magnitude
  const uint32_t sp = ((d & kExp) == kExp ? 0x0000FFFFu : 0u) | (((d >> 16) & kExp) == kExp ? 0xFFFF0000u : 0u);
  return (d & ~sp) | (((d & 0x80008000u) | (kMax * 0x00010001u)) & sp);
}
template <typename T>
__device__ __forceinline__ uint4 finite16(uint4 u) {
  return make_uint4(finite2<T>(u.x), finite2<T>(u.y), finite2<T>(u.z), finite2<T>(u.w));
}

// Key masks folded into the bias operand of the identity MFMA (bf16, row-
// shared key masks, at most kFoldTiles 64-key tiles): a masked key's bias
// element becomes -3.39e38, so its logit is -inf or below -1e38 and its P
// underflows to exactly 0 with no per-score select.  Every tile a kernel
// visits has a kept key (fully masked tiles are skipped), so each row's
// maximum is a kept key's.  Masked keys' K and V rows are still read as
// zeros, so their products stay finite.  The fold table holds, per tile and
// lane half g2, 16 dwords of 16-bit keep masks: dword (2 t2 + c) * 4 + k
// covers keys 32 t2 + 16 c + 8 g2 + 2 k and + 1, the elements of dword k of
// the bias fragment of 32-key tile t2 and chunk c.
constexpr int kFoldTiles = 16;                // Lk <= 1024
constexpr uint32_t kFoldNeg = 0xFF7FFF7Fu;    // two bf16 -3.39e38
__device__ __forceinline__ void build_fold_table(uint32_t* tab, const uint64_t* keep, int ntiles, int tid,
                                                 int nthreads) {
  for (int e = tid; e < ntiles * 32; e += nthreads) {
    const int t = e >> 5, g2 = (e >> 4) & 1, i = e & 15;
    const int key0 = 32 * (i >> 3) + 16 * ((i >> 2) & 1) + 8 * g2 + 2 * (i & 3);
    const uint64_t b = keep[t];
    tab[e] = (((b >> key0) & 1) ? 0x0000FFFFu : 0u) | (((b >> (key0 + 1)) & 1) ? 0xFFFF0000u : 0u);
  }
}
// bias fragment b with its masked keys' elements replaced (m: keep masks)
__device__ __forceinline__ uint4 fold_bias(uint4 b, uint4 m) {
  return make_uint4((b.x & m.x) | (~m.x & kFoldNeg), (b.y & m.y) | (~m.y & kFoldNeg),
                    (b.z & m.z) | (~m.z & kFoldNeg), (b.w & m.w) | (~m.w & kFoldNeg));
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

// two floats rounded to T (to nearest even) in one 32-bit word, x in the low half: a vector
// conversion, so bf16 pairs become one v_cvt_pk_bf16_f32
template <typename T>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
  typedef float F2 __attribute__((ext_vector_type(2)));
  typedef T T2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((F2){x, y}, T2));
}

// Write one 32x32 accumulator tile's 32 head-dim values (lane (col, g) holds
// acc[j] = row kappa(g, j)) to row[d0 .. d0+31], times s, for d < D (D % 8 == 0).
// The two 32-lane halves trade values through v_permlane32_swap so that the
// lower half holds d0 .. d0+15 and the upper half d0+16 .. d0+31: each lane
// then writes 32 contiguous bytes and every 64-byte row segment is written
// whole by one instruction, instead of four instructions each leaving it
// partially written (which doubles the write traffic reaching HBM).
template <typename T, typename Acc>
__device__ __forceinline__ void store_tile(T* row, int d0, int D, int g, const Acc& acc, float s) {
  uint32_t p[8];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    p[2 * q] = pack2<T>(acc[4 * q] * s, acc[4 * q + 1] * s);
    p[2 * q + 1] = pack2<T>(acc[4 * q + 2] * s, acc[4 * q + 3] * s);
  }
  // p[0..1]: d kappa(g,0..3) = 4g..4g+3; p[2..3]: 8+4g..; p[4..5]: 16+4g..; p[6..7]: 24+4g..
  const auto a = __builtin_amdgcn_permlane32_swap(p[0], p[4], false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(p[1], p[5], false, false);
  const auto c = __builtin_amdgcn_permlane32_swap(p[2], p[6], false, false);
  const auto e = __builtin_amdgcn_permlane32_swap(p[3], p[7], false, false);
  const uint4 lo = make_uint4(a[0], b[0], a[1], b[1]);  // d0 + 16g + 0 .. 7
  const uint4 hi = make_uint4(c[0], e[0], c[1], e[1]);  // d0 + 16g + 8 .. 15
  const int d = d0 + 16 * g;
  if (d + 8 <= D) *reinterpret_cast<uint4*>(row + d) = lo;
  if (d + 16 <= D) *reinterpret_cast<uint4*>(row + d + 8) = hi;
}

// ---- LDS tiles filled by direct global -> LDS loads (buffer_load ... lds).
// One such load of a wave writes 64 consecutive 16-byte slots (lane i: slot
// i).  A tile row of DP 16-bit elements spans DP/8 slots; logical 16-byte
// chunk c of row r sits in slot c ^ swz(r) of that row, so the 16 rows read
// by one 16-lane group of a fragment read (same logical chunk) land in 16
// distinct 16-byte bank groups.
template <int DP>
__device__ __forceinline__ int swz(int row) {
  static_assert(DP == 32 || DP == 64, "swizzle defined for 32- and 64-element rows");
  return (row >> (DP == 32 ? 2 : 1)) & (DP / 8 - 1);
}
// element offset of (row, col) in a swizzled tile of DP-element rows
template <int DP>
__device__ __forceinline__ int swz_off(int row, int col) {
  return row * DP + ((((col >> 3) ^ swz<DP>(row))) << 3) + (col & 7);
}
// Transposed fragment reads (lds_read_tr_frag) from a swizzled tile: the
// lane-dependent part of the two element offsets, valid for every r0 that is
// a multiple of 16 and, with 32-element rows, every c0 that is a multiple of
// 32 (then the swizzle leaves r0 * DP + c0 unchanged; 64-element rows keep
// one pair per 32-column half).
struct TrLane {
  int lo, hi;
};
template <int DP>
__device__ __forceinline__ TrLane tr_lane(int lane, int c0) {
  const int j = lane & 15;
  const int grp = lane >> 4;
  const int col = c0 + ((grp & 1) << 4) + ((j & 3) << 2);
  const int row = ((grp >> 1) << 2) + (j >> 2);
  return TrLane{swz_off<DP>(row, col) - c0, swz_off<DP>(row + 8, col) - c0};
}
template <typename T>
__device__ __forceinline__ typename Elem<T>::Frag lds_read_tr_frag_sw(const T* at, const TrLane& tl) {
  const s16x4 lo = lds_read_tr4(at + tl.lo);
  const s16x4 hi = lds_read_tr4(at + tl.hi);
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(typename Elem<T>::Frag, v);
}

// 16 bytes per lane from a buffer resource into 64 consecutive LDS slots
// starting at lds (wave-uniform); an out-of-range offset writes zeros
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, const void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds), 16, voff, soff, 0, 0);
}
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Buffer resource as four scalar dwords (the same descriptor as make_rsrc):
// the operand form of the inline-assembly load below.
__device__ __forceinline__ u32x4 rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  u32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((uint32_t)p);
  r[1] = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32)) & 0xffffu;
  r[2] = __builtin_amdgcn_readfirstlane(bytes);
  r[3] = 0x00020000u;
  return r;
}

// 16 bytes per lane from a buffer into 64 consecutive 16-byte LDS slots at
// lds (wave-uniform), like dma16, but issued through inline assembly.  The
// compiler then does not know that this load writes LDS, so it does not wait
// for it before every later LDS read it cannot prove disjoint (it cannot
// tell ring slots apart, and would wait for each step's own prefetch); the
// kernel's explicit vmcnt waits order these loads instead.  Two rules for a
// kernel that uses it: every direct-to-LDS load of the kernel goes this way
// (the compiler does not know that M0 changes), and no compiler-visible
// register load is waited for while one of these, issued after it, may be
// in flight (the compiler's count would leave it out and wait for it too).
__device__ __forceinline__ void dma16_asm(const u32x4& r, const void* lds, uint32_t voff, uint32_t soff) {
  const uint32_t m0 =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)(lds));
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(m0),
      "v"(voff), "s"(r), "s"(soff)
      : "memory", "m0");
}

// wait until at most N vector-memory operations of this wave are outstanding
template <int N>
__device__ __forceinline__ void vmem_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
}  // namespace fast
}  // namespace oops
