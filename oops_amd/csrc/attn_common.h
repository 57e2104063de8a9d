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

// Buffer resource over `bytes` bytes at `base`: raw buffer loads through it
// return zeros for offsets at or past `bytes` instead of faulting.  Callers
// pass wave-uniform values only; they are moved to scalar registers here
// (the compiler cannot always prove uniformity of values derived from the
// geometry table and would otherwise wrap every load in a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  void* up = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(up, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}
__device__ __forceinline__ void buffer_store4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned int, v), r, byte_off, 0, 0);
}
// 16-byte range-checked store: an offset past the resource's size writes nothing, so a store needs no
// branch around it
__device__ __forceinline__ void buffer_store16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, uint4 v) {
  typedef unsigned int U4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(U4, v), r, byte_off, 0, 0);
}

// s_waitcnt vmcnt(0): wait for every outstanding vector-memory load.
__device__ __forceinline__ void vmem_wait_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Workgroup barrier for LDS producer/consumer hand-off only: waits for this
// wave's LDS operations (lgkmcnt(0)) but, unlike __syncthreads(), not for
// its outstanding global loads, so prefetches stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// gfx950 LDS transpose read (ds_read_b64_tr_b16).  Within each group of 16
// lanes, lane i receives in slot k element i % 4 of the 8-byte chunk addressed
// by lane 4k + i / 4 of its group.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
__device__ __forceinline__ s16x4 lds_read_tr4(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

// 32x32x16 MFMA k-operand of X^T from a row-major LDS tile X[row][col]
// (16-bit elements, row stride ld): lane (c = lane % 32, g = lane / 32) gets
// X[r][c0 + c] for the 8 rows r of k-slots g*8 .. g*8+7, where k-slot j maps
// to row r0 + kappa(g, j) (the accumulator row order, so accumulators feed
// the other operand directly).  Two transpose reads of four rows each.
template <typename T>
__device__ __forceinline__ typename Elem<T>::Frag lds_read_tr_frag(const T* tile, int ld, int r0, int c0, int lane) {
  const int j = lane & 15;                 // lane within its 16-lane group
  const int grp = lane >> 4;               // 0..3: (column half, k half g)
  const int col = c0 + ((grp & 1) << 4) + ((j & 3) << 2);
  const int g = grp >> 1;
  const int row = r0 + (g << 2) + (j >> 2);  // kappa(g, 0..3) + (j>>2) over 4 consecutive rows
  const s16x4 lo = lds_read_tr4(tile + row * ld + col);
  const s16x4 hi = lds_read_tr4(tile + (row + 8) * ld + col);
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(typename Elem<T>::Frag, v);
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
    // (launch grids stay below 2^31 workgroups: 32-bit division)
    const uint32_t t = (uint32_t)tile, u = (uint32_t)uniform;
    const uint32_t s = t / u;
    tile = (int64_t)(t - s * u);
    return (int)s;
  }
  for (int s = 0; s < num_samples; ++s) {
    const int64_t c = count(table[s]);
    if (tile < c) return s;
    tile -= c;
  }
  return -1;
}

__device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Group ranges ("parts") of a sample's shared-dBias reduction when every part
// should cover about part_groups groups: tiles of samples of different sizes
// then cost about the same.
__host__ __device__ __forceinline__ int parts_for(int64_t G, int64_t part_groups, int max_parts) {
  int64_t p = (G + part_groups - 1) / part_groups;
  if (p > max_parts) p = max_parts;
  if (p > G) p = G;
  return p < 1 ? 1 : (int)p;
}

// MI355X has 8 XCDs, each with its own L2; workgroup b of a launch runs on XCD
// b % 8.  xcd_tile maps b to a logical tile.  chunk == 0 (tables whose
// samples all have the same tile count): each XCD processes one contiguous
// range of logical tiles, so neighbouring tiles (which share K/V rows and
// bias blocks) meet in one L2.  chunk > 0 (ragged tables, where tiles of
// different samples cost differently): runs of `chunk` consecutive tiles are
// dealt to the XCDs in turn, so every XCD gets a like share of every sample
// (a contiguous split would give the last XCD only the largest sample's
// tiles).  xcd_grid pads the grid to what the mapping needs.
constexpr int kNumXcds = 8;
constexpr int kXcdChunk = 16;
__host__ __device__ __forceinline__ int xcd_chunk(int64_t uniform_tiles) { return uniform_tiles ? 0 : kXcdChunk; }
__host__ __device__ __forceinline__ int64_t xcd_grid(int64_t tiles, int chunk) {
  const int64_t m = (int64_t)kNumXcds * (chunk > 0 ? chunk : 1);
  return (tiles + m - 1) / m * m;
}
// (chunk is 0 or kXcdChunk; grids stay below 2^31 workgroups)
__device__ __forceinline__ int64_t xcd_tile(int64_t block, int64_t grid, int chunk) {
  const uint32_t b = (uint32_t)block, x = b % kNumXcds, j = b / kNumXcds;
  if (chunk == 0) return (int64_t)(x * ((uint32_t)grid / kNumXcds) + j);
  return (int64_t)(((j / kXcdChunk) * kNumXcds + x) * kXcdChunk + j % kXcdChunk);
}
// Heads whose D-element rows together fill one 128-byte line.
__host__ __forceinline__ int head_group(const oops_attn_geometry& geo) {
  const int bytes = geo.head_size * (geo.dtype == OOPS_F32 ? 4 : 2);
  int hg = 1;
  while (hg * 2 <= geo.num_heads && geo.num_heads % (hg * 2) == 0 && hg * 2 * bytes <= 128) hg *= 2;
  return hg;
}

}  // namespace oops
