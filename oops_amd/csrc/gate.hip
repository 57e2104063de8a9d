// Gated output stage (gfx950): gated = round(sigmoid(logits)) * attention with
// logits = single . W^T, and its backward elementwise part.
//
// gate_projection_kernel: one workgroup = 4 waves x 32 tokens (rows) and 128
// gate channels n = h * D + d.  The channel is the MFMA row and the token the
// column, so a lane's accumulator holds 16 channels of one token; after a
// v_permlane32_swap each lane owns 16 consecutive channels of its token, which
// are one contiguous 32-byte run of the logits, of the output and (D a
// multiple of 16) of the attention row of one head.  W (shared by the four
// waves) goes through a two-buffer LDS tile of 128 channels x 64 k with
// XOR-swizzled rows; each wave reads its tokens' `single` k-fragments
// straight from global memory (every element is read once).  The epilogue
// rounds the logits to the dtype, stores them (training), rounds the sigmoid
// to the dtype and multiplies by the attention values, as the reference's
// _gate_projection_body does (oops/attention/gate/triton/kernel.py:117-180).
//
// gate_multiply_*_kernel: elementwise over [rows][H*D], 16 bytes per lane
// where the layout allows, else one element per lane; the roundings follow
// _gate_forward / _gate_backward (kernel.py:39-114).
#include <algorithm>
#include <initializer_list>
#include <type_traits>

#include "attn_fast_common.h"
#include "gate_kernels.h"

namespace oops {

using namespace fast;

namespace {

struct GateArgs {
  const void* single;
  const void* weight;
  const void* attention;
  const void* logits_in;
  const void* grad;
  void* gated;
  void* logits;
  void* grad_attention;
  void* grad_logits;
  int64_t rows, tokens, groups;
  int64_t a_sb, a_sg, a_st, a_sh, a_sd;
  int64_t s_row, w_row;
  int64_t tiles;  // projection: token tiles x channel tiles (W-resident form: token runs x channel tiles)
  int heads, width, channels;
  int tpw;  // W-resident form: token tiles per workgroup
};

GateArgs make_args(const oops_gate_geometry& g) {
  GateArgs a{};
  a.rows = g.rows;
  a.tokens = g.tokens;
  a.groups = g.groups;
  a.a_sb = g.a_sb;
  a.a_sg = g.a_sg;
  a.a_st = g.a_st;
  a.a_sh = g.a_sh;
  a.a_sd = g.a_sd;
  a.s_row = g.s_row;
  a.w_row = g.w_row;
  a.heads = g.heads;
  a.width = g.width;
  a.channels = g.channels;
  return a;
}

template <typename T>
__device__ __forceinline__ float to_f(T x) {
  return (float)x;
}
// x rounded to T and back (identity for float)
template <typename T>
__device__ __forceinline__ float rnd(float x) {
  return (float)(T)x;
}
// 1 / (1 + 2^(-x log2 e)) on the hardware exp2 and reciprocal
__device__ __forceinline__ float sigmoid_f(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// element offset of row r's attention values (head 0, d 0)
__device__ __forceinline__ int64_t att_row(const GateArgs& a, int64_t r) {
  const int64_t t = r % a.tokens, smp = r / a.tokens;
  return (smp / a.groups) * a.a_sb + (smp % a.groups) * a.a_sg + t * a.a_st;
}

// ------------------------------------------------------------------ projection
constexpr int kBM = 128;  // tokens per workgroup (32 per wave)
constexpr int kBN = 128;  // gate channels per workgroup
constexpr int kBK = 64;   // k per step
#ifndef OOPS_GATE_WGS
#define OOPS_GATE_WGS 256  // workgroups of the W-resident projection (one per CU)
#endif

// epilogue of one token tile: lane (lq, g2) of accumulator tile t owns channels n0 + 32 t + 16 g2 .. +15
// of token r; logits rounded to T (stored in training), sigmoid rounded to T, times the attention values
template <typename T, bool STORE_LOGITS>
__device__ __forceinline__ void gate_epilogue(const GateArgs& a, int64_t r, int n0, int N, int g2,
                                              const f32x16 (&acc)[4], const uint4 (&att_lo)[4],
                                              const uint4 (&att_hi)[4]) {
  T* lrow = STORE_LOGITS ? static_cast<T*>(a.logits) + r * N : nullptr;
  T* grow = static_cast<T*>(a.gated) + r * N;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    uint32_t p[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      p[2 * q] = pack2<T>(acc[t][4 * q], acc[t][4 * q + 1]);
      p[2 * q + 1] = pack2<T>(acc[t][4 * q + 2], acc[t][4 * q + 3]);
    }
    const auto x0 = __builtin_amdgcn_permlane32_swap(p[0], p[4], false, false);
    const auto x1 = __builtin_amdgcn_permlane32_swap(p[1], p[5], false, false);
    const auto x2 = __builtin_amdgcn_permlane32_swap(p[2], p[6], false, false);
    const auto x3 = __builtin_amdgcn_permlane32_swap(p[3], p[7], false, false);
    const uint4 lo = make_uint4(x0[0], x1[0], x0[1], x1[1]);  // channels +0 .. +7
    const uint4 hi = make_uint4(x2[0], x3[0], x2[1], x3[1]);  // channels +8 .. +15
    const int n = n0 + 32 * t + 16 * g2;
    if (n >= N) continue;  // N is a multiple of 16: a run is wholly in or out
    if constexpr (STORE_LOGITS) {
      *reinterpret_cast<uint4*>(lrow + n) = lo;
      *reinterpret_cast<uint4*>(lrow + n + 8) = hi;
    }
    const uint4 alo = att_lo[t];
    const uint4 ahi = att_hi[t];
    const T* le = reinterpret_cast<const T*>(&lo);
    const T* he = reinterpret_cast<const T*>(&hi);
    const T* ae = reinterpret_cast<const T*>(&alo);
    const T* be = reinterpret_cast<const T*>(&ahi);
    uint32_t o[8];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      o[e / 2] = pack2<T>(rnd<T>(sigmoid_f(to_f(le[e]))) * to_f(ae[e]), rnd<T>(sigmoid_f(to_f(le[e + 1]))) * to_f(ae[e + 1]));
      o[4 + e / 2] =
          pack2<T>(rnd<T>(sigmoid_f(to_f(he[e]))) * to_f(be[e]), rnd<T>(sigmoid_f(to_f(he[e + 1]))) * to_f(be[e + 1]));
    }
    *reinterpret_cast<uint4*>(grow + n) = make_uint4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<uint4*>(grow + n + 8) = make_uint4(o[4], o[5], o[6], o[7]);
  }
}

// the same epilogue with range-checked buffer stores and no branches (lane_off is kOut for a lane past
// the rows): the loop around it then knows how many stores are outstanding and does not drain them
template <typename T, bool STORE_LOGITS>
__device__ __forceinline__ void gate_epilogue_buf(const __amdgpu_buffer_rsrc_t& lr, const __amdgpu_buffer_rsrc_t& gr,
                                                  uint32_t lane_off, int n0, int N, int g2, const f32x16 (&acc)[4],
                                                  const uint4 (&att_lo)[4], const uint4 (&att_hi)[4]) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    uint32_t p[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      p[2 * q] = pack2<T>(acc[t][4 * q], acc[t][4 * q + 1]);
      p[2 * q + 1] = pack2<T>(acc[t][4 * q + 2], acc[t][4 * q + 3]);
    }
    uint4 lo, hi;
    trade16(p, lo, hi);  // channels n .. n + 7, n + 8 .. n + 15 of the lane's token
    const int n = n0 + 32 * t + 16 * g2;
    const uint32_t off = lane_off != kOut && n < N ? lane_off + (uint32_t)(n * 2) : kOut;
    if constexpr (STORE_LOGITS) {
      buffer_store16(lr, off, lo);
      buffer_store16(lr, off + 16, hi);
    }
    const T* le = reinterpret_cast<const T*>(&lo);
    const T* he = reinterpret_cast<const T*>(&hi);
    const T* ae = reinterpret_cast<const T*>(&att_lo[t]);
    const T* be = reinterpret_cast<const T*>(&att_hi[t]);
    uint32_t o[8];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      o[e / 2] = pack2<T>(rnd<T>(sigmoid_f(to_f(le[e]))) * to_f(ae[e]), rnd<T>(sigmoid_f(to_f(le[e + 1]))) * to_f(ae[e + 1]));
      o[4 + e / 2] =
          pack2<T>(rnd<T>(sigmoid_f(to_f(he[e]))) * to_f(be[e]), rnd<T>(sigmoid_f(to_f(he[e + 1]))) * to_f(be[e + 1]));
    }
    buffer_store16(gr, off, make_uint4(o[0], o[1], o[2], o[3]));
    buffer_store16(gr, off + 16, make_uint4(o[4], o[5], o[6], o[7]));
  }
}

template <typename T, bool STORE_LOGITS>
__global__ __launch_bounds__(256) void gate_projection_kernel(GateArgs a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int WT = kBN * kBK;  // W tile elements
  __shared__ __attribute__((aligned(16))) T w_lds[2 * WT];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int g2 = lane >> 5;
  const int N = a.heads * a.width;
  const int C = a.channels;
  const int nbn = (N + kBN - 1) / kBN;
  // the channel tiles of one token tile are neighbours in one XCD's range, so
  // the token rows they share are fetched from HBM once and met in that L2
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x, 0);
  if (tile >= a.tiles) return;
  const int bn = (int)(tile % nbn);
  const int64_t bm = tile / nbn;
  const int n0 = bn * kBN;
  const int64_t r = bm * kBM + wave * 32 + lq;  // this lane's token
  const bool rv = r < a.rows;

  // single k-fragments of this lane's token (B operand: lane = token, 8 k);
  // the resource spans the workgroup's rows, the lane's row is in the offset
  const T* s_base = static_cast<const T*>(a.single) + bm * kBM * a.s_row;
  const int64_t s_rows_left = a.rows - bm * kBM;
  const uint32_t s_bytes =
      (uint32_t)(((s_rows_left < kBM ? s_rows_left : kBM) - 1) * a.s_row * 2 + (int64_t)C * 2);
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(s_base, s_bytes);
  const uint32_t s_lane = rv ? (uint32_t)((wave * 32 + lq) * a.s_row * 2) : kOut;
  auto load_s = [&](int k0, uint4 (&sf)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int k = k0 + 16 * c + 8 * g2;
      sf[c] = buffer_load16(sr, k < C && s_lane != kOut ? s_lane + (uint32_t)(k * 2) : kOut);
    }
  };
  // W tile: 128 channels x 64 k, 4 chunks of 16 bytes per thread
  const T* w_base = static_cast<const T*>(a.weight) + (int64_t)n0 * a.w_row;
  const int w_rows = N - n0 < kBN ? N - n0 : kBN;
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(w_base, (uint32_t)(((int64_t)(w_rows - 1) * a.w_row + C) * 2));
  auto load_w = [&](int k0, uint4 (&wu)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int id = tid + 256 * j;
      const int row = id >> 3, ch = id & 7;
      const int k = k0 + ch * 8;
      wu[j] = buffer_load16(wr, row < w_rows && k < C ? (uint32_t)((row * a.w_row + k) * 2) : kOut);
    }
  };
  auto store_w = [&](int buf, const uint4 (&wu)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int id = tid + 256 * j;
      const int row = id >> 3, ch = id & 7;
      *reinterpret_cast<uint4*>(&w_lds[buf * WT + swz_off<kBK>(row, ch * 8)]) = wu[j];
    }
  };

  // the epilogue's attention runs, loaded before the k loop and unconditionally: an absent run (token
  // past the rows, channels past N) reads a valid address of row 0 and is never used, so no load waits
  // at a branch
  uint4 att_lo[4], att_hi[4];
  {
    const T* att = static_cast<const T*>(a.attention) + att_row(a, rv ? r : 0);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int n = n0 + 32 * t + 16 * g2;
      const int nn = rv && n < N ? n : 0;
      const int h = nn / a.width, d = nn - h * a.width;
      const T* arow = att + h * a.a_sh + d;
      att_lo[t] = *reinterpret_cast<const uint4*>(arow);
      att_hi[t] = *reinterpret_cast<const uint4*>(arow + 8);
    }
  }

  f32x16 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x16{};

  const int nsteps = (C + kBK - 1) / kBK;
  uint4 sf[4], sn[4], wu[4];
  load_w(0, wu);
  load_s(0, sf);
  store_w(0, wu);
  __syncthreads();
  for (int i = 0; i < nsteps; ++i) {
    const int buf = i & 1;
    const bool more = i + 1 < nsteps;
    if (more) {
      load_w((i + 1) * kBK, wu);
      load_s((i + 1) * kBK, sn);
    }
    const T* wt = &w_lds[buf * WT];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const Frag bfr = __builtin_bit_cast(Frag, sf[c]);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        acc[t] = E::mma(lds_frag<T>(wt + swz_off<kBK>(32 * t + lq, 16 * c + 8 * g2)), bfr, acc[t]);
    }
    if (more) store_w(buf ^ 1, wu);
    lds_barrier();
#pragma unroll
    for (int c = 0; c < 4; ++c) sf[c] = sn[c];
  }

  if (!rv) return;
  gate_epilogue<T, STORE_LOGITS>(a, r, n0, N, g2, acc, att_lo, att_hi);
}

// gate_projection_w_kernel (C <= 256): the same tile and epilogue, with the workgroup's W block (128
// channels x C) loaded into LDS once and kept across a run of tpw token tiles (about one workgroup per
// CU for the whole launch, so no workgroup start-up, W reload or k-step barrier per tile).  While a
// tile's MFMAs consume k-panel p of its `single` fragments, panel p of the next tile loads into the same
// registers; the tile's attention runs load before its MFMAs.  Every load is unconditional (past the
// rows it reads out of range, which returns zeros, or a valid address that is never used).
template <typename T, bool STORE_LOGITS, int NP>
__global__ __launch_bounds__(256, 2) void gate_projection_w_kernel(GateArgs a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int WT = kBN * kBK;
  extern __shared__ __attribute__((aligned(16))) char lds_raw[];
  T* w_lds = reinterpret_cast<T*>(lds_raw);

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int g2 = lane >> 5;
  const int N = a.heads * a.width;
  const int C = a.channels;
  const int nbn = (N + kBN - 1) / kBN;
  // the channel tiles of one token run are neighbours in one XCD's range and walk the same rows
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x, 0);
  if (tile >= a.tiles) return;
  const int bn = (int)(tile % nbn);
  const int64_t run = tile / nbn;
  const int n0 = bn * kBN;
  const int64_t tiles_m = (a.rows + kBM - 1) / kBM;

  {
    const T* w_base = static_cast<const T*>(a.weight) + (int64_t)n0 * a.w_row;
    const int w_rows = N - n0 < kBN ? N - n0 : kBN;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w_base, (uint32_t)(((int64_t)(w_rows - 1) * a.w_row + C) * 2));
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int id = tid + 256 * j, row = id >> 3, ch = id & 7, k = p * kBK + ch * 8;
        const uint4 u = buffer_load16(wr, row < w_rows && k < C ? (uint32_t)((row * a.w_row + k) * 2) : kOut);
        *reinterpret_cast<uint4*>(&w_lds[p * WT + swz_off<kBK>(row, ch * 8)]) = u;
      }
  }

  // token tile tm's `single` resource and this lane's row offset (kOut past the rows or the run)
  auto tile_src = [&](int64_t tm, bool live, uint32_t& lane_off) {
    const int64_t r0 = tm * kBM;
    const int64_t left = live ? a.rows - r0 : 0;
    const int nrows = (int)(left < kBM ? left : kBM);
    lane_off = wave * 32 + lq < nrows ? (uint32_t)((wave * 32 + lq) * a.s_row * 2) : kOut;
    const T* base = static_cast<const T*>(a.single) + (nrows > 0 ? r0 * a.s_row : 0);
    return make_rsrc(base, nrows > 0 ? (uint32_t)(((int64_t)(nrows - 1) * a.s_row + C) * 2) : 0u);
  };
  auto load_panel = [&](const __amdgpu_buffer_rsrc_t& sr, uint32_t lane_off, int p, uint4 (&x)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int k = p * kBK + 16 * c + 8 * g2;
      x[c] = buffer_load16(sr, k < C && lane_off != kOut ? lane_off + (uint32_t)(k * 2) : kOut);
    }
  };

  const int64_t tm0 = run * a.tpw;
  uint4 xs[NP][4];
  {
    uint32_t off;
    const __amdgpu_buffer_rsrc_t sr = tile_src(tm0, true, off);
#pragma unroll
    for (int p = 0; p < NP; ++p) load_panel(sr, off, p, xs[p]);
  }
  __syncthreads();  // W block written

  for (int it = 0; it < a.tpw; ++it) {
    const int64_t tm = tm0 + it;
    if (tm >= tiles_m) break;
    const int64_t r = tm * kBM + wave * 32 + lq;  // this lane's token
    const bool rv = r < a.rows;
    uint4 att_lo[4], att_hi[4];
    {
      const T* att = static_cast<const T*>(a.attention) + att_row(a, rv ? r : 0);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int n = n0 + 32 * t + 16 * g2;
        const int nn = rv && n < N ? n : 0;
        const int h = nn / a.width, d = nn - h * a.width;
        const T* arow = att + h * a.a_sh + d;
        att_lo[t] = *reinterpret_cast<const uint4*>(arow);
        att_hi[t] = *reinterpret_cast<const uint4*>(arow + 8);
      }
    }
    // keeps the attention loads here, ahead of the MFMAs (the compiler would otherwise sink them into the
    // epilogue, next to their first use)
    asm volatile("" ::: "memory");
    uint32_t noff;
    const __amdgpu_buffer_rsrc_t nsr = tile_src(tm + 1, it + 1 < a.tpw && tm + 1 < tiles_m, noff);
    f32x16 acc[4];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const T* wt = &w_lds[p * WT];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const Frag bfr = __builtin_bit_cast(Frag, xs[p][c]);
#pragma unroll
        for (int t = 0; t < 4; ++t)
          acc[t] = E::mma(lds_frag<T>(wt + swz_off<kBK>(32 * t + lq, 16 * c + 8 * g2)), bfr,
                          p == 0 && c == 0 ? f32x16{} : acc[t]);
      }
      load_panel(nsr, noff, p, xs[p]);  // the next tile's panel p
    }
    const int64_t r0 = tm * kBM;
    const int64_t left = a.rows - r0;
    const int nrows = (int)(left < kBM ? left : kBM);
    const uint32_t out_bytes = (uint32_t)((int64_t)nrows * N * 2);
    const __amdgpu_buffer_rsrc_t lr = make_rsrc(STORE_LOGITS ? static_cast<T*>(a.logits) + r0 * N : nullptr, out_bytes);
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(static_cast<T*>(a.gated) + r0 * N, out_bytes);
    gate_epilogue_buf<T, STORE_LOGITS>(lr, gr, rv ? (uint32_t)((wave * 32 + lq) * N * 2) : kOut, n0, N, g2, acc,
                                       att_lo, att_hi);
  }
}

// ------------------------------------------------------------------ elementwise
// VEC consecutive channels per thread (VEC = 1, or 16 bytes of T when the
// attention channels are unit-stride and every run is 16-byte aligned)
template <typename T, int VEC>
__device__ __forceinline__ void load_run(const T* p, int64_t stride, float (&x)[VEC]) {
  if constexpr (VEC == 1) {
    x[0] = to_f(p[0]);
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
    for (int i = 0; i < VEC; ++i) x[i] = to_f(e[i]);
  }
  (void)stride;
}
template <typename T, int VEC>
__device__ __forceinline__ void store_run(T* p, const float (&x)[VEC]) {
  if constexpr (VEC == 1) {
    p[0] = (T)x[0];
  } else {
    uint4 u;
    T* e = reinterpret_cast<T*>(&u);
#pragma unroll
    for (int i = 0; i < VEC; ++i) e[i] = (T)x[i];
    *reinterpret_cast<uint4*>(p) = u;
  }
}

template <typename T, int VEC>
__global__ __launch_bounds__(256) void gate_multiply_forward_kernel(GateArgs a) {
  const int N = a.heads * a.width;
  const int64_t runs = (int64_t)N / VEC;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.rows * runs) return;
  const int64_t r = idx / runs;
  const int n = (int)(idx - r * runs) * VEC;
  const int h = n / a.width, d = n - h * a.width;
  const T* ap = static_cast<const T*>(a.attention) + att_row(a, r) + h * a.a_sh + d * a.a_sd;
  float lg[VEC], at[VEC], o[VEC];
  load_run<T, VEC>(static_cast<const T*>(a.logits_in) + r * N + n, 1, lg);
  if constexpr (VEC == 1) at[0] = to_f(ap[0]);
  else load_run<T, VEC>(ap, 1, at);
#pragma unroll
  for (int i = 0; i < VEC; ++i) o[i] = rnd<T>(sigmoid_f(lg[i])) * at[i];
  store_run<T, VEC>(static_cast<T*>(a.gated) + r * N + n, o);
}

template <typename T, int VEC>
__global__ __launch_bounds__(256) void gate_multiply_backward_kernel(GateArgs a) {
  const int N = a.heads * a.width;
  const int64_t runs = (int64_t)N / VEC;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.rows * runs) return;
  const int64_t r = idx / runs;
  const int n = (int)(idx - r * runs) * VEC;
  float lg[VEC], gr[VEC], o[VEC];
  load_run<T, VEC>(static_cast<const T*>(a.logits_in) + r * N + n, 1, lg);
  load_run<T, VEC>(static_cast<const T*>(a.grad) + r * N + n, 1, gr);
  float g[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) g[i] = rnd<T>(sigmoid_f(lg[i]));
  if (a.grad_attention != nullptr) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) o[i] = gr[i] * g[i];
    store_run<T, VEC>(static_cast<T*>(a.grad_attention) + r * N + n, o);
  }
  if (a.grad_logits != nullptr) {
    const int h = n / a.width, d = n - h * a.width;
    const T* ap = static_cast<const T*>(a.attention) + att_row(a, r) + h * a.a_sh + d * a.a_sd;
    float at[VEC];
    if constexpr (VEC == 1) at[0] = to_f(ap[0]);
    else load_run<T, VEC>(ap, 1, at);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      // torch's low-precision sigmoid backward rounds every step
      const float gg = rnd<T>(gr[i] * at[i]);
      const float comp = rnd<T>(1.0f - g[i]);
      const float inter = rnd<T>(gg * comp);
      o[i] = inter * g[i];
    }
    store_run<T, VEC>(static_cast<T*>(a.grad_logits) + r * N + n, o);
  }
}

bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// VEC-wide runs are possible: unit-stride channels, runs inside one head and
// every run start 16-byte aligned
bool vec_layout(const oops_gate_geometry& g, int vec, std::initializer_list<const void*> ptrs) {
  if (vec <= 1) return false;
  const int64_t N = (int64_t)g.heads * g.width;
  if (g.a_sd != 1 || g.width % vec || N % vec) return false;
  for (int64_t s : {g.a_sb, g.a_sg, g.a_st, g.a_sh})
    if (s % vec) return false;
  for (const void* p : ptrs)
    if (!aligned16(p)) return false;
  return true;
}

template <typename F>
hipError_t by_dtype(int dtype, F&& f) {
  if (dtype == OOPS_BF16) return f(Tag<__bf16>{});
  if (dtype == OOPS_F16) return f(Tag<_Float16>{});
  return f(Tag<float>{});
}

}  // namespace

bool gate_projection_ok(const oops_gate_geometry& g, const void* single, const void* weight, const void* attention,
                        const void* gated, const void* logits) {
  if (g.dtype == OOPS_F32) return false;
  if (g.channels % 8 || g.width % 16 || g.a_sd != 1) return false;
  if (g.s_row % 8 || g.w_row % 8) return false;
  for (int64_t s : {g.a_sb, g.a_sg, g.a_st, g.a_sh})
    if (s % 8) return false;
  for (const void* p : {single, weight, attention, gated, logits})
    if (!aligned16(p)) return false;
  // 32-bit buffer offsets within one workgroup's rows and the weight block
  if ((int64_t)kBM * g.s_row * 2 >= (int64_t(1) << 31) || (int64_t)kBN * g.w_row * 2 >= (int64_t(1) << 31))
    return false;
  return true;
}

hipError_t launch_gate_projection(const oops_gate_geometry& g, const void* single, const void* weight,
                                  const void* attention, void* gated, void* logits, hipStream_t stream) {
  GateArgs a = make_args(g);
  a.single = single;
  a.weight = weight;
  a.attention = attention;
  a.gated = gated;
  a.logits = logits;
  const int64_t N = (int64_t)g.heads * g.width;
  const int64_t tiles_m = (g.rows + kBM - 1) / kBM, nbn = (N + kBN - 1) / kBN;
  const int64_t blocks = tiles_m * nbn;
  if (blocks == 0) return hipSuccess;
  if (g.channels <= 4 * kBK) {
    // W-resident form: about OOPS_GATE_WGS workgroups, each a run of token tiles of one channel tile
    const int runs_max = (int)std::max<int64_t>(1, OOPS_GATE_WGS / nbn);
    a.tpw = (int)((tiles_m + runs_max - 1) / runs_max);
    a.tiles = (tiles_m + a.tpw - 1) / a.tpw * nbn;
    const int np = (int)((g.channels + kBK - 1) / kBK);
    const size_t lds = (size_t)(np == 3 ? 4 : np) * kBN * kBK * 2;
    const int64_t grid = xcd_grid(a.tiles, 0);
    return by_dtype(g.dtype, [&](auto tag) -> hipError_t {
      using T = typename decltype(tag)::type;
      if constexpr (std::is_same<T, float>::value) {
        return hipErrorInvalidValue;
      } else {
        auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(256), lds, stream, a); };
        auto by_np = [&](auto logits_tag) {
          constexpr bool L = decltype(logits_tag)::value;
          if (np == 1)
            go(gate_projection_w_kernel<T, L, 1>);
          else if (np == 2)
            go(gate_projection_w_kernel<T, L, 2>);
          else
            go(gate_projection_w_kernel<T, L, 4>);
        };
        logits != nullptr ? by_np(std::true_type{}) : by_np(std::false_type{});
        return hipGetLastError();
      }
    });
  }
  a.tiles = blocks;
  const int64_t grid = xcd_grid(blocks, 0);
  return by_dtype(g.dtype, [&](auto tag) -> hipError_t {
    using T = typename decltype(tag)::type;
    if constexpr (std::is_same<T, float>::value) {
      return hipErrorInvalidValue;
    } else {
      if (logits != nullptr)
        hipLaunchKernelGGL((gate_projection_kernel<T, true>), dim3((unsigned)grid), dim3(256), 0, stream, a);
      else
        hipLaunchKernelGGL((gate_projection_kernel<T, false>), dim3((unsigned)grid), dim3(256), 0, stream, a);
      return hipGetLastError();
    }
  });
}

hipError_t launch_gate_multiply_forward(const oops_gate_geometry& g, const void* attention, const void* logits,
                                        void* gated, hipStream_t stream) {
  GateArgs a = make_args(g);
  a.attention = attention;
  a.logits_in = logits;
  a.gated = gated;
  const int64_t N = (int64_t)g.heads * g.width;
  return by_dtype(g.dtype, [&](auto tag) -> hipError_t {
    using T = typename decltype(tag)::type;
    constexpr int V = 16 / sizeof(T);
    const bool vec = vec_layout(g, V, {attention, logits, gated});
    const int64_t work = g.rows * (vec ? N / V : N);
    if (work == 0) return hipSuccess;
    const dim3 grid((unsigned)((work + 255) / 256));
    if (vec)
      hipLaunchKernelGGL((gate_multiply_forward_kernel<T, V>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((gate_multiply_forward_kernel<T, 1>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
  });
}

hipError_t launch_gate_multiply_backward(const oops_gate_geometry& g, const void* attention, const void* logits,
                                         const void* grad, void* grad_attention, void* grad_logits,
                                         hipStream_t stream) {
  GateArgs a = make_args(g);
  a.attention = attention;
  a.logits_in = logits;
  a.grad = grad;
  a.grad_attention = grad_attention;
  a.grad_logits = grad_logits;
  const int64_t N = (int64_t)g.heads * g.width;
  return by_dtype(g.dtype, [&](auto tag) -> hipError_t {
    using T = typename decltype(tag)::type;
    constexpr int V = 16 / sizeof(T);
    const bool vec = vec_layout(g, V, {attention, logits, grad, grad_attention, grad_logits});
    const int64_t work = g.rows * (vec ? N / V : N);
    if (work == 0) return hipSuccess;
    const dim3 grid((unsigned)((work + 255) / 256));
    if (vec)
      hipLaunchKernelGGL((gate_multiply_backward_kernel<T, V>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((gate_multiply_backward_kernel<T, 1>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
  });
}

}  // namespace oops
