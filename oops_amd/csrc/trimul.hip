// Triangle multiplicative update (gfx950) and the row LayerNorm it starts with.
//
// The update (oops/pair/triangle_multiplication/triton/generic.py:111-200):
//
//   xn       = LayerNorm_C(pair)                              row_norm_*_kernel
//   left/right[h][p] = mask[p] * (xn W_v^T + b_v) * sigmoid(xn W_g^T + b_g)
//                                                             trimul_factor_kernel
//   combined = left . right^T (outgoing) or left^T . right   batched GEMM (host)
//   nrm      = LayerNorm_H(combined) over the channel axis    trimul_out_norm_*_kernel
//   out      = (nrm W_o^T + b_o) * sigmoid(xn W_og^T + b_og)  trimul_output_kernel
//
// row_norm: one row per 64/LPR lanes (LPR lanes per row, 8 elements per lane
// and chunk, 16-byte accesses where the row layout allows); float32 statistics;
// the backward writes per-wave float32 partials of the affine gradients.
//
// trimul_factor_kernel: one workgroup = 4 waves x 32 tokens and 64 hidden
// channels of one factor, value and gate together (128 rows of W through a
// two-buffer XOR-swizzled LDS tile).  The token is the MFMA row, so a lane's
// accumulator holds 4 consecutive tokens of one channel: the channel-major
// factor layout the contraction reads is written 8 bytes per lane.  The
// backward recomputes both projections (K = C is short; re-reading saved
// projections would cost more HBM traffic than the MFMA work) and writes the
// value and gate-logit gradients channel-major, [4H][R], plus per-workgroup
// mask-gradient partials.
//
// trimul_out_norm: 64 (or fewer, for wide H) positions of one group per
// workgroup; the [H][positions] tile is staged through LDS so both the
// channel-major combined tensor and the token-major normalized rows are read
// and written with consecutive addresses.
//
// trimul_output_kernel: 4 waves x 32 tokens and 64 output channels; two
// K loops (K = H over the normalized combined rows with W_o, K = C over xn
// with W_og) into separate accumulators, the product in the epilogue, and a
// v_permlane32_swap so each lane stores 16 consecutive channels of its token.
// The backward recomputes both projections and writes the two gradients.
#include <algorithm>
#include <type_traits>

#include "attn_fast_common.h"
#include "trimul_kernels.h"

namespace oops {

using namespace fast;

namespace {

template <typename T>
__device__ __forceinline__ float to_f(T x) {
  return (float)x;
}
__device__ __forceinline__ float sigmoid_f(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}
template <typename T>
__device__ __forceinline__ float lo_f(uint32_t u) {
  return to_f(__builtin_bit_cast(T, (uint16_t)(u & 0xffffu)));
}
template <typename T>
__device__ __forceinline__ float hi_f(uint32_t u) {
  return to_f(__builtin_bit_cast(T, (uint16_t)(u >> 16)));
}
template <typename T>
__device__ __forceinline__ void unpack8(const uint4& u, float (&x)[8]) {
  x[0] = lo_f<T>(u.x), x[1] = hi_f<T>(u.x), x[2] = lo_f<T>(u.y), x[3] = hi_f<T>(u.y);
  x[4] = lo_f<T>(u.z), x[5] = hi_f<T>(u.z), x[6] = lo_f<T>(u.w), x[7] = hi_f<T>(u.w);
}
template <typename T>
__device__ __forceinline__ uint4 pack8(const float (&x)[8]) {
  return make_uint4(pack2<T>(x[0], x[1]), pack2<T>(x[2], x[3]), pack2<T>(x[4], x[5]), pack2<T>(x[6], x[7]));
}
// 8 consecutive elements of a 16-byte aligned run: one 16-byte access for 16-bit
// types, two for float32
template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&x)[8]) {
  if constexpr (sizeof(T) == 4) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
  } else {
    unpack8<T>(*reinterpret_cast<const uint4*>(p), x);
  }
}
template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&x)[8]) {
  if constexpr (sizeof(T) == 4) {
    reinterpret_cast<float4*>(p)[0] = make_float4(x[0], x[1], x[2], x[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(x[4], x[5], x[6], x[7]);
  } else {
    *reinterpret_cast<uint4*>(p) = pack8<T>(x);
  }
}

// ------------------------------------------------------------------ row LayerNorm
struct RowNormArgs {
  const void* x;
  const float* w;
  const float* b;
  void* y;
  float* mean;
  float* rstd;
  const void* dy;
  void* dx;
  float* dw;
  float* db;
  int64_t rows, x_row, y_row;
  int width, lpr;
  float eps;
};

template <typename T, int CH, bool VEC>
__device__ __forceinline__ void load_chunks(const T* row, bool valid, int width, int lpr, int sub, float (&x)[CH][8]) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * lpr + sub) * 8;
    if constexpr (VEC) {
      // width % 8 == 0: a chunk is wholly inside or outside the row.  The load is unconditional (an absent
      // chunk reads the row's first one and is replaced), so it does not sit behind a branch that waits
      const bool in = valid && col < width;
      load8<T>(row + (in ? col : 0), x[c]);
      if (!in) {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[c][e] = 0.f;
      }
    } else {
      // clamped (always in-bounds) loads, selected afterwards: no divergent branches around loads
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int cc = col + e < width ? col + e : width - 1;
        const float v = to_f(row[cc]);
        x[c][e] = valid && col + e < width ? v : 0.f;
      }
    }
  }
}

// per-column affine parameters for a lane's chunks (clamped indices; 1 / 0 when absent)
template <int CH>
__device__ __forceinline__ void load_affine(const float* p, float none, int width, int lpr, int sub, float (&v)[CH][8]) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * lpr + sub) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int cc = col + e < width ? col + e : width - 1;
      v[c][e] = p ? p[cc] : none;
    }
  }
}

__device__ __forceinline__ float group_sum(float s, int lpr) {
  for (int o = lpr >> 1; o > 0; o >>= 1) s += __shfl_xor(s, o);
  return s;
}

// 16-bit rows of at most 16 chunks per lane group (CH <= 2): each wave takes groups of kRowU row sets (rpw
// rows each, contiguous), the next group's chunks loading while the current one is normalized, with
// range-checked buffer loads and stores and no branches, so the loop never drains its stores
#ifndef OOPS_ROW_U
#define OOPS_ROW_U 4
#endif
constexpr int kRowU = OOPS_ROW_U;
template <typename T, int CH>
__device__ __forceinline__ void row_norm_forward_pipelined(const RowNormArgs& a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr = a.lpr, rpw = 64 / lpr;
  const int sub = lane & (lpr - 1), rw = lane / lpr;
  const int W = a.width;
  constexpr int U = kRowU / CH;
  float wv[CH][8], bv[CH][8];
  load_affine<CH>(a.w, 1.f, W, lpr, sub, wv);
  load_affine<CH>(a.b, 0.f, W, lpr, sub, bv);
  const int64_t gsize = (int64_t)U * rpw;  // rows per group
  const int64_t gstep = (int64_t)gridDim.x * 4 * gsize;
  auto group_rows = [&](int64_t base) {
    const int64_t left = a.rows - base;
    return (int)(left < 0 ? 0 : left < gsize ? left : gsize);
  };
  auto load_group = [&](int64_t base, uint4 (&raw)[U][CH]) {
    const int n = group_rows(base);
    const __amdgpu_buffer_rsrc_t xr =
        make_rsrc(static_cast<const T*>(a.x) + (n ? base : 0) * a.x_row, (uint32_t)((int64_t)n * a.x_row * 2));
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int r = u * rpw + rw, col = (c * lpr + sub) * 8;
        raw[u][c] = buffer_load16(xr, r < n && col < W ? (uint32_t)((r * a.x_row + col) * 2) : kOut);
      }
  };
  int64_t base = ((int64_t)blockIdx.x * 4 + wave) * gsize;
  uint4 raw[U][CH];
  load_group(base, raw);
  for (; base < a.rows; base += gstep) {
    uint4 cur[U][CH];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int c = 0; c < CH; ++c) cur[u][c] = raw[u][c];
    load_group(base + gstep, raw);  // the next group (out of range past the rows: no request)
    const int n = group_rows(base);
    const __amdgpu_buffer_rsrc_t yr =
        make_rsrc(static_cast<T*>(a.y) + base * a.y_row, (uint32_t)((int64_t)n * a.y_row * 2));
    const __amdgpu_buffer_rsrc_t mr = make_rsrc(a.mean + base, (uint32_t)(n * 4));
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.rstd + base, (uint32_t)(n * 4));
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = u * rpw + rw;
      float x[CH][8];
#pragma unroll
      for (int c = 0; c < CH; ++c) unpack8<T>(cur[u][c], x[c]);
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) s += x[c][e];
      const float mean = group_sum(s, lpr) / (float)W;
      float q = 0.f;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int col = (c * lpr + sub) * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = col + e < W ? x[c][e] - mean : 0.f;
          q += d * d;
        }
      }
      const float rstd = rsqrtf(group_sum(q, lpr) / (float)W + a.eps);
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int col = (c * lpr + sub) * 8;
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = col + e < W ? (x[c][e] - mean) * rstd * wv[c][e] + bv[c][e] : 0.f;
        buffer_store16(yr, r < n && col < a.y_row ? (uint32_t)((r * a.y_row + col) * 2) : kOut, pack8<T>(o));
      }
      const uint32_t so = r < n && sub == 0 ? (uint32_t)(r * 4) : kOut;
      buffer_store4(mr, so, mean);
      buffer_store4(sr, so, rstd);
    }
  }
}

template <typename T, int CH, bool VEC>
__global__ __launch_bounds__(256) void row_norm_forward_kernel(RowNormArgs a) {
  if constexpr (VEC && sizeof(T) == 2 && CH <= 2) {
    row_norm_forward_pipelined<T, CH>(a);
    return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr = a.lpr, rpw = 64 / lpr;
  const int sub = lane & (lpr - 1), rw = lane / lpr;
  const int W = a.width;
  float wv[CH][8], bv[CH][8];
  load_affine<CH>(a.w, 1.f, W, lpr, sub, wv);
  load_affine<CH>(a.b, 0.f, W, lpr, sub, bv);
  // a bounded grid walks the rows: many rows per wave keep the loads of
  // successive rows in flight (one short row per wave leaves HBM idle)
  const int64_t step = (int64_t)gridDim.x * 4 * rpw;
  for (int64_t base = ((int64_t)blockIdx.x * 4 + wave) * rpw; base < a.rows; base += step) {
    const int64_t row = base + rw;
    const bool rv = row < a.rows;
    float x[CH][8];
    load_chunks<T, CH, VEC>(static_cast<const T*>(a.x) + (rv ? row : 0) * a.x_row, rv, W, lpr, sub, x);
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) s += x[c][e];
    const float mean = group_sum(s, lpr) / (float)W;
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int col = (c * lpr + sub) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = col + e < W ? x[c][e] - mean : 0.f;
        q += d * d;
      }
    }
    const float rstd = rsqrtf(group_sum(q, lpr) / (float)W + a.eps);
    if (!rv) continue;
    T* yr = static_cast<T*>(a.y) + row * a.y_row;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int col = (c * lpr + sub) * 8;
      if (col >= a.y_row) continue;
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = col + e < W ? (x[c][e] - mean) * rstd * wv[c][e] + bv[c][e] : 0.f;
      if (VEC) {
        store8<T>(yr + col, o);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (col + e < a.y_row) yr[col + e] = (T)o[e];
      }
    }
    if (sub == 0) {
      a.mean[row] = mean;
      a.rstd[row] = rstd;
    }
  }
}

template <typename T, int CH, bool VEC>
__global__ __launch_bounds__(256) void row_norm_backward_kernel(RowNormArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr = a.lpr, rpw = 64 / lpr;
  const int sub = lane & (lpr - 1), rw = lane / lpr;
  const int W = a.width;
  const float inv_w = 1.0f / (float)W;
  float wv[CH][8];
  load_affine<CH>(a.w, 1.f, W, lpr, sub, wv);
  float dw[CH][8], db[CH][8];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) dw[c][e] = db[c][e] = 0.f;
  const int64_t step = (int64_t)gridDim.x * 4 * rpw;
  for (int64_t base = ((int64_t)blockIdx.x * 4 + wave) * rpw; base < a.rows; base += step) {
    const int64_t row = base + rw;
    const bool rv = row < a.rows;
    const int64_t rr = rv ? row : 0;
    float x[CH][8], g[CH][8];
    load_chunks<T, CH, VEC>(static_cast<const T*>(a.x) + rr * a.x_row, rv, W, lpr, sub, x);
    load_chunks<T, CH, VEC>(static_cast<const T*>(a.dy) + rr * a.y_row, rv, W, lpr, sub, g);
    const float mean = rv ? a.mean[rr] : 0.f, rstd = rv ? a.rstd[rr] : 0.f;
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int col = (c * lpr + sub) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool in = col + e < W;
        const float xh = in ? (x[c][e] - mean) * rstd : 0.f;
        const float wdy = in ? g[c][e] * wv[c][e] : 0.f;
        x[c][e] = xh;
        s1 += wdy;
        s2 += wdy * xh;
        dw[c][e] += g[c][e] * xh;
        db[c][e] += g[c][e];
      }
    }
    s1 = group_sum(s1, lpr) * inv_w;
    s2 = group_sum(s2, lpr) * inv_w;
    if (!rv) continue;
    T* dxr = static_cast<T*>(a.dx) + row * a.x_row;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int col = (c * lpr + sub) * 8;
      if (col >= W) continue;
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o[e] = rstd * (g[c][e] * wv[c][e] - s1 - x[c][e] * s2);
      if (VEC) {
        store8<T>(dxr + col, o);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (col + e < W) dxr[col + e] = (T)o[e];
      }
    }
  }
  // sum the rows this wave held, then one partial row per wave
  for (int o = lpr; o < 64; o <<= 1) {
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dw[c][e] += __shfl_xor(dw[c][e], o);
        db[c][e] += __shfl_xor(db[c][e], o);
      }
  }
  if (rw != 0) return;
  const int64_t part = (int64_t)blockIdx.x * 4 + wave;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * lpr + sub) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (col + e >= W) continue;
      if (a.dw) a.dw[part * W + col + e] = dw[c][e];
      if (a.db) a.db[part * W + col + e] = db[c][e];
    }
  }
}

// ------------------------------------------------------------------ factors
struct FactorArgs {
  const void* xn;
  const void* w;
  const float* bias;
  const float* mask;
  void* factors;
  const void* grad_factors;
  void* grad_proj;
  float* mask_parts;
  float* bias_parts;  // backward: [token groups][4H] sums of the value / gate-logit gradients
  int64_t rows, positions, groups, c_row, tiles;
  int H, cblocks, tpw;
};

constexpr int kFM = 128;  // tokens per tile (32 per wave)
constexpr int kFK = 64;   // k per panel / step
#ifndef OOPS_FACTOR_FULLW_MAX_K
#define OOPS_FACTOR_FULLW_MAX_K 256
#endif
constexpr int kFullWMaxK = OOPS_FACTOR_FULLW_MAX_K;  // the whole W block stays in LDS up to this c_row

template <typename T>
__device__ __forceinline__ void load4(const T* p, bool vec, int64_t left, float (&x)[4]) {
  if (vec) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    x[0] = lo_f<T>(u.x), x[1] = hi_f<T>(u.x), x[2] = lo_f<T>(u.y), x[3] = hi_f<T>(u.y);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = i < left ? to_f(p[i]) : 0.f;
  }
}

// One workgroup = one (factor, 64-channel block) and TPW consecutive tiles of
// 128 tokens.  FULLW (c_row <= 256): the block's 128 W rows (64 value, 64
// gate) x c_row are loaded into LDS once, as 64-wide swizzled panels, and
// every token tile reuses them with no further barrier; otherwise W streams
// through a two-buffer LDS tile per tile (TPW = 1).
// streamed W: three workgroups per CU; W kept whole in LDS: two
#ifndef OOPS_FACTOR_BWD_OCC
#define OOPS_FACTOR_BWD_OCC 3
#endif
template <typename T, bool BWD, bool FULLW>
__global__ __launch_bounds__(256, FULLW ? 2 : OOPS_FACTOR_BWD_OCC) void trimul_factor_kernel(FactorArgs a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int WT = 128 * kFK;  // one panel: 128 rows x 64 k
  extern __shared__ __attribute__((aligned(16))) char lds_raw[];
  T* w_lds = reinterpret_cast<T*>(lds_raw);

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, lq = lane & 31, g2 = lane >> 5;
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x, 0);
  if (tile >= a.tiles) return;
  const int nb = 2 * a.cblocks;
  const int fc = (int)(tile % nb);
  const int f = fc / a.cblocks, cb = fc - f * a.cblocks;
  const int64_t bmg = tile / nb;
  const int H = a.H;
  const int K = (int)a.c_row;
  const int64_t P = a.positions, R = a.rows;

  // W rows: 0..63 value channels, 64..127 gate channels of block cb, factor f
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, (uint32_t)((int64_t)4 * H * a.c_row * 2));
  auto w_row_off = [&](int row) -> int64_t {
    const int hv = cb * 64 + (row & 63);
    return hv < H ? (int64_t)(f * 2 * H + (row >= 64 ? H : 0) + hv) * a.c_row * 2 : -1;
  };
  uint32_t w_off[4];
  bool w_ok[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int id = tid + 256 * j;
    const int64_t o = w_row_off(id >> 3);
    w_ok[j] = o >= 0;
    w_off[j] = (uint32_t)((o >= 0 ? o : 0) + (id & 7) * 16);
  }
  auto load_w = [&](int k0, uint4 (&wu)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ch = (tid + 256 * j) & 7;
      wu[j] = buffer_load16(wr, w_ok[j] && k0 + ch * 8 < K ? w_off[j] + (uint32_t)(k0 * 2) : kOut);
    }
  };
  auto store_w = [&](int panel, const uint4 (&wu)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int id = tid + 256 * j;
      *reinterpret_cast<uint4*>(&w_lds[panel * WT + swz_off<kFK>(id >> 3, (id & 7) * 8)]) = wu[j];
    }
  };
  const int npanels = (K + kFK - 1) / kFK;
  if constexpr (FULLW) {
    for (int p = 0; p < npanels; ++p) {
      uint4 wu[4];
      load_w(p * kFK, wu);
      store_w(p, wu);
    }
    __syncthreads();
  }

  float bsum[2][2] = {{0.f, 0.f}, {0.f, 0.f}};  // [t][value, gate] over this lane's tokens
  const int tpw = FULLW ? a.tpw : 1;
  const uint32_t x_lane = (uint32_t)((wave * 32 + lq) * a.c_row * 2);
  // the token rows of the tile at r0 as one buffer resource; rv: this lane's row exists
  auto tile_x = [&](int64_t r0, __amdgpu_buffer_rsrc_t& xr, bool& rv) {
    const int64_t rows_left = R - r0;
    const int nrows = (int)(rows_left < kFM ? rows_left : kFM);
    xr = make_rsrc(static_cast<const T*>(a.xn) + r0 * a.c_row, (uint32_t)((int64_t)nrows * a.c_row * 2));
    rv = wave * 32 + lq < nrows;
  };
  auto load_x_of = [&](const __amdgpu_buffer_rsrc_t& xr, bool rv, int k0, uint4 (&xf)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int k = k0 + 16 * c + 8 * g2;
      xf[c] = buffer_load16(xr, rv && k < K ? x_lane + (uint32_t)(k * 2) : kOut);
    }
  };
  uint4 xf[4];
  bool prefetched = false;  // xf holds this tile's first panel, loaded during the previous epilogue
  // (group, position) of this lane's first token r0 + 32 wave + 4 g2: one 64-bit division per
  // workgroup, then stepped forward by 128 tokens per tile
  int64_t g_cur, p_cur;
  {
    const int64_t rb = bmg * tpw * kFM + wave * 32 + 4 * g2;
    g_cur = rb / P;
    p_cur = rb - g_cur * P;
  }
  const int64_t fG = (int64_t)f * a.groups;
  for (int it = 0; it < tpw; ++it) {
    const int64_t r0 = (bmg * tpw + it) * kFM;
    if (r0 >= R) break;
    __amdgpu_buffer_rsrc_t xr;
    bool rv;
    tile_x(r0, xr, rv);
    auto load_x = [&](int k0, uint4 (&dst)[4]) { load_x_of(xr, rv, k0, dst); };

    f32x16 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = f32x16{};
    uint4 xn[4], wu[4];
    if constexpr (!FULLW) {
      load_w(0, wu);
      store_w(0, wu);
    }
    if (!prefetched) load_x(0, xf);
    if constexpr (!FULLW) __syncthreads();
    for (int i = 0; i < npanels; ++i) {
      const bool more = i + 1 < npanels;
      if (more) {
        if constexpr (!FULLW) load_w((i + 1) * kFK, wu);
        load_x((i + 1) * kFK, xn);
      }
      const T* wt = &w_lds[(FULLW ? i : (i & 1)) * WT];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const Frag afr = __builtin_bit_cast(Frag, xf[c]);
#pragma unroll
        for (int t = 0; t < 4; ++t)
          acc[t] = E::mma(afr, lds_frag<T>(wt + swz_off<kFK>(32 * t + lq, 16 * c + 8 * g2)), acc[t]);
      }
      if constexpr (!FULLW) {
        if (more) store_w((i & 1) ^ 1, wu);
        lds_barrier();
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) xf[c] = xn[c];
    }
    if constexpr (FULLW) {
      // the next tile's first panel loads while this tile's epilogue runs
      const int64_t rn = r0 + kFM;
      prefetched = it + 1 < tpw && rn < R;
      if (prefetched) {
        __amdgpu_buffer_rsrc_t xr_n;
        bool rv_n;
        tile_x(rn, xr_n, rv_n);
        load_x_of(xr_n, rv_n, 0, xf);
      }
    }

    // ---- epilogue: tile t in {0, 1} holds value channel cb*64 + 32t + lq (tile t+2 its gate)
    // for tokens r0 + 32 wave + 8q + 4 g2 + i
    const bool vec4 = (P & 3) == 0;  // 4 tokens from a multiple of 4 share a group, 8-byte aligned
    // 16 tokens from a multiple of 16 share a group: the halves trade values so each lane stores 32 bytes
    const bool vec16 = (P & 15) == 0;
    const float* mask = a.mask;
    // element offset of channel 0 for the tokens 8q further on: ((f G + g) H) P + p, to which a
    // channel adds hv P
    int64_t base_q[4];
    {
      int64_t g = g_cur, p = p_cur;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        base_q[q] = (fG + g) * H * P + p;
        p += 8;
        while (p >= P) p -= P, ++g;
      }
      p_cur += kFM;
      while (p_cur >= P) p_cur -= P, ++g_cur;
    }
    // every load of the epilogue is issued before its first store (a store could alias a later
    // load, so loads interleaved with stores would each wait a full memory round trip)
    float4 keep4[4];
    uint2 dpre[2][4];
    if (vec4) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t r4 = r0 + wave * 32 + 8 * q + 4 * g2;
        keep4[q] = mask && r4 < R ? *reinterpret_cast<const float4*>(mask + r4) : make_float4(1.f, 1.f, 1.f, 1.f);
      }
      if constexpr (BWD) {
        const T* gf = static_cast<const T*>(a.grad_factors);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int hv = cb * 64 + 32 * t + lq;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t r4 = r0 + wave * 32 + 8 * q + 4 * g2;
            dpre[t][q] = hv < H && r4 < R
                             ? *reinterpret_cast<const uint2*>(gf + base_q[q] + (int64_t)hv * P)
                             : make_uint2(0, 0);
          }
        }
      }
    }
    float bvs[2], bgs[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int hv = min(cb * 64 + 32 * t + lq, H - 1);
      bvs[t] = a.bias ? a.bias[f * 2 * H + hv] : 0.f;
      bgs[t] = a.bias ? a.bias[f * 2 * H + H + hv] : 0.f;
    }
    float mp[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) mp[v] = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int hv = cb * 64 + 32 * t + lq;
      if (hv >= H) continue;
      const float bv = bvs[t], bg = bgs[t];
      // vec16: packed pairs of this lane's tokens 8q + 4 g2 .. +3 (pair 2q: first two), stored after the loop
      uint32_t po[8] = {0, 0, 0, 0, 0, 0, 0, 0}, pg[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t r4 = r0 + wave * 32 + 8 * q + 4 * g2;
        if (r4 >= R) continue;
        const int64_t left = R - r4;
        float keep[4] = {1.f, 1.f, 1.f, 1.f};
        if (vec4) {
          keep[0] = keep4[q].x, keep[1] = keep4[q].y, keep[2] = keep4[q].z, keep[3] = keep4[q].w;
        } else if (mask) {
          {
#pragma unroll
            for (int i = 0; i < 4; ++i) keep[i] = i < left ? mask[r4 + i] : 0.f;
          }
        }
        float v[4], sg[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = acc[t][4 * q + i] + bv;
          sg[i] = sigmoid_f(acc[t + 2][4 * q + i] + bg);
        }
        if constexpr (!BWD) {
          T* out = static_cast<T*>(a.factors);
          if (vec4) {
            po[2 * q] = pack2<T>(v[0] * sg[0] * keep[0], v[1] * sg[1] * keep[1]);
            po[2 * q + 1] = pack2<T>(v[2] * sg[2] * keep[2], v[3] * sg[3] * keep[3]);
            if (!vec16) {
              const int64_t off = base_q[q] + (int64_t)hv * P;
              *reinterpret_cast<uint2*>(out + off) = make_uint2(po[2 * q], po[2 * q + 1]);
            }
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if (i >= left) break;
              const int64_t g = (r4 + i) / P, p = r4 + i - g * P;
              out[((f * a.groups + g) * H + hv) * P + p] = (T)(v[i] * sg[i] * keep[i]);
            }
          }
        } else {
          const T* gf = static_cast<const T*>(a.grad_factors);
          float d[4];
          if (vec4) {
            const uint2 u = dpre[t][q];
            d[0] = lo_f<T>(u.x), d[1] = hi_f<T>(u.x), d[2] = lo_f<T>(u.y), d[3] = hi_f<T>(u.y);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              d[i] = 0.f;
              if (i < left) {
                const int64_t g = (r4 + i) / P, p = r4 + i - g * P;
                d[i] = to_f(gf[((f * a.groups + g) * H + hv) * P + p]);
              }
            }
          }
          float dv[4], dg[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            dv[i] = d[i] * keep[i] * sg[i];
            dg[i] = d[i] * keep[i] * v[i] * sg[i] * (1.f - sg[i]);
            mp[4 * q + i] += d[i] * v[i] * sg[i];
          }
          T* gp = static_cast<T*>(a.grad_proj);
          T* gv = gp + (int64_t)(f * 2 * H + hv) * R + r4;
          T* gg = gp + (int64_t)(f * 2 * H + H + hv) * R + r4;
          if (vec4) {
            po[2 * q] = pack2<T>(dv[0], dv[1]), po[2 * q + 1] = pack2<T>(dv[2], dv[3]);
            pg[2 * q] = pack2<T>(dg[0], dg[1]), pg[2 * q + 1] = pack2<T>(dg[2], dg[3]);
            if (!vec16) {
              *reinterpret_cast<uint2*>(gv) = make_uint2(po[2 * q], po[2 * q + 1]);
              *reinterpret_cast<uint2*>(gg) = make_uint2(pg[2 * q], pg[2 * q + 1]);
            }
            // the bias gradient sums the float32 values (before their rounding to the dtype)
            bsum[t][0] += (dv[0] + dv[1]) + (dv[2] + dv[3]);
            bsum[t][1] += (dg[0] + dg[1]) + (dg[2] + dg[3]);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (i < left) {
                gv[i] = (T)dv[i];
                gg[i] = (T)dg[i];
                bsum[t][0] += dv[i];
                bsum[t][1] += dg[i];
              }
          }
        }
      }
      if (vec16) {
        // lane (lq, g2) stores tokens 16 g2 .. 16 g2 + 15 of the wave's 32 (wholly in or past R);
        // the trade runs in every lane, the stores only where the tokens exist
        uint4 lo, hi, glo, ghi;
        trade16(po, lo, hi);
        if constexpr (BWD) trade16(pg, glo, ghi);
        const int64_t r16 = r0 + wave * 32 + 16 * g2;
        if (r16 < R) {
          if constexpr (!BWD) {
            // base_q[2] of an upper lane is token 20: token 16 is 4 positions before it in the same group
            T* dst = static_cast<T*>(a.factors) + (g2 ? base_q[2] - 4 : base_q[0]) + (int64_t)hv * P;
            *reinterpret_cast<uint4*>(dst) = lo;
            *reinterpret_cast<uint4*>(dst + 8) = hi;
          } else {
            T* gp = static_cast<T*>(a.grad_proj);
            T* dv16 = gp + (int64_t)(f * 2 * H + hv) * R + r16;
            T* dg16 = gp + (int64_t)(f * 2 * H + H + hv) * R + r16;
            *reinterpret_cast<uint4*>(dv16) = lo;
            *reinterpret_cast<uint4*>(dv16 + 8) = hi;
            *reinterpret_cast<uint4*>(dg16) = glo;
            *reinterpret_cast<uint4*>(dg16 + 8) = ghi;
          }
        }
      }
    }
    if constexpr (BWD) {
      if (a.mask_parts != nullptr) {
        // sum over the 32 channels of the half-wave (lanes of one g2 share tokens)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          for (int o = 1; o < 32; o <<= 1) mp[v] += __shfl_xor(mp[v], o);
        float val = 0.f;
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (v == lq) val = mp[v];
        const int64_t r = r0 + wave * 32 + 8 * (lq >> 2) + 4 * g2 + (lq & 3);
        if (lq < 16 && r < R) a.mask_parts[(int64_t)(f * a.cblocks + cb) * R + r] = val;
      }
    }
  }

  if constexpr (BWD) {
    if (a.bias_parts == nullptr) return;
    // channel sums: the two half-waves, then the four waves through LDS
    __shared__ float bred[4][2][2][32];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        bsum[t][k] += __shfl_xor(bsum[t][k], 32);
        if (g2 == 0) bred[wave][t][k][lq] = bsum[t][k];
      }
    __syncthreads();
    if (tid < 128) {
      const int t = tid >> 6, k = (tid >> 5) & 1, c = tid & 31;
      const int hv = cb * 64 + 32 * t + c;
      if (hv < H) {
        const float sum = bred[0][t][k][c] + bred[1][t][k][c] + bred[2][t][k][c] + bred[3][t][k][c];
        a.bias_parts[bmg * 4 * H + f * 2 * H + k * H + hv] = sum;
      }
    }
  }
}

// trimul_factor_v16_kernel: the factor projections for 16-bit inputs when every
// 16 consecutive tokens share a group (positions % 16 == 0) and the W block
// fits in LDS (c_row <= 256): the same work split and MFMA loop as the FULLW
// form above, with a straight-line epilogue.  A wave's 32 tokens are two
// 16-token blocks whose (group, position) are wave-uniform and stepped per tile,
// every global access of the epilogue is 8 bytes (mask: 16) per lane, and each
// lane stores 32 bytes per channel after the half-wave trade.
__device__ __forceinline__ void step_block(int64_t& g, int& p, int P, int by) {
  p += by;
  while (p >= P) p -= P, ++g;
}

#ifndef V16_PREFETCH
#define V16_PREFETCH !BWD
#endif
#ifndef V16_STAGE
#define V16_STAGE 1
#endif
#ifndef V16_FWD_OCC
#define V16_FWD_OCC 2
#endif
// NP: 64-wide k panels (K <= 64 NP; panels past K are zeros); MASKED: a token mask is given
template <typename T, bool BWD, int NP, bool MASKED>
__global__ __launch_bounds__(256, BWD ? 2 : V16_FWD_OCC) void trimul_factor_v16_kernel(FactorArgs a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int WT = 128 * kFK;
  constexpr bool STAGE = V16_STAGE && NP <= 2;
  extern __shared__ __attribute__((aligned(16))) char lds_raw[];
  T* w_lds = reinterpret_cast<T*>(lds_raw);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, lq = lane & 31, g2 = lane >> 5;
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x, 0);
  if (tile >= a.tiles) return;
  const int nb = 2 * a.cblocks;
  const int fc = (int)(tile % nb);
  const int f = fc / a.cblocks, cb = fc - f * a.cblocks;
  const int64_t bmg = tile / nb;
  const int H = a.H;
  const int K = (int)a.c_row;
  const int P = (int)a.positions;
  const int64_t R = a.rows;

  // the block's 128 W rows (64 value, 64 gate channels) x K, as 64-wide swizzled panels
  {
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, (uint32_t)((int64_t)4 * H * a.c_row * 2));
#pragma unroll
    for (int p = 0; p < NP; ++p) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int id = tid + 256 * j, row = id >> 3, ch = id & 7;
        const int hv = cb * 64 + (row & 63), k = p * kFK + ch * 8;
        const int64_t o = (int64_t)(f * 2 * H + (row >= 64 ? H : 0) + hv) * a.c_row * 2 + k * 2;
        const uint4 u = buffer_load16(wr, hv < H && k < K ? (uint32_t)o : kOut);
        *reinterpret_cast<uint4*>(&w_lds[p * WT + swz_off<kFK>(row, ch * 8)]) = u;
      }
    }
    __syncthreads();
  }

  // lane channels: tile t in {0, 1} of the accumulator holds value channel hv[t] (tile t + 2 its gate)
  int hv[2];
  bool hv_ok[2];
  float bv[2], bgl[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    hv[t] = cb * 64 + 32 * t + lq;
    hv_ok[t] = hv[t] < H;
    const int hc = hv_ok[t] ? hv[t] : H - 1;
    bv[t] = a.bias ? a.bias[f * 2 * H + hc] : 0.f;
    bgl[t] = a.bias ? -a.bias[f * 2 * H + H + hc] * kLog2e : 0.f;
  }

  const int tpw = a.tpw;
  const uint32_t x_lane = (uint32_t)((wave * 32 + lq) * a.c_row * 2);
  auto tile_x = [&](int64_t r0, __amdgpu_buffer_rsrc_t& xr, bool& rv) {
    const int64_t rows_left = R - r0;
    const int nrows = (int)(rows_left < kFM ? rows_left : kFM);
    xr = make_rsrc(static_cast<const T*>(a.xn) + r0 * a.c_row, (uint32_t)((int64_t)nrows * a.c_row * 2));
    rv = wave * 32 + lq < nrows;
  };
  auto load_x_of = [&](const __amdgpu_buffer_rsrc_t& xr, bool rv, int k0, uint4 (&xf)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int k = k0 + 16 * c + 8 * g2;
      xf[c] = buffer_load16(xr, rv && k < K ? x_lane + (uint32_t)(k * 2) : kOut);
    }
  };

  // (group, position) of the wave's two 16-token blocks, wave-uniform
  int64_t gb[2];
  int pb[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t rb = bmg * tpw * kFM + wave * 32 + 16 * h;
    gb[h] = rb / P;
    pb[h] = (int)(rb - gb[h] * P);
  }
  const int64_t fG = (int64_t)f * a.groups;
  const __amdgpu_buffer_rsrc_t mask_rs = make_rsrc(a.mask, MASKED ? (uint32_t)(R * 4) : 0u);
  float bsum[2][2] = {{0.f, 0.f}, {0.f, 0.f}};  // [t][value, gate] over this lane's tokens

  uint4 xs[2][4];  // panel i of a tile in xs[i % 2]; xs[0] may hold the next tile's first panel
  bool prefetched = false;
  // STAGE: the wave's 32 rows are loaded whole (each instruction reads 64 / (8 NP) complete rows) into
  // registers one tile ahead, then copied to the wave's own LDS rows and read back as fragments
  T* x_w = w_lds + NP * WT + wave * NP * 32 * kFK;
  uint4 xc[STAGE ? 4 * NP : 1];
  auto load_rows = [&](int64_t r0, bool live) {
    const int64_t left = live ? R - r0 - wave * 32 : 0;
    const int nrows = (int)(left < 0 ? 0 : left < 32 ? left : 32);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(static_cast<const T*>(a.xn) + (nrows ? r0 + wave * 32 : 0) * a.c_row,
                                                (uint32_t)((int64_t)nrows * a.c_row * 2));
#pragma unroll
    for (int j = 0; j < 4 * NP; ++j) {
      const int id = lane + 64 * j, row = id / (8 * NP), k = (id % (8 * NP)) * 8;
      xc[j] = buffer_load16(rr, row < nrows && k < K ? (uint32_t)((row * a.c_row + k) * 2) : kOut);
    }
  };
  if constexpr (STAGE) load_rows(bmg * tpw * kFM, true);
  for (int it = 0; it < tpw; ++it) {
    const int64_t r0 = (bmg * tpw + it) * kFM;
    if (r0 >= R) break;
    __amdgpu_buffer_rsrc_t xr;
    bool rv;
    if constexpr (STAGE) {
#pragma unroll
      for (int j = 0; j < 4 * NP; ++j) {
        const int id = lane + 64 * j, row = id / (8 * NP), ch = id % (8 * NP);
        *reinterpret_cast<uint4*>(&x_w[(ch >> 3) * 32 * kFK + swz_off<kFK>(row, (ch & 7) * 8)]) = xc[j];
      }
    } else {
      tile_x(r0, xr, rv);
      if (!prefetched) load_x_of(xr, rv, 0, xs[0]);
    }

    // the epilogue's loads go out before the MFMA loop (and before the next tile's prefetch, which
    // the epilogue must not wait for).  Accumulator entry 4q + i is token r0 + 32 wave + 8q + 4 g2 + i,
    // in block q / 2.
    const int64_t rw = r0 + wave * 32;
    const bool blk_ok[2] = {rw < R, rw + 16 < R};  // R % 16 == 0: a block is wholly in or out
    // element offsets of block h's first token in the [f][G][H][P] factor layout, channel 0
    const int64_t fbase[2] = {(fG + gb[0]) * H * P + pb[0], (fG + gb[1]) * H * P + pb[1]};
    const bool st_ok = g2 ? blk_ok[1] : blk_ok[0];  // this lane's 16 post-trade tokens exist
    // every load is unconditional (an absent block reads a valid address and is replaced afterwards), so
    // no load sits behind a branch that waits for it
    // (absent blocks read out of range: zeros, no request).  The factor layout's accesses go through a
    // window from block 0's group (block 1 is in that group or the next), so the offsets stay 32-bit.
    const int64_t fwin = (fG + gb[0]) * H * P;
    const uint32_t fwin_bytes = (uint32_t)((int64_t)4 * H * P);
    uint32_t f_off[2];  // byte offset of the lane's 16 post-trade tokens of channel hv[t] in the window
#pragma unroll
    for (int t = 0; t < 2; ++t)
      f_off[t] = hv_ok[t] && st_ok ? (uint32_t)(((g2 ? fbase[1] : fbase[0]) - fwin + (int64_t)hv[t] * P) * 2) : kOut;
    float keep[4][4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float4 k4 = make_float4(1.f, 1.f, 1.f, 1.f);
      if constexpr (MASKED)
        k4 = __builtin_bit_cast(float4, buffer_load16(mask_rs, blk_ok[q >> 1] ? (uint32_t)((rw + 8 * q + 4 * g2) * 4) : kOut));
      keep[q][0] = k4.x, keep[q][1] = k4.y, keep[q][2] = k4.z, keep[q][3] = k4.w;
    }
    // BWD: the factor gradients of the lane's 16 post-trade tokens (2 x 16 bytes per channel tile),
    // traded back to the accumulator layout in the epilogue
    uint4 dlo[2], dhi[2];
    if constexpr (BWD) {
      const T* gf = static_cast<const T*>(a.grad_factors);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bool ok = hv_ok[t] && st_ok;
        const T* src = gf + (ok ? (g2 ? fbase[1] : fbase[0]) + (int64_t)hv[t] * P : 0);
        dlo[t] = *reinterpret_cast<const uint4*>(src);
        dhi[t] = *reinterpret_cast<const uint4*>(src + 8);
        if (!ok) dlo[t] = dhi[t] = make_uint4(0, 0, 0, 0);
      }
    }

    // the next tile's rows load during this tile (after the epilogue's loads, which are waited for first)
    if constexpr (STAGE) load_rows(r0 + kFM, it + 1 < tpw);

    // the first panel starts from zero accumulators (no register clear)
    f32x16 acc[4];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      if (!STAGE && i + 1 < NP) load_x_of(xr, rv, (i + 1) * kFK, xs[(i + 1) & 1]);
      const T* wt = &w_lds[i * WT];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const Frag afr = STAGE ? lds_frag<T>(x_w + i * 32 * kFK + swz_off<kFK>(lq, 16 * c + 8 * g2))
                               : __builtin_bit_cast(Frag, xs[i & 1][c]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const Frag bfr = lds_frag<T>(wt + swz_off<kFK>(32 * t + lq, 16 * c + 8 * g2));
          // the first panel starts from zero accumulators (no register clear)
          acc[t] = E::mma(afr, bfr, i == 0 && c == 0 ? f32x16{} : acc[t]);
        }
      }
    }
    // the next tile's first panel loads while this tile's epilogue runs
    prefetched = !STAGE && V16_PREFETCH && it + 1 < tpw && r0 + kFM < R;
    if (prefetched) {
      __amdgpu_buffer_rsrc_t xr_n;
      bool rv_n;
      tile_x(r0 + kFM, xr_n, rv_n);
      load_x_of(xr_n, rv_n, 0, xs[0]);
    }

    float mp[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) mp[v] = 0.f;
    const int64_t r16 = rw + 16 * g2;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      uint32_t po[8], pg[8], pd[8];
      if constexpr (BWD) {
        // inverse of trade16: pd[2q], pd[2q + 1] hold tokens 8q + 4 g2 + (0, 1), (2, 3)
        const auto y0 = __builtin_amdgcn_permlane32_swap(dlo[t].x, dlo[t].z, false, false);
        const auto y1 = __builtin_amdgcn_permlane32_swap(dlo[t].y, dlo[t].w, false, false);
        const auto y2 = __builtin_amdgcn_permlane32_swap(dhi[t].x, dhi[t].z, false, false);
        const auto y3 = __builtin_amdgcn_permlane32_swap(dhi[t].y, dhi[t].w, false, false);
        pd[0] = y0[0], pd[1] = y1[0], pd[2] = y2[0], pd[3] = y3[0];
        pd[4] = y0[1], pd[5] = y1[1], pd[6] = y2[1], pd[7] = y3[1];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float o[4], og[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = acc[t][4 * q + i] + bv[t];
          const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(__builtin_fmaf(acc[t + 2][4 * q + i], -kLog2e, bgl[t])));
          if constexpr (!BWD) {
            o[i] = v * s * keep[q][i];
          } else {
            const uint32_t u = pd[2 * q + (i >> 1)];
            const float d = (i & 1) ? hi_f<T>(u) : lo_f<T>(u);
            const float dk = d * keep[q][i], vs = v * s;
            mp[4 * q + i] += d * vs;
            o[i] = dk * s;                      // value gradient
            og[i] = dk * vs * (1.f - s);        // gate-logit gradient
          }
        }
        po[2 * q] = pack2<T>(o[0], o[1]), po[2 * q + 1] = pack2<T>(o[2], o[3]);
        if constexpr (BWD) {
          pg[2 * q] = pack2<T>(og[0], og[1]), pg[2 * q + 1] = pack2<T>(og[2], og[3]);
          // the bias gradient sums the float32 values (before their rounding to the dtype)
          bsum[t][0] += (o[0] + o[1]) + (o[2] + o[3]);
          bsum[t][1] += (og[0] + og[1]) + (og[2] + og[3]);
        }
      }
      uint4 lo, hi;
      trade16(po, lo, hi);
      // forward: branch-free range-checked stores (absent lanes store out of range), so the wait counts of
      // the loop stay exact (the backward measured faster with its plain stores)
      if constexpr (!BWD) {
        const __amdgpu_buffer_rsrc_t fr = make_rsrc(static_cast<T*>(a.factors) + fwin, fwin_bytes);
        buffer_store16(fr, f_off[t], lo);
        buffer_store16(fr, f_off[t] + 16, hi);
      } else {
        uint4 glo, ghi;
        trade16(pg, glo, ghi);
        if (hv_ok[t] && st_ok) {
          T* gp = static_cast<T*>(a.grad_proj);
          T* dv16 = gp + (int64_t)(f * 2 * H + hv[t]) * R + r16;
          T* dg16 = dv16 + (int64_t)H * R;
          *reinterpret_cast<uint4*>(dv16) = lo;
          *reinterpret_cast<uint4*>(dv16 + 8) = hi;
          *reinterpret_cast<uint4*>(dg16) = glo;
          *reinterpret_cast<uint4*>(dg16 + 8) = ghi;
        }
      }
    }
    if constexpr (BWD && MASKED) {
      if (a.mask_parts != nullptr) {
        // sum over the 32 channels of the half-wave by recursive halving: after the steps over lane
        // bits 4..1, lane lq holds the sum for entry lq / 2 (bit 4 picks the upper 8 entries, ...)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int half = 8 >> s, bit = 16 >> s;
          // per-lane select mask (bit arithmetic, so the selection stays on the two registers)
          const uint32_t up = (lq & bit) ? 0xffffffffu : 0u;
#pragma unroll
          for (int j = 0; j < half; ++j) {
            const uint32_t x = __builtin_bit_cast(uint32_t, mp[j]), y = __builtin_bit_cast(uint32_t, mp[half + j]);
            const float keep_v = __builtin_bit_cast(float, (y & up) | (x & ~up));
            const float send = __builtin_bit_cast(float, (x & up) | (y & ~up));
            mp[j] = keep_v + __shfl_xor(send, bit);
          }
        }
        mp[0] += __shfl_xor(mp[0], 1);
        const int v = lq >> 1, q = v >> 2;
        const __amdgpu_buffer_rsrc_t mpr = make_rsrc(a.mask_parts + (int64_t)(f * a.cblocks + cb) * R, (uint32_t)(R * 4));
        buffer_store4(mpr, (lq & 1) == 0 && blk_ok[q >> 1] ? (uint32_t)((rw + 8 * q + 4 * g2 + (v & 3)) * 4) : kOut,
                      mp[0]);
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) step_block(gb[h], pb[h], P, kFM);
  }

  if constexpr (BWD) {
    if (a.bias_parts == nullptr) return;
    // channel sums: the two half-waves, then the four waves through LDS
    __shared__ float bred[4][2][2][32];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        bsum[t][k] += __shfl_xor(bsum[t][k], 32);
        if (g2 == 0) bred[wave][t][k][lq] = bsum[t][k];
      }
    __syncthreads();
    if (tid < 128) {
      const int t = tid >> 6, k = (tid >> 5) & 1, c = tid & 31;
      const int h = cb * 64 + 32 * t + c;
      if (h < H) {
        const float sum = bred[0][t][k][c] + bred[1][t][k][c] + bred[2][t][k][c] + bred[3][t][k][c];
        a.bias_parts[bmg * 4 * H + f * 2 * H + k * H + h] = sum;
      }
    }
  }
}

// ------------------------------------------------------------------ output LayerNorm (channel-major)
struct OutNormArgs {
  const void* comb;
  const float* w;
  const float* b;
  void* nrm;
  float* mean;
  float* rstd;
  const void* dn;
  void* dcomb;
  float* dw;
  float* db;
  int64_t groups, positions, h_row, pblocks;
  int H, npb;
  float eps;
};

// VEC (P % 8 == 0, and for the backward H % 8 == 0): 16-byte global accesses,
// 8 positions of one channel or 8 channels of one position per lane; else one
// element per lane.
template <typename T, bool VEC>
__device__ __forceinline__ void stage_channel_major(const T* cg, int64_t P, int H, int np, int npb, int ld, float* sm) {
  const int tid = threadIdx.x;
  if constexpr (VEC) {
    const int cpl = npb / 8;
    for (int idx = tid; idx < H * cpl; idx += 256) {
      const int h = idx / cpl, p = (idx - h * cpl) * 8;
      float v[8];
      if (p < np) {
        unpack8<T>(*reinterpret_cast<const uint4*>(cg + (int64_t)h * P + p), v);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) sm[h * ld + p + e] = v[e];
    }
  } else {
    for (int idx = tid; idx < H * npb; idx += 256) {
      const int h = idx / npb, p = idx - h * npb;
      sm[h * ld + p] = p < np ? to_f(cg[(int64_t)h * P + p]) : 0.f;
    }
  }
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void trimul_out_norm_forward_kernel(OutNormArgs a) {
  extern __shared__ float sm[];  // [H][npb + 1]
  __shared__ float red[256];
  const int npb = a.npb, ld = npb + 1, parts = 256 / npb, H = a.H;
  const int64_t g = blockIdx.x / a.pblocks, p0 = (blockIdx.x % a.pblocks) * npb;
  const int tid = threadIdx.x, pp = tid % npb, part = tid / npb;
  const int64_t P = a.positions;
  const int np = (int)(P - p0 < npb ? P - p0 : npb);
  const bool pv = pp < np;
  stage_channel_major<T, VEC>(static_cast<const T*>(a.comb) + g * H * P + p0, P, H, np, npb, ld, sm);
  __syncthreads();
  float s = 0.f;
  for (int h = part; h < H; h += parts) s += sm[h * ld + pp];
  red[tid] = s;
  __syncthreads();
  float mean = 0.f;
  for (int j = 0; j < parts; ++j) mean += red[j * npb + pp];
  mean /= (float)H;
  __syncthreads();
  float q = 0.f;
  for (int h = part; h < H; h += parts) {
    const float d = sm[h * ld + pp] - mean;
    q += d * d;
  }
  red[tid] = q;
  __syncthreads();
  float var = 0.f;
  for (int j = 0; j < parts; ++j) var += red[j * npb + pp];
  const float rstd = rsqrtf(var / (float)H + a.eps);
  for (int h = part; h < H; h += parts)
    sm[h * ld + pp] = (sm[h * ld + pp] - mean) * rstd * (a.w ? a.w[h] : 1.f) + (a.b ? a.b[h] : 0.f);
  if (part == 0 && pv) {
    a.mean[g * P + p0 + pp] = mean;
    a.rstd[g * P + p0 + pp] = rstd;
  }
  __syncthreads();
  // rows g*P + p0 .. + np - 1 are consecutive: write them as one run
  T* out = static_cast<T*>(a.nrm) + (g * P + p0) * a.h_row;
  const int hr = (int)a.h_row;
  if constexpr (VEC) {
    const int cpr = hr / 8;  // h_row is a multiple of 8
    for (int idx = tid; idx < np * cpr; idx += 256) {
      const int i = idx / cpr, h = (idx - i * cpr) * 8;
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = h + e < H ? sm[(h + e) * ld + i] : 0.f;
      *reinterpret_cast<uint4*>(out + (int64_t)i * hr + h) = pack8<T>(o);
    }
  } else {
    for (int e = tid; e < np * hr; e += 256) {
      const int i = e / hr, h = e - i * hr;
      out[e] = h < H ? (T)sm[h * ld + i] : (T)0.f;
    }
  }
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void trimul_out_norm_backward_kernel(OutNormArgs a) {
  extern __shared__ float sm[];  // x-hat [H][npb + 1], then grad [H][npb + 1]
  __shared__ float red[2][256];
  __shared__ float stat[3][64];  // rstd, s1, s2 per position
  const int npb = a.npb, ld = npb + 1, parts = 256 / npb, H = a.H;
  float* xs = sm;
  float* gs = sm + H * ld;
  const int64_t g = blockIdx.x / a.pblocks, p0 = (blockIdx.x % a.pblocks) * npb;
  const int tid = threadIdx.x, pp = tid % npb, part = tid / npb;
  const int64_t P = a.positions;
  const int np = (int)(P - p0 < npb ? P - p0 : npb);
  const bool pv = pp < np;
  // grad rows [R][H] of this block's positions are consecutive
  const T* dn = static_cast<const T*>(a.dn) + (g * P + p0) * H;
  if constexpr (VEC) {
    const int cpr = H / 8;
    for (int idx = tid; idx < npb * cpr; idx += 256) {
      const int i = idx / cpr, h = (idx - i * cpr) * 8;
      float v[8];
      if (i < np) {
        unpack8<T>(*reinterpret_cast<const uint4*>(dn + (int64_t)i * H + h), v);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) gs[(h + e) * ld + i] = v[e];
    }
  } else {
    for (int e = tid; e < npb * H; e += 256) {
      const int i = e / H, h = e - i * H;
      gs[h * ld + i] = i < np ? to_f(dn[e]) : 0.f;
    }
  }
  stage_channel_major<T, VEC>(static_cast<const T*>(a.comb) + g * H * P + p0, P, H, np, npb, ld, xs);
  if (tid < npb) {
    const bool v = tid < np;
    stat[0][tid] = v ? a.rstd[g * P + p0 + tid] : 0.f;
    red[0][tid] = v ? a.mean[g * P + p0 + tid] : 0.f;  // the mean, until the x-hat pass below
  }
  __syncthreads();
  const float mean = red[0][pp], rstd = stat[0][pp];
  __syncthreads();
  float s1 = 0.f, s2 = 0.f;
  for (int h = part; h < H; h += parts) {
    const float xh = (xs[h * ld + pp] - mean) * rstd;
    xs[h * ld + pp] = pv ? xh : 0.f;
    const float wdy = gs[h * ld + pp] * (a.w ? a.w[h] : 1.f);
    s1 += wdy;
    s2 += wdy * xh;
  }
  red[0][tid] = s1;
  red[1][tid] = s2;
  __syncthreads();
  if (tid < npb) {
    float t1 = 0.f, t2 = 0.f;
    for (int j = 0; j < parts; ++j) {
      t1 += red[0][j * npb + tid];
      t2 += red[1][j * npb + tid];
    }
    stat[1][tid] = t1 / (float)H;
    stat[2][tid] = t2 / (float)H;
  }
  __syncthreads();
  T* dc = static_cast<T*>(a.dcomb) + g * H * P + p0;
  if constexpr (VEC) {
    const int cpl = npb / 8;
    for (int idx = tid; idx < H * cpl; idx += 256) {
      const int h = idx / cpl, p = (idx - h * cpl) * 8;
      if (p >= np) continue;
      const float wh = a.w ? a.w[h] : 1.f;
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o[e] = stat[0][p + e] * (gs[h * ld + p + e] * wh - stat[1][p + e] - xs[h * ld + p + e] * stat[2][p + e]);
      *reinterpret_cast<uint4*>(dc + (int64_t)h * P + p) = pack8<T>(o);
    }
  } else if (pv) {
    for (int h = part; h < H; h += parts) {
      const float wdy = gs[h * ld + pp] * (a.w ? a.w[h] : 1.f);
      dc[(int64_t)h * P + pp] = (T)(rstd * (wdy - stat[1][pp] - xs[h * ld + pp] * stat[2][pp]));
    }
  }
  for (int h = tid; h < H; h += 256) {
    float sw = 0.f, sb = 0.f;
    for (int i = 0; i < np; ++i) {
      sw += gs[h * ld + i] * xs[h * ld + i];
      sb += gs[h * ld + i];
    }
    if (a.dw) a.dw[(int64_t)blockIdx.x * H + h] = sw;
    if (a.db) a.db[(int64_t)blockIdx.x * H + h] = sb;
  }
}

// ------------------------------------------------------------------ output LayerNorm, wave tiles
// trimul_out_norm_t_*: 16-bit pairs, H = 8 NI (NI = 4, 8 or 16), positions a multiple of 8.  Each wave owns
// tiles of TP consecutive positions (64, or 32 at H = 128) of one group and all H channels, with no
// workgroup barrier.  Lane (c = lane % CL, j = lane / CL), CL = TP / 8, holds channels h = j + JL i (JL =
// 64 / CL) of positions 8c .. 8c + 7: 16-byte loads and stores of the channel-major tensors.  Per-position
// sums run over the lane's channels and then over the JL lanes of one c (xor CL .. 32).  The token-major
// rows go through a wave-private LDS tile [H][TP] whose rows are rotated by 4 (h / 8) dwords: 16-byte
// accesses of channel rows, 2-byte column accesses of the token-major side.  Loads are unconditional
// range-checked buffer loads (positions past P read zeros), so no load sits behind a branch.
template <int TP>
__device__ __forceinline__ int tile_elem(int h, int p) {  // element offset of (channel h, position p)
  constexpr int RW = TP / 2;                              // dwords per row
  return (h * RW + (((p >> 1) + 4 * (h >> 3)) & (RW - 1))) * 2 + (p & 1);
}

// A register value the compiler must treat as redefined at this point: what is derived from it is then not
// hoisted out of the enclosing loop nor reused across passes (which would hold dozens of lane-dependent
// LDS addresses, or every unpacked element, in registers for the whole loop).
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}
template <int N>
__device__ __forceinline__ void opaque(uint4 (&u)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(u[i].x), "+v"(u[i].y), "+v"(u[i].z), "+v"(u[i].w));
}

// Orders a channel loop: the next iteration's reads and unpacking wait for this iteration's sums (so the
// compiler does not unpack every channel up front).
__device__ __forceinline__ void chain(int& z, uint4& next, float s, float t) {
  asm volatile("" : "+v"(z), "+v"(next.x), "+v"(next.y), "+v"(next.z), "+v"(next.w) : "v"(s), "v"(t));
}

template <int CL>
__device__ __forceinline__ void reduce_same_c(float (&v)[8]) {  // sums over the lanes of one c
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int o = CL; o < 64; o <<= 1) v[e] += __shfl_xor(v[e], o);
}

template <int NI>
constexpr int out_norm_tp() {
  return NI == 16 ? 32 : 64;
}

template <typename T, int NI>
__global__ __launch_bounds__(256, 2) void trimul_out_norm_t_forward_kernel(OutNormArgs a) {
  constexpr int H = 8 * NI, TP = out_norm_tp<NI>(), CL = TP / 8, JL = 64 / CL, NC = H / JL;
  __shared__ __attribute__((aligned(16))) uint16_t tile_lds[4][H * TP];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane % CL, j = lane / CL;
  uint16_t* lt = tile_lds[wave];
  const int64_t P = a.positions, tpg = (P + TP - 1) / TP, ntiles = a.groups * tpg;
  float w[NC], b[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    w[i] = a.w ? a.w[j + JL * i] : 1.f;
    b[i] = a.b ? a.b[j + JL * i] : 0.f;
  }
  constexpr float inv_h = 1.0f / H;
  for (int64_t t = (int64_t)blockIdx.x * 4 + wave; t < ntiles; t += (int64_t)gridDim.x * 4) {
    const int64_t g = t / tpg, p0 = (t - g * tpg) * TP, p = p0 + 8 * c;
    const bool pv = p < P;  // P % 8 == 0: a lane's 8 positions are wholly in or out
    const __amdgpu_buffer_rsrc_t cr = make_rsrc(static_cast<const T*>(a.comb) + g * H * P, (uint32_t)(H * P * 2));
    uint4 xu[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) xu[i] = buffer_load16(cr, pv ? (uint32_t)(((j + JL * i) * P + p) * 2) : kOut);
    float mean[8], rstd[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) mean[e] = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      float x[8];
      unpack8<T>(xu[i], x);
#pragma unroll
      for (int e = 0; e < 8; ++e) mean[e] += x[e];
    }
    reduce_same_c<CL>(mean);
#pragma unroll
    for (int e = 0; e < 8; ++e) mean[e] *= inv_h, rstd[e] = 0.f;
    opaque<NC>(xu);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      float x[8];
      unpack8<T>(xu[i], x);
#pragma unroll
      for (int e = 0; e < 8; ++e) rstd[e] += (x[e] - mean[e]) * (x[e] - mean[e]);
    }
    reduce_same_c<CL>(rstd);
#pragma unroll
    for (int e = 0; e < 8; ++e) rstd[e] = rsqrtf(rstd[e] * inv_h + a.eps);
    if (j == 0 && pv) {
      float* mo = a.mean + g * P + p;
      float* ro = a.rstd + g * P + p;
      reinterpret_cast<float4*>(mo)[0] = make_float4(mean[0], mean[1], mean[2], mean[3]);
      reinterpret_cast<float4*>(mo)[1] = make_float4(mean[4], mean[5], mean[6], mean[7]);
      reinterpret_cast<float4*>(ro)[0] = make_float4(rstd[0], rstd[1], rstd[2], rstd[3]);
      reinterpret_cast<float4*>(ro)[1] = make_float4(rstd[4], rstd[5], rstd[6], rstd[7]);
    }
    // normalized channel rows into the tile
    opaque<NC>(xu);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      float x[8];
      unpack8<T>(xu[i], x);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (x[e] - mean[e]) * rstd[e] * w[i] + b[i];
      *reinterpret_cast<uint4*>(lt + tile_elem<TP>(j + JL * i, 8 * c)) = pack8<T>(x);
    }
    // token-major rows out: instruction k writes position k (64 / NI) + lane / NI, channels 8 (lane % NI) ..
    T* dst = static_cast<T*>(a.nrm) + (g * P + p0) * a.h_row;
    const int ln = opaque(lane);
#pragma unroll
    for (int k = 0; k < TP * NI / 64; ++k) {
      const int q = k * (64 / NI) + ln / NI, m = ln % NI;
      uint32_t u[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        u[e] = (uint32_t)lt[tile_elem<TP>(8 * m + 2 * e, q)] | ((uint32_t)lt[tile_elem<TP>(8 * m + 2 * e + 1, q)] << 16);
      if (p0 + q < P) *reinterpret_cast<uint4*>(dst + q * a.h_row + 8 * m) = make_uint4(u[0], u[1], u[2], u[3]);
    }
  }
}

template <typename T, int NI>
__global__ __launch_bounds__(256, 2) void trimul_out_norm_t_backward_kernel(OutNormArgs a) {
  constexpr int H = 8 * NI, TP = out_norm_tp<NI>(), CL = TP / 8, JL = 64 / CL, NC = H / JL;
  __shared__ __attribute__((aligned(16))) uint16_t tile_lds[4][H * TP];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane % CL, j = lane / CL;
  uint16_t* lt = tile_lds[wave];
  const int64_t P = a.positions, tpg = (P + TP - 1) / TP, ntiles = a.groups * tpg;
  float w[NC], dw[NC], db[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    w[i] = a.w ? a.w[j + JL * i] : 1.f;
    dw[i] = 0.f, db[i] = 0.f;
  }
  constexpr float inv_h = 1.0f / H;
  for (int64_t t = (int64_t)blockIdx.x * 4 + wave; t < ntiles; t += (int64_t)gridDim.x * 4) {
    const int64_t g = t / tpg, p0 = (t - g * tpg) * TP, p = p0 + 8 * c;
    const bool pv = p < P;
    // the tile's grad rows [R][H] (token-major), the channel-major inputs and the statistics
    const int np = (int)(P - p0 < TP ? P - p0 : TP);
    const __amdgpu_buffer_rsrc_t dr =
        make_rsrc(static_cast<const T*>(a.dn) + (g * P + p0) * H, (uint32_t)(np * H * 2));
    uint4 du[TP * NI / 64];
#pragma unroll
    for (int k = 0; k < TP * NI / 64; ++k) {
      const int q = k * (64 / NI) + lane / NI, m = lane % NI;
      du[k] = buffer_load16(dr, (uint32_t)((q * H + 8 * m) * 2));
    }
    const __amdgpu_buffer_rsrc_t cr = make_rsrc(static_cast<const T*>(a.comb) + g * H * P, (uint32_t)(H * P * 2));
    uint4 xu[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) xu[i] = buffer_load16(cr, pv ? (uint32_t)(((j + JL * i) * P + p) * 2) : kOut);
    const __amdgpu_buffer_rsrc_t mr = make_rsrc(a.mean + g * P + p0, (uint32_t)(np * 4));
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.rstd + g * P + p0, (uint32_t)(np * 4));
    float mean[8], rstd[8];
    {
      const uint4 m0 = buffer_load16(mr, 32 * c), m1 = buffer_load16(mr, 32 * c + 16);
      const uint4 r0 = buffer_load16(rr, 32 * c), r1 = buffer_load16(rr, 32 * c + 16);
      const uint32_t mv[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
      const uint32_t rv[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) mean[e] = __builtin_bit_cast(float, mv[e]), rstd[e] = __builtin_bit_cast(float, rv[e]);
    }
    // grad rows into the tile as column writes
    const int ln = opaque(lane);
#pragma unroll
    for (int k = 0; k < TP * NI / 64; ++k) {
      const int q = k * (64 / NI) + ln / NI, m = ln % NI;
      const uint32_t v[4] = {du[k].x, du[k].y, du[k].z, du[k].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lt[tile_elem<TP>(8 * m + 2 * e, q)] = (uint16_t)(v[e] & 0xffffu);
        lt[tile_elem<TP>(8 * m + 2 * e + 1, q)] = (uint16_t)(v[e] >> 16);
      }
    }
    // x-hat, w dy and the two per-position means; the grad rows are read from the tile in both passes
    float s1[8], s2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) s1[e] = 0.f, s2[e] = 0.f;
    int z = 0;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const uint4 gu = *reinterpret_cast<const uint4*>(lt + z + tile_elem<TP>(j + JL * i, 8 * c));
      float x[8], d[8];
      unpack8<T>(xu[i], x);
      unpack8<T>(gu, d);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xh = (x[e] - mean[e]) * rstd[e], wdy = d[e] * w[i];
        s1[e] += wdy;
        s2[e] += wdy * xh;
        dw[i] += d[e] * xh;
        db[i] += d[e];
      }
      if (i + 1 < NC) chain(z, xu[i + 1], s2[7], dw[i]);
    }
    reduce_same_c<CL>(s1);
    reduce_same_c<CL>(s2);
#pragma unroll
    for (int e = 0; e < 8; ++e) s1[e] *= inv_h, s2[e] *= inv_h;
    opaque<NC>(xu);
    z = opaque(0);  // a second read of the rows, not the first one kept
    T* dc = static_cast<T*>(a.dcomb) + g * H * P + p;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const uint4 gu = *reinterpret_cast<const uint4*>(lt + z + tile_elem<TP>(j + JL * i, 8 * c));
      float x[8], d[8], o[8];
      unpack8<T>(xu[i], x);
      unpack8<T>(gu, d);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xh = (x[e] - mean[e]) * rstd[e];
        o[e] = rstd[e] * (d[e] * w[i] - s1[e] - xh * s2[e]);
      }
      if (pv) *reinterpret_cast<uint4*>(dc + (int64_t)(j + JL * i) * P) = pack8<T>(o);
      if (i + 1 < NC) chain(z, xu[i + 1], o[7], o[3]);
    }
  }
  // affine partials of this wave: sums over the CL lanes of one j
#pragma unroll
  for (int i = 0; i < NC; ++i) {
#pragma unroll
    for (int o = 1; o < CL; o <<= 1) {
      dw[i] += __shfl_xor(dw[i], o);
      db[i] += __shfl_xor(db[i], o);
    }
  }
  if (c == 0) {
    const int64_t part = (int64_t)blockIdx.x * 4 + wave;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      if (a.dw) a.dw[part * H + j + JL * i] = dw[i];
      if (a.db) a.db[part * H + j + JL * i] = db[i];
    }
  }
}

// ------------------------------------------------------------------ gated output
struct OutArgs {
  const void* nrm;
  const void* xn;
  const void* wo;
  const void* wg;
  const float* bo;
  const float* bg;
  void* out;
  const void* gout;
  void* gval;
  void* ggate;
  int64_t rows, c_row, h_row, tiles;
  int C, cblocks;
  int tpw;  // W-resident form: token tiles per workgroup
};

constexpr int kOM = 128;  // tokens per workgroup
constexpr int kON = 64;   // output channels per workgroup
constexpr int kOK = 64;   // k per step

template <typename T, bool BWD>
__global__ __launch_bounds__(256) void trimul_output_kernel(OutArgs a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int WT = kON * kOK;
  __shared__ __attribute__((aligned(16))) T w_lds[2 * WT];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, lq = lane & 31, g2 = lane >> 5;
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x, 0);
  if (tile >= a.tiles) return;
  const int cb = (int)(tile % a.cblocks);
  const int64_t r0 = (tile / a.cblocks) * kOM;
  const int c0 = cb * kON;
  const int C = a.C;
  const int64_t rows_left = a.rows - r0;
  const int nrows = (int)(rows_left < kOM ? rows_left : kOM);
  const bool rv = wave * 32 + lq < nrows;
  const int wrows = C - c0 < kON ? C - c0 : kON;
  // the block's output bias and -log2(e) x gate bias, read by the epilogue as float4 (visible after the
  // first W tile's barrier)
  __shared__ __attribute__((aligned(16))) float b_lds[2][kON];
  if (tid < 2 * kON) {
    const int ph = tid / kON, ch = c0 + tid % kON;
    const float* bsrc = ph == 0 ? a.bo : a.bg;
    const float bv = bsrc != nullptr && ch < C ? bsrc[ch] : 0.f;
    b_lds[ph][tid % kON] = ph == 0 ? bv : -bv * kLog2e;
  }
  const int64_t r = r0 + wave * 32 + lq;
  // BWD: grad_out for the lane's 16 post-swap channels n .. n + 15 of each tile t, loaded before the
  // projections (unconditionally: an absent chunk reads the row's first one and is replaced)
  uint4 gin[2][2] = {};
  if (BWD && (C & 7) == 0) {  // 16-byte rows (the element-wise path below reads its own)
    const T* grow = static_cast<const T*>(a.gout) + (rv ? r : r0) * C;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int n = c0 + 32 * t + 16 * g2;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const bool in = rv && n + 8 * hh < C;
        gin[t][hh] = *reinterpret_cast<const uint4*>(grow + (in ? n + 8 * hh : 0));
        if (!in) gin[t][hh] = make_uint4(0, 0, 0, 0);
      }
    }
  }

  f32x16 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x16{};

  // acc[2 * phase + t]: phase 0 value (K = h_row, normalized rows x W_out),
  // phase 1 gate logits (K = c_row, xn x W_gate)
#pragma unroll
  for (int phase = 0; phase < 2; ++phase) {
    const int64_t stride = phase == 0 ? a.h_row : a.c_row;
    const T* act = static_cast<const T*>(phase == 0 ? a.nrm : a.xn) + r0 * stride;
    const T* wb = static_cast<const T*>(phase == 0 ? a.wo : a.wg) + (int64_t)c0 * stride;
    const int K = (int)stride;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(act, (uint32_t)((int64_t)nrows * stride * 2));
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wb, (uint32_t)((int64_t)wrows * stride * 2));
    const uint32_t x_lane = (uint32_t)((wave * 32 + lq) * stride * 2);
    auto load_x = [&](int k0, uint4 (&xf)[4]) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int k = k0 + 16 * c + 8 * g2;
        xf[c] = buffer_load16(xr, rv && k < K ? x_lane + (uint32_t)(k * 2) : kOut);
      }
    };
    auto load_w = [&](int k0, uint4 (&wu)[2]) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int id = tid + 256 * j;
        const int row = id >> 3, k = k0 + (id & 7) * 8;
        wu[j] = buffer_load16(wr, row < wrows && k < K ? (uint32_t)((row * stride + k) * 2) : kOut);
      }
    };
    auto store_w = [&](int buf, const uint4 (&wu)[2]) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int id = tid + 256 * j;
        *reinterpret_cast<uint4*>(&w_lds[buf * WT + swz_off<kOK>(id >> 3, (id & 7) * 8)]) = wu[j];
      }
    };
    const int nsteps = (K + kOK - 1) / kOK;
    uint4 xf[4], xn[4], wu[2];
    load_w(0, wu);
    load_x(0, xf);
    store_w(0, wu);
    __syncthreads();
    for (int i = 0; i < nsteps; ++i) {
      const int buf = i & 1;
      const bool more = i + 1 < nsteps;
      if (more) {
        load_w((i + 1) * kOK, wu);
        load_x((i + 1) * kOK, xn);
      }
      const T* wt = &w_lds[buf * WT];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const Frag bfr = __builtin_bit_cast(Frag, xf[c]);
#pragma unroll
        for (int t = 0; t < 2; ++t)
          acc[2 * phase + t] =
              E::mma(lds_frag<T>(wt + swz_off<kOK>(32 * t + lq, 16 * c + 8 * g2)), bfr, acc[2 * phase + t]);
      }
      if (more) store_w(buf ^ 1, wu);
      lds_barrier();
#pragma unroll
      for (int c = 0; c < 4; ++c) xf[c] = xn[c];
    }
  }

  // ---- epilogue: lane (lq, g2) of tile t holds channels c0 + 32t + 8q + 4g2 + i of token r
  if (!rv) return;
  const bool vecc = (C & 7) == 0;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int n = c0 + 32 * t + 16 * g2;  // first of this lane's 16 channels after the swap
    float v[16], s[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 bo4 = *reinterpret_cast<const float4*>(&b_lds[0][32 * t + 8 * q + 4 * g2]);
      const float4 bg4 = *reinterpret_cast<const float4*>(&b_lds[1][32 * t + 8 * q + 4 * g2]);
      const float bo[4] = {bo4.x, bo4.y, bo4.z, bo4.w}, bgl[4] = {bg4.x, bg4.y, bg4.z, bg4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[4 * q + i] = acc[t][4 * q + i] + bo[i];
        s[4 * q + i] = __builtin_amdgcn_rcpf(
            1.0f + __builtin_amdgcn_exp2f(__builtin_fmaf(acc[2 + t][4 * q + i], -kLog2e, bgl[i])));
      }
    }
    if constexpr (!BWD) {
      uint32_t p[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        p[2 * q] = pack2<T>(v[4 * q] * s[4 * q], v[4 * q + 1] * s[4 * q + 1]);
        p[2 * q + 1] = pack2<T>(v[4 * q + 2] * s[4 * q + 2], v[4 * q + 3] * s[4 * q + 3]);
      }
      const auto x0 = __builtin_amdgcn_permlane32_swap(p[0], p[4], false, false);
      const auto x1 = __builtin_amdgcn_permlane32_swap(p[1], p[5], false, false);
      const auto x2 = __builtin_amdgcn_permlane32_swap(p[2], p[6], false, false);
      const auto x3 = __builtin_amdgcn_permlane32_swap(p[3], p[7], false, false);
      const uint4 lo = make_uint4(x0[0], x1[0], x0[1], x1[1]);
      const uint4 hi = make_uint4(x2[0], x3[0], x2[1], x3[1]);
      T* orow = static_cast<T*>(a.out) + r * C;
      if (vecc) {
        if (n < C) *reinterpret_cast<uint4*>(orow + n) = lo;
        if (n + 8 < C) *reinterpret_cast<uint4*>(orow + n + 8) = hi;
      } else {
        float e[8];
        unpack8<T>(lo, e);
        for (int j = 0; j < 8; ++j)
          if (n + j < C) orow[n + j] = (T)e[j];
        unpack8<T>(hi, e);
        for (int j = 0; j < 8; ++j)
          if (n + 8 + j < C) orow[n + 8 + j] = (T)e[j];
      }
    } else {
      // grad_out for the lane's 16 post-swap channels, swapped back to the accumulator layout
      const T* grow = static_cast<const T*>(a.gout) + r * C;
      uint4 lo, hi;
      if (vecc) {
        lo = gin[t][0];
        hi = gin[t][1];
      } else {
        float e[8];
        for (int j = 0; j < 8; ++j) e[j] = n + j < C ? to_f(grow[n + j]) : 0.f;
        lo = pack8<T>(e);
        for (int j = 0; j < 8; ++j) e[j] = n + 8 + j < C ? to_f(grow[n + 8 + j]) : 0.f;
        hi = pack8<T>(e);
      }
      const auto y0 = __builtin_amdgcn_permlane32_swap(lo.x, lo.z, false, false);
      const auto y1 = __builtin_amdgcn_permlane32_swap(lo.y, lo.w, false, false);
      const auto y2 = __builtin_amdgcn_permlane32_swap(hi.x, hi.z, false, false);
      const auto y3 = __builtin_amdgcn_permlane32_swap(hi.y, hi.w, false, false);
      const uint32_t p[8] = {y0[0], y1[0], y2[0], y3[0], y0[1], y1[1], y2[1], y3[1]};
      uint32_t pv[8], pg[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float d[4] = {lo_f<T>(p[2 * q]), hi_f<T>(p[2 * q]), lo_f<T>(p[2 * q + 1]), hi_f<T>(p[2 * q + 1])};
        float dv[4], dg[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float sv = s[4 * q + i];
          dv[i] = d[i] * sv;
          dg[i] = d[i] * v[4 * q + i] * sv * (1.f - sv);
        }
        pv[2 * q] = pack2<T>(dv[0], dv[1]);
        pv[2 * q + 1] = pack2<T>(dv[2], dv[3]);
        pg[2 * q] = pack2<T>(dg[0], dg[1]);
        pg[2 * q + 1] = pack2<T>(dg[2], dg[3]);
      }
      const int cr = (int)a.c_row;
#pragma unroll
      for (int which = 0; which < 2; ++which) {
        const uint32_t* pp = which == 0 ? pv : pg;
        const auto z0 = __builtin_amdgcn_permlane32_swap(pp[0], pp[4], false, false);
        const auto z1 = __builtin_amdgcn_permlane32_swap(pp[1], pp[5], false, false);
        const auto z2 = __builtin_amdgcn_permlane32_swap(pp[2], pp[6], false, false);
        const auto z3 = __builtin_amdgcn_permlane32_swap(pp[3], pp[7], false, false);
        T* drow = static_cast<T*>(which == 0 ? a.gval : a.ggate) + r * a.c_row;
        if (n < cr) *reinterpret_cast<uint4*>(drow + n) = make_uint4(z0[0], z1[0], z0[1], z1[1]);
        if (n + 8 < cr) *reinterpret_cast<uint4*>(drow + n + 8) = make_uint4(z2[0], z3[0], z2[1], z3[1]);
      }
    }
  }
}

// trimul_output_w_kernel: the output kernel for 16-bit rows with h_row, c_row <= 128 and C % 8 == 0.  Same
// tile, MFMAs and epilogue; both W blocks of the workgroup's 64 channels (two 64-wide k panels each) stay
// in LDS across a run of tpw token tiles (about two workgroups per CU for the launch, no W reload or k-step
// barrier per tile).  As a tile's MFMAs finish with k panel j of a projection, panel j of the next tile
// loads into the same registers; the upstream gradient (backward) loads before the MFMAs.  Loads and stores
// are range-checked buffer accesses with no branches around them (absent rows and channels use an
// out-of-range offset), so the loop never drains its outstanding stores.
#ifndef OOPS_OUTPUT_WGS
#define OOPS_OUTPUT_WGS 512
#endif
template <typename T, bool BWD>
__global__ __launch_bounds__(256, 2) void trimul_output_w_kernel(OutArgs a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int WT = kON * kOK;                              // one 64-channel x 64-k panel
  __shared__ __attribute__((aligned(16))) T w_lds[4 * WT];  // [projection][k panel]
  __shared__ __attribute__((aligned(16))) float b_lds[2][kON];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, lq = lane & 31, g2 = lane >> 5;
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x, 0);
  if (tile >= a.tiles) return;
  const int cb = (int)(tile % a.cblocks);
  const int64_t run = tile / a.cblocks;
  const int c0 = cb * kON;
  const int C = a.C;
  const int wrows = C - c0 < kON ? C - c0 : kON;
  if (tid < 2 * kON) {
    const int ph = tid / kON, ch = c0 + tid % kON;
    const float* bsrc = ph == 0 ? a.bo : a.bg;
    const float bv = bsrc != nullptr && ch < C ? bsrc[ch] : 0.f;
    b_lds[ph][tid % kON] = ph == 0 ? bv : -bv * kLog2e;
  }
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int64_t stride = p == 0 ? a.h_row : a.c_row;
    const T* wb = static_cast<const T*>(p == 0 ? a.wo : a.wg) + (int64_t)c0 * stride;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wb, (uint32_t)((int64_t)wrows * stride * 2));
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int id = tid + 256 * q, row = id >> 3, k = 64 * j + (id & 7) * 8;
        const uint4 u = buffer_load16(wr, row < wrows && k < stride ? (uint32_t)((row * stride + k) * 2) : kOut);
        *reinterpret_cast<uint4*>(&w_lds[(2 * p + j) * WT + swz_off<kOK>(row, (id & 7) * 8)]) = u;
      }
  }

  const int64_t tiles_m = (a.rows + kOM - 1) / kOM;
  // projection p's rows of token tile tm (none when !live) and this lane's row offset
  auto src = [&](int p, int64_t tm, bool live, uint32_t& off) {
    const int64_t stride = p == 0 ? a.h_row : a.c_row;
    const int64_t r0 = tm * kOM;
    const int64_t left = live ? a.rows - r0 : 0;
    const int nrows = (int)(left < 0 ? 0 : left < kOM ? left : kOM);
    off = wave * 32 + lq < nrows ? (uint32_t)((wave * 32 + lq) * stride * 2) : kOut;
    const T* act = static_cast<const T*>(p == 0 ? a.nrm : a.xn) + (nrows > 0 ? r0 * stride : 0);
    return make_rsrc(act, (uint32_t)((int64_t)nrows * stride * 2));
  };
  auto load_panel = [&](const __amdgpu_buffer_rsrc_t& sr, uint32_t off, int p, int j, uint4 (&x)[4]) {
    const int K = (int)(p == 0 ? a.h_row : a.c_row);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int k = 64 * j + 16 * c + 8 * g2;
      x[c] = buffer_load16(sr, k < K && off != kOut ? off + (uint32_t)(k * 2) : kOut);
    }
  };
  const int64_t tm0 = run * a.tpw;
  uint4 xs[4][4];  // [2 projection + k panel][fragment]
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    uint32_t off;
    const __amdgpu_buffer_rsrc_t sr = src(p, tm0, true, off);
#pragma unroll
    for (int j = 0; j < 2; ++j) load_panel(sr, off, p, j, xs[2 * p + j]);
  }
  __syncthreads();  // W blocks and biases written

  for (int it = 0; it < a.tpw; ++it) {
    const int64_t tm = tm0 + it;
    if (tm >= tiles_m) break;
    const int64_t r0 = tm * kOM;
    const int64_t left = a.rows - r0;
    const int nrows = (int)(left < kOM ? left : kOM);
    const bool rv = wave * 32 + lq < nrows;
    const uint32_t row_lane = (uint32_t)(wave * 32 + lq);
    // BWD: grad_out of the lane's 16 post-swap channels n .. n + 15 of each tile t
    uint4 gin[2][2];
    if constexpr (BWD) {
      const __amdgpu_buffer_rsrc_t gr = make_rsrc(static_cast<const T*>(a.gout) + r0 * C, (uint32_t)((int64_t)nrows * C * 2));
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int n = c0 + 32 * t + 16 * g2 + 8 * hh;
          gin[t][hh] = buffer_load16(gr, rv && n < C ? (row_lane * C + n) * 2 : kOut);
        }
      // keeps these loads ahead of the MFMAs (the compiler would sink them to their first use)
      asm volatile("" ::: "memory");
    }
    uint32_t noff[2];
    __amdgpu_buffer_rsrc_t nsr[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) nsr[p] = src(p, tm + 1, it + 1 < a.tpw && tm + 1 < tiles_m, noff[p]);

    f32x16 acc[4];  // acc[2 p + t]: projection p (0 value, 1 gate logits), channels c0 + 32 t ..
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const T* wt = &w_lds[(2 * p + j) * WT];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const Frag bfr = __builtin_bit_cast(Frag, xs[2 * p + j][c]);
#pragma unroll
          for (int t = 0; t < 2; ++t)
            acc[2 * p + t] = E::mma(lds_frag<T>(wt + swz_off<kOK>(32 * t + lq, 16 * c + 8 * g2)), bfr,
                                    j == 0 && c == 0 ? f32x16{} : acc[2 * p + t]);
        }
        load_panel(nsr[p], noff[p], p, j, xs[2 * p + j]);  // the next tile's panel
      }

    // ---- epilogue: lane (lq, g2) of tile t holds channels c0 + 32t + 8q + 4g2 + i of its token
    const int cr = (int)a.c_row;
    const __amdgpu_buffer_rsrc_t o0 = make_rsrc(
        BWD ? static_cast<void*>(static_cast<T*>(a.gval) + r0 * cr) : static_cast<void*>(static_cast<T*>(a.out) + r0 * C),
        (uint32_t)((int64_t)nrows * (BWD ? cr : C) * 2));
    const __amdgpu_buffer_rsrc_t o1 =
        make_rsrc(BWD ? static_cast<T*>(a.ggate) + r0 * cr : nullptr, BWD ? (uint32_t)((int64_t)nrows * cr * 2) : 0u);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int n = c0 + 32 * t + 16 * g2;  // first of this lane's 16 channels after the swap
      float v[16], s[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 bo4 = *reinterpret_cast<const float4*>(&b_lds[0][32 * t + 8 * q + 4 * g2]);
        const float4 bg4 = *reinterpret_cast<const float4*>(&b_lds[1][32 * t + 8 * q + 4 * g2]);
        const float bo[4] = {bo4.x, bo4.y, bo4.z, bo4.w}, bgl[4] = {bg4.x, bg4.y, bg4.z, bg4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[4 * q + i] = acc[t][4 * q + i] + bo[i];
          s[4 * q + i] = __builtin_amdgcn_rcpf(
              1.0f + __builtin_amdgcn_exp2f(__builtin_fmaf(acc[2 + t][4 * q + i], -kLog2e, bgl[i])));
        }
      }
      if constexpr (!BWD) {
        uint32_t p[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          p[2 * q] = pack2<T>(v[4 * q] * s[4 * q], v[4 * q + 1] * s[4 * q + 1]);
          p[2 * q + 1] = pack2<T>(v[4 * q + 2] * s[4 * q + 2], v[4 * q + 3] * s[4 * q + 3]);
        }
        uint4 lo, hi;
        trade16(p, lo, hi);
        const uint32_t off = rv && n < C ? (row_lane * C + n) * 2 : kOut;
        buffer_store16(o0, off, lo);
        buffer_store16(o0, rv && n + 8 < C ? off + 16 : kOut, hi);
      } else {
        const uint4 lo = gin[t][0], hi = gin[t][1];
        const auto y0 = __builtin_amdgcn_permlane32_swap(lo.x, lo.z, false, false);
        const auto y1 = __builtin_amdgcn_permlane32_swap(lo.y, lo.w, false, false);
        const auto y2 = __builtin_amdgcn_permlane32_swap(hi.x, hi.z, false, false);
        const auto y3 = __builtin_amdgcn_permlane32_swap(hi.y, hi.w, false, false);
        const uint32_t p[8] = {y0[0], y1[0], y2[0], y3[0], y0[1], y1[1], y2[1], y3[1]};
        uint32_t pv[8], pg[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float d[4] = {lo_f<T>(p[2 * q]), hi_f<T>(p[2 * q]), lo_f<T>(p[2 * q + 1]), hi_f<T>(p[2 * q + 1])};
          float dv[4], dg[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float sv = s[4 * q + i];
            dv[i] = d[i] * sv;
            dg[i] = d[i] * v[4 * q + i] * sv * (1.f - sv);
          }
          pv[2 * q] = pack2<T>(dv[0], dv[1]);
          pv[2 * q + 1] = pack2<T>(dv[2], dv[3]);
          pg[2 * q] = pack2<T>(dg[0], dg[1]);
          pg[2 * q + 1] = pack2<T>(dg[2], dg[3]);
        }
        // channels up to c_row: the padding past C receives zeros (its weights and gradient are zero)
        const uint32_t off = rv && n < cr ? (row_lane * cr + n) * 2 : kOut;
        const uint32_t off8 = rv && n + 8 < cr ? off + 16 : kOut;
        uint4 vlo, vhi, glo, ghi;
        trade16(pv, vlo, vhi);
        trade16(pg, glo, ghi);
        buffer_store16(o0, off, vlo);
        buffer_store16(o0, off8, vhi);
        buffer_store16(o1, off, glo);
        buffer_store16(o1, off8, ghi);
      }
    }
  }
}

// ------------------------------------------------------------------ output-projection gradients
// trimul_output_grad_kernel: for C = H = 128 and 16-bit rows, the products of the gated output's backward
// that share one operand X [R][128]:
//   D = X W          W [128][128]: d_normalized = grad_value W_out, d_pair = grad_gate W_gate
//   G = sum_r X^T Y  Y [R][128]:   d_W_out = grad_value^T normalized, d_W_gate = grad_gate^T xn
//   S = sum_r X      the output and gate bias gradients
// One workgroup = 8 waves walking TPW tiles of 128 rows; the X and Y tiles sit in LDS as 64-element row
// halves with XOR-swizzled 16-byte chunks, the next tile's rows in registers meanwhile.  Waves 0-3 compute
// D: wave w holds the W^T fragments of columns 32w .. 32w + 31 in registers (staged through LDS once) and
// produces those columns for the tile's rows, the row being the MFMA column, so after the half-wave trade
// each lane stores 32 bytes of one D row.  Waves 4-7 accumulate G and S: wave 4 + v rows 32v .. 32v + 31 of
// G (X columns) over all of the workgroup's tiles, X^T and Y read with the LDS transpose read (within a
// 16-row slab the row order of the sum is that read's, the same for both operands), S as one more MFMA
// against an all-ones operand.  Per-workgroup partials of G and S, summed by oops_sum_partials.
constexpr int kGT = 128;  // rows per tile
constexpr int kGN = 128;  // width of X, W, Y and D

struct GradArgs {
  const void* x;
  const void* w;
  const void* y;
  void* d;
  float* g_parts;
  float* s_parts;
  int64_t rows, x_row, w_row, y_row, d_row;
  int tpw;
};

// element offset of (row r, column c) in a tile of `rows` rows stored as two 64-element halves
__device__ __forceinline__ int half_off(int rows, int r, int c) { return (c >> 6) * rows * 64 + swz_off<64>(r, c & 63); }

template <typename T>
__global__ __launch_bounds__(512, 2) void trimul_output_grad_kernel(GradArgs a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  __shared__ __attribute__((aligned(16))) T x_lds[kGT * kGN];  // X tile [r][c] (first: W^T [n][c])
  __shared__ __attribute__((aligned(16))) T y_lds[kGT * kGN];  // Y tile [r][n]
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, lq = lane & 31, g2 = lane >> 5;
  const int64_t R = a.rows;
  const int64_t tile0 = (int64_t)blockIdx.x * a.tpw;

  // W^T through x_lds: each thread reads 16-byte chunks of W rows and writes their elements transposed
  {
    const T* w = static_cast<const T*>(a.w);
    uint16_t* wt16 = reinterpret_cast<uint16_t*>(x_lds);
#pragma unroll
    for (int it = 0; it < kGN * kGN / 8 / 512; ++it) {
      const int id = tid + 512 * it, c = id >> 4, n0 = (id & 15) * 8;
      const uint4 u = *reinterpret_cast<const uint4*>(w + (int64_t)c * a.w_row + n0);
      const uint32_t v[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        wt16[half_off(kGN, n0 + 2 * e, c)] = (uint16_t)(v[e] & 0xffffu);
        wt16[half_off(kGN, n0 + 2 * e + 1, c)] = (uint16_t)(v[e] >> 16);
      }
    }
  }
  // a tile's X and Y rows: 128 rows x 16 chunks each, 4 chunks per thread (rows past R read zeros)
  auto load_tile = [&](int64_t t, uint4 (&xr)[4], uint4 (&yr)[4]) {
    const int64_t r0 = t * kGT;
    const int64_t left = R - r0;
    const int nrows = (int)(left < 0 ? 0 : left < kGT ? left : kGT);
    const __amdgpu_buffer_rsrc_t xs =
        make_rsrc(static_cast<const T*>(a.x) + (nrows ? r0 : 0) * a.x_row, (uint32_t)(nrows * a.x_row * 2));
    const __amdgpu_buffer_rsrc_t ys =
        make_rsrc(static_cast<const T*>(a.y) + (nrows ? r0 : 0) * a.y_row, (uint32_t)(nrows * a.y_row * 2));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int id = tid + 512 * k, r = id >> 4, ch = (id & 15) * 8;
      xr[k] = buffer_load16(xs, r < nrows ? (uint32_t)((r * a.x_row + ch) * 2) : kOut);
      yr[k] = buffer_load16(ys, r < nrows ? (uint32_t)((r * a.y_row + ch) * 2) : kOut);
    }
  };
  // barrier, the prefetched rows into the tiles, the next tile's loads, barrier; false past the rows
  uint4 xr[4], yr[4];
  auto stage = [&](int it) {
    const int64_t r0 = (tile0 + it) * kGT;
    if (r0 >= R) return false;
    __syncthreads();  // the previous tile's reads are done
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int id = tid + 512 * k, r = id >> 4, ch = (id & 15) * 8;
      *reinterpret_cast<uint4*>(&x_lds[half_off(kGT, r, ch)]) = xr[k];
      *reinterpret_cast<uint4*>(&y_lds[half_off(kGT, r, ch)]) = yr[k];
    }
    if (it + 1 < a.tpw) load_tile(tile0 + it + 1, xr, yr);  // in flight during this tile
    __syncthreads();
    return true;
  };

  if (wave < 4) {
    // ---- D: this wave's W^T fragments (columns 32 wave + lq, k = 16 ks + 8 g2 ..), then per tile the
    // columns 32 wave + 8q + 4 g2 + i of rows r0 + 32 tt + lq
    Frag wf[kGN / 16];
    __syncthreads();  // W^T written
#pragma unroll
    for (int ks = 0; ks < kGN / 16; ++ks) wf[ks] = lds_frag<T>(&x_lds[half_off(kGN, 32 * wave + lq, 16 * ks + 8 * g2)]);
    load_tile(tile0, xr, yr);
    for (int it = 0; it < a.tpw; ++it) {
      if (!stage(it)) break;
      const int64_t r0 = (tile0 + it) * kGT;
      f32x16 dacc[kGT / 32];
#pragma unroll
      for (int tt = 0; tt < kGT / 32; ++tt) dacc[tt] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < kGN / 16; ++ks)
#pragma unroll
        for (int tt = 0; tt < kGT / 32; ++tt)
          dacc[tt] = E::mma(wf[ks], lds_frag<T>(&x_lds[half_off(kGT, 32 * tt + lq, 16 * ks + 8 * g2)]), dacc[tt]);
#pragma unroll
      for (int tt = 0; tt < kGT / 32; ++tt) {
        uint32_t p[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          p[2 * q] = pack2<T>(dacc[tt][4 * q], dacc[tt][4 * q + 1]);
          p[2 * q + 1] = pack2<T>(dacc[tt][4 * q + 2], dacc[tt][4 * q + 3]);
        }
        uint4 lo, hi;
        trade16(p, lo, hi);  // columns 32 wave + 16 g2 .. + 15
        const int64_t row = r0 + 32 * tt + lq;
        if (row < R) {
          T* dst = static_cast<T*>(a.d) + row * a.d_row + 32 * wave + 16 * g2;
          *reinterpret_cast<uint4*>(dst) = lo;
          *reinterpret_cast<uint4*>(dst + 8) = hi;
        }
      }
    }
  } else {
    // ---- G and S: rows 32 v .. + 31 (X columns), over each tile's rows in slabs of 16
    const int v = wave - 4;
    Frag ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = (T)1.0f;
    f32x16 gacc[kGN / 32], sacc = f32x16{};
#pragma unroll
    for (int nb = 0; nb < kGN / 32; ++nb) gacc[nb] = f32x16{};
    __syncthreads();  // W^T written (the D waves read it before the first tile overwrites it)
    load_tile(tile0, xr, yr);
    const TrLane tx = tr_lane<64>(lane, (32 * v) & 63);
    const T* xa = x_lds + ((32 * v) >> 6) * kGT * 64 + ((32 * v) & 63);
    for (int it = 0; it < a.tpw; ++it) {
      if (!stage(it)) break;
#pragma unroll
      for (int ks = 0; ks < kGT / 16; ++ks) {
        const Frag af = lds_read_tr_frag_sw<T>(xa + 16 * ks * 64, tx);
#pragma unroll
        for (int nb = 0; nb < kGN / 32; ++nb) {
          const TrLane ty = tr_lane<64>(lane, (32 * nb) & 63);
          const Frag bf = lds_read_tr_frag_sw<T>(y_lds + ((32 * nb) >> 6) * kGT * 64 + 16 * ks * 64 + ((32 * nb) & 63), ty);
          gacc[nb] = E::mma(af, bf, gacc[nb]);
        }
        sacc = E::mma(af, ones, sacc);
      }
    }
    // partials: gacc[nb] lane (lq, g2) holds G[32 v + 8q + 4 g2 + i][32 nb + lq]; every column of sacc holds
    // S[32 v + 8q + 4 g2 + i]
    float* gp = a.g_parts + (int64_t)blockIdx.x * kGN * kGN;
#pragma unroll
    for (int nb = 0; nb < kGN / 32; ++nb)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i) gp[(32 * v + 8 * q + 4 * g2 + i) * kGN + 32 * nb + lq] = gacc[nb][4 * q + i];
    if (lq == 0) {
      float* sp = a.s_parts + (int64_t)blockIdx.x * kGN;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i) sp[32 * v + 8 * q + 4 * g2 + i] = sacc[4 * q + i];
    }
  }
}

template <typename F>
hipError_t by_half(int dtype, F&& f) {
  if (dtype == OOPS_BF16) return f(__bf16{});
  if (dtype == OOPS_F16) return f(_Float16{});
  return hipErrorInvalidValue;
}

}  // namespace

// ------------------------------------------------------------------ launchers
namespace {
struct RowPlan {
  int lpr, ch, blocks;
  bool vec;
};
RowPlan row_plan(const oops_row_norm_geometry& g, bool backward, const void* const* ptrs, int nptr) {
  const int64_t span = g.y_row > g.width ? g.y_row : g.width;
  const int64_t chunks = (span + 7) / 8;
  int lpr = 1;
  while (lpr < 64 && lpr < chunks) lpr *= 2;
  int ch = 1;
  while ((int64_t)ch * lpr < chunks) ch *= 2;
  bool vec = g.width % 8 == 0 && g.x_row % 8 == 0 && g.y_row % 8 == 0;
  for (int i = 0; i < nptr; ++i)
    if (ptrs[i] && reinterpret_cast<uintptr_t>(ptrs[i]) % 16 != 0) vec = false;
  const int rpw = 64 / lpr;
  // the pipelined forward (16-bit rows, vector layout, CH <= 2) takes kRowU / CH row sets per wave and step
  const int per_wave = !backward && vec && g.dtype != OOPS_F32 && ch <= 2 ? rpw * (kRowU / ch) : rpw;
  int64_t blocks = (g.rows + 4 * per_wave - 1) / (4 * per_wave);
  if (blocks > 1024) blocks = 1024;  // both kernels walk the rows with a bounded grid
  return {lpr, ch, (int)blocks, vec};
}

template <typename T, int CH>
hipError_t launch_rows(bool backward, bool vec, int blocks, const RowNormArgs& a, hipStream_t stream) {
  if (backward) {
    if (vec)
      hipLaunchKernelGGL((row_norm_backward_kernel<T, CH, true>), dim3(blocks), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((row_norm_backward_kernel<T, CH, false>), dim3(blocks), dim3(256), 0, stream, a);
  } else {
    if (vec)
      hipLaunchKernelGGL((row_norm_forward_kernel<T, CH, true>), dim3(blocks), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((row_norm_forward_kernel<T, CH, false>), dim3(blocks), dim3(256), 0, stream, a);
  }
  return hipGetLastError();
}

template <typename F>
hipError_t by_any(int dtype, F&& f) {
  if (dtype == OOPS_F32) return f(float{});
  return by_half(dtype, f);
}

hipError_t run_rows(const oops_row_norm_geometry& g, bool backward, RowNormArgs& a, const RowPlan& pl,
                    hipStream_t stream) {
  a.rows = g.rows;
  a.x_row = g.x_row;
  a.y_row = g.y_row;
  a.width = g.width;
  a.lpr = pl.lpr;
  a.eps = g.eps;
  if (g.rows == 0) return hipSuccess;
  return by_any(g.dtype, [&](auto tag) -> hipError_t {
    using T = decltype(tag);
    switch (pl.ch) {
      case 1: return launch_rows<T, 1>(backward, pl.vec, pl.blocks, a, stream);
      case 2: return launch_rows<T, 2>(backward, pl.vec, pl.blocks, a, stream);
      case 4: return launch_rows<T, 4>(backward, pl.vec, pl.blocks, a, stream);
      case 8: return launch_rows<T, 8>(backward, pl.vec, pl.blocks, a, stream);
      case 16: return launch_rows<T, 16>(backward, pl.vec, pl.blocks, a, stream);  // widths above 4096
      default: return hipErrorInvalidValue;
    }
  });
}
}  // namespace

hipError_t launch_layer_norm_rows_forward(const oops_row_norm_geometry& g, const void* x, const float* weight,
                                          const float* bias, void* y, float* mean, float* rstd, hipStream_t stream) {
  RowNormArgs a{};
  a.x = x, a.w = weight, a.b = bias, a.y = y, a.mean = mean, a.rstd = rstd;
  const void* ptrs[] = {x, y};
  return run_rows(g, false, a, row_plan(g, false, ptrs, 2), stream);
}

int64_t layer_norm_rows_parts(const oops_row_norm_geometry& g) {
  const void* ptrs[] = {nullptr};
  return (int64_t)row_plan(g, true, ptrs, 0).blocks * 4;
}

hipError_t launch_layer_norm_rows_backward(const oops_row_norm_geometry& g, const void* x, const float* weight,
                                           const float* mean, const float* rstd, const void* grad_y, void* grad_x,
                                           float* grad_weight_parts, float* grad_bias_parts, hipStream_t stream) {
  RowNormArgs a{};
  a.x = x, a.w = weight, a.mean = const_cast<float*>(mean), a.rstd = const_cast<float*>(rstd);
  a.dy = grad_y, a.dx = grad_x, a.dw = grad_weight_parts, a.db = grad_bias_parts;
  const void* ptrs[] = {x, grad_y, grad_x};
  return run_rows(g, true, a, row_plan(g, true, ptrs, 3), stream);
}

namespace {
int64_t factor_cblocks(const oops_trimul_geometry& g) { return (g.hidden + 63) / 64; }
}  // namespace

int64_t trimul_mask_parts(const oops_trimul_geometry& g) { return 2 * factor_cblocks(g); }

namespace {
struct FactorPlan {
  bool fullw, v16;
  int tpw;
  int64_t groups, tiles;
  size_t lds;
};
// workgroups of the factor kernels (each keeps its W block across its token tiles): the straight-line
// forward runs best with two resident workgroups per CU and no second round
#ifndef OOPS_FACTOR_WGS
#define OOPS_FACTOR_WGS 2048
#endif
#ifndef OOPS_FACTOR_FWD_WGS
#define OOPS_FACTOR_FWD_WGS 512
#endif
FactorPlan factor_plan(const oops_trimul_geometry& g, bool backward) {
  const int64_t cblocks = factor_cblocks(g);
  const int64_t token_tiles = (g.groups * g.positions + kFM - 1) / kFM;
  FactorPlan pl{};
  // 16-token blocks within one group: the straight-line kernel, W whole in LDS.  Otherwise the
  // backward's epilogue holds more live values: the streaming form keeps it under 256 VGPRs
  // (its range-checked resources take 32-bit sizes: two groups of the factor layout, and the mask)
  pl.v16 = g.positions % 16 == 0 && g.c_row <= kFullWMaxK && (int64_t)4 * g.hidden * g.positions < (int64_t(1) << 31) &&
           g.groups * g.positions * 4 < (int64_t(1) << 31);
  pl.fullw = g.c_row <= kFullWMaxK && (!backward || pl.v16);
  const int64_t wgs = backward || !pl.v16 ? OOPS_FACTOR_WGS : OOPS_FACTOR_FWD_WGS;
  pl.tpw = pl.fullw ? (int)std::max<int64_t>(1, (token_tiles * 2 * cblocks + wgs - 1) / wgs) : 1;
  pl.groups = (token_tiles + pl.tpw - 1) / pl.tpw;
  pl.tiles = pl.groups * 2 * cblocks;
  int64_t panels = (g.c_row + kFK - 1) / kFK;
  if (pl.v16 && panels == 3) panels = 4;  // the straight-line kernel is built for 1, 2 or 4 panels
  pl.lds = (size_t)(pl.fullw ? panels : 2) * 128 * kFK * 2;
  // the forward straight-line kernel of one or two panels also stages each wave's 32 x rows
  if (V16_STAGE && pl.v16 && panels <= 2) pl.lds += (size_t)panels * 4 * 32 * kFK * 2;
  return pl;
}
}  // namespace

int64_t trimul_bias_parts(const oops_trimul_geometry& g) {
  return g.dtype == OOPS_F32 ? trimul_bias_parts_f32(g) : factor_plan(g, true).groups;
}

hipError_t launch_trimul_factors(const oops_trimul_geometry& g, const void* normalized, const void* weight,
                                 const float* bias, const void* mask, void* factors, const void* grad_factors,
                                 void* grad_projection, float* grad_mask_parts, float* grad_bias_parts,
                                 hipStream_t stream) {
  if (g.dtype == OOPS_F32)
    return launch_trimul_factors_f32(g, normalized, weight, bias, mask, factors, grad_factors, grad_projection,
                                     grad_mask_parts, grad_bias_parts, stream);
  FactorArgs a{};
  a.xn = normalized, a.w = weight, a.bias = bias, a.mask = g.has_mask ? static_cast<const float*>(mask) : nullptr;
  a.factors = factors, a.grad_factors = grad_factors, a.grad_proj = grad_projection;
  a.mask_parts = g.has_mask ? grad_mask_parts : nullptr;
  a.bias_parts = grad_bias_parts;
  a.rows = g.groups * g.positions, a.positions = g.positions, a.groups = g.groups, a.c_row = g.c_row;
  a.H = g.hidden;
  a.cblocks = (int)factor_cblocks(g);
  const bool bwd = grad_factors != nullptr;
  const FactorPlan pl = factor_plan(g, bwd);
  if (pl.tiles == 0) return hipSuccess;
  a.tiles = pl.tiles;
  a.tpw = pl.tpw;
  const dim3 grid((unsigned)xcd_grid(pl.tiles, 0));
  return by_half(g.dtype, [&](auto tag) -> hipError_t {
    using T = decltype(tag);
    if (pl.v16) {
      const int np = (int)((g.c_row + kFK - 1) / kFK);
      auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(256), pl.lds, stream, a); };
      auto by_np = [&](auto bwd_tag, auto masked_tag) {
        constexpr bool B = decltype(bwd_tag)::value, M = decltype(masked_tag)::value;
        if (np == 1)
          go(trimul_factor_v16_kernel<T, B, 1, M>);
        else if (np == 2)
          go(trimul_factor_v16_kernel<T, B, 2, M>);
        else
          go(trimul_factor_v16_kernel<T, B, 4, M>);
      };
      const bool m = a.mask != nullptr;
      if (bwd)
        m ? by_np(std::true_type{}, std::true_type{}) : by_np(std::true_type{}, std::false_type{});
      else
        m ? by_np(std::false_type{}, std::true_type{}) : by_np(std::false_type{}, std::false_type{});
    } else if (bwd && pl.fullw)
      hipLaunchKernelGGL((trimul_factor_kernel<T, true, true>), grid, dim3(256), pl.lds, stream, a);
    else if (bwd)
      hipLaunchKernelGGL((trimul_factor_kernel<T, true, false>), grid, dim3(256), pl.lds, stream, a);
    else if (pl.fullw)
      hipLaunchKernelGGL((trimul_factor_kernel<T, false, true>), grid, dim3(256), pl.lds, stream, a);
    else
      hipLaunchKernelGGL((trimul_factor_kernel<T, false, false>), grid, dim3(256), pl.lds, stream, a);
    return hipGetLastError();
  });
}

namespace {
#ifndef OOPS_OUTNORM_NPB
#define OOPS_OUTNORM_NPB 32
#endif
#ifndef OOPS_OUTNORM_T_WGS
#define OOPS_OUTNORM_T_WGS 1024
#endif
// positions per output-norm workgroup: a divisor of 256 whose LDS tiles fit
int out_norm_npb(int H, bool backward) {
  const int tiles = backward ? 2 : 1;
  int npb = OOPS_OUTNORM_NPB;
  while (npb > 1 && (int64_t)tiles * H * (npb + 1) * 4 > 64 * 1024) npb /= 2;
  return npb;
}

// the wave-tile kernels: 16-bit pairs, H = 32, 64 or 128, positions a multiple of 8; workgroups of 4 waves
int out_norm_t_ni(const oops_trimul_geometry& g) {
  const bool ok = g.dtype != OOPS_F32 && g.positions % 8 == 0 && g.h_row == g.hidden &&
                  (g.hidden == 32 || g.hidden == 64 || g.hidden == 128);
  return ok ? g.hidden / 8 : 0;
}
int64_t out_norm_t_grid(const oops_trimul_geometry& g) {
  const int tp = g.hidden == 128 ? 32 : 64;  // out_norm_tp
  const int64_t tiles = g.groups * ((g.positions + tp - 1) / tp);
  return std::min<int64_t>(OOPS_OUTNORM_T_WGS, (tiles + 3) / 4);
}
}  // namespace

int64_t trimul_output_norm_parts(const oops_trimul_geometry& g) {
  if (out_norm_t_ni(g)) return 4 * out_norm_t_grid(g);
  const int npb = out_norm_npb(g.hidden, true);
  return g.groups * ((g.positions + npb - 1) / npb);
}

namespace {
hipError_t run_out_norm(const oops_trimul_geometry& g, OutNormArgs& a, bool backward, hipStream_t stream) {
  a.groups = g.groups, a.positions = g.positions, a.h_row = g.h_row, a.H = g.hidden, a.eps = g.eps;
  if (const int ni = out_norm_t_ni(g)) {
    const int64_t grid = out_norm_t_grid(g);
    if (grid == 0) return hipSuccess;
    return by_half(g.dtype, [&](auto tag) -> hipError_t {
      using T = decltype(tag);
      auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(256), 0, stream, a); };
      if (backward)
        ni == 4 ? go(trimul_out_norm_t_backward_kernel<T, 4>)
        : ni == 8 ? go(trimul_out_norm_t_backward_kernel<T, 8>) : go(trimul_out_norm_t_backward_kernel<T, 16>);
      else
        ni == 4 ? go(trimul_out_norm_t_forward_kernel<T, 4>)
        : ni == 8 ? go(trimul_out_norm_t_forward_kernel<T, 8>) : go(trimul_out_norm_t_forward_kernel<T, 16>);
      return hipGetLastError();
    });
  }
  a.npb = out_norm_npb(g.hidden, backward);
  a.pblocks = (g.positions + a.npb - 1) / a.npb;
  const int64_t blocks = g.groups * a.pblocks;
  if (blocks == 0) return hipSuccess;
  const size_t lds = (size_t)(backward ? 2 : 1) * g.hidden * (a.npb + 1) * sizeof(float);
  // (the 16-byte paths move eight 16-bit elements; float32 takes the element-wise ones)
  const bool vec = g.dtype != OOPS_F32 && g.positions % 8 == 0 && a.npb >= 8 && (!backward || g.hidden % 8 == 0);
  return by_any(g.dtype, [&](auto tag) -> hipError_t {
    using T = decltype(tag);
    constexpr bool kVecOk = sizeof(T) == 2;
    const dim3 grid((unsigned)blocks);
    if (backward && vec && kVecOk)
      hipLaunchKernelGGL((trimul_out_norm_backward_kernel<T, kVecOk>), grid, dim3(256), lds, stream, a);
    else if (backward)
      hipLaunchKernelGGL((trimul_out_norm_backward_kernel<T, false>), grid, dim3(256), lds, stream, a);
    else if (vec && kVecOk)
      hipLaunchKernelGGL((trimul_out_norm_forward_kernel<T, kVecOk>), grid, dim3(256), lds, stream, a);
    else
      hipLaunchKernelGGL((trimul_out_norm_forward_kernel<T, false>), grid, dim3(256), lds, stream, a);
    return hipGetLastError();
  });
}
}  // namespace

hipError_t launch_trimul_output_norm_forward(const oops_trimul_geometry& g, const void* combined, const float* weight,
                                             const float* bias, void* normalized, float* mean, float* rstd,
                                             hipStream_t stream) {
  OutNormArgs a{};
  a.comb = combined, a.w = weight, a.b = bias, a.nrm = normalized, a.mean = mean, a.rstd = rstd;
  return run_out_norm(g, a, false, stream);
}

hipError_t launch_trimul_output_norm_backward(const oops_trimul_geometry& g, const void* combined,
                                              const float* weight, const float* mean, const float* rstd,
                                              const void* grad_normalized, void* grad_combined,
                                              float* grad_weight_parts, float* grad_bias_parts, hipStream_t stream) {
  OutNormArgs a{};
  a.comb = combined, a.w = weight, a.mean = const_cast<float*>(mean), a.rstd = const_cast<float*>(rstd);
  a.dn = grad_normalized, a.dcomb = grad_combined, a.dw = grad_weight_parts, a.db = grad_bias_parts;
  return run_out_norm(g, a, true, stream);
}

hipError_t launch_trimul_output(const oops_trimul_geometry& g, const void* normalized, const void* pair_normalized,
                                const void* output_weight, const void* gate_weight, const float* output_bias,
                                const float* gate_bias, void* out, const void* grad_out, void* grad_value,
                                void* grad_gate, hipStream_t stream) {
  if (g.dtype == OOPS_F32)
    return launch_trimul_output_f32(g, normalized, pair_normalized, output_weight, gate_weight, output_bias,
                                    gate_bias, out, grad_out, grad_value, grad_gate, stream);
  OutArgs a{};
  a.nrm = normalized, a.xn = pair_normalized, a.wo = output_weight, a.wg = gate_weight;
  a.bo = output_bias, a.bg = gate_bias, a.out = out, a.gout = grad_out, a.gval = grad_value, a.ggate = grad_gate;
  a.rows = g.groups * g.positions, a.c_row = g.c_row, a.h_row = g.h_row, a.C = g.channels;
  a.cblocks = (g.channels + kON - 1) / kON;
  const int64_t tiles = (a.rows + kOM - 1) / kOM * a.cblocks;
  if (tiles == 0) return hipSuccess;
  const bool bwd = grad_out != nullptr;
  if (g.h_row <= 2 * kOK && g.c_row <= 2 * kOK && g.channels % 8 == 0) {
    const int64_t tiles_m = (a.rows + kOM - 1) / kOM;
    const int64_t runs = std::max<int64_t>(1, OOPS_OUTPUT_WGS / a.cblocks);
    a.tpw = (int)((tiles_m + runs - 1) / runs);
    a.tiles = (tiles_m + a.tpw - 1) / a.tpw * a.cblocks;
    const dim3 wgrid((unsigned)xcd_grid(a.tiles, 0));
    return by_half(g.dtype, [&](auto tag) -> hipError_t {
      using T = decltype(tag);
      if (bwd)
        hipLaunchKernelGGL((trimul_output_w_kernel<T, true>), wgrid, dim3(256), 0, stream, a);
      else
        hipLaunchKernelGGL((trimul_output_w_kernel<T, false>), wgrid, dim3(256), 0, stream, a);
      return hipGetLastError();
    });
  }
  a.tiles = tiles;
  const dim3 grid((unsigned)xcd_grid(tiles, 0));
  return by_half(g.dtype, [&](auto tag) -> hipError_t {
    using T = decltype(tag);
    if (bwd)
      hipLaunchKernelGGL((trimul_output_kernel<T, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((trimul_output_kernel<T, false>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
  });
}


namespace {
#ifndef OOPS_OUTGRAD_WGS
#define OOPS_OUTGRAD_WGS 256
#endif
struct GradPlan {
  int tpw;
  int64_t grid;
};
GradPlan grad_plan(const oops_trimul_geometry& g) {
  const int64_t tiles = (g.groups * g.positions + kGT - 1) / kGT;
  GradPlan pl{};
  pl.tpw = (int)std::max<int64_t>(1, (tiles + OOPS_OUTGRAD_WGS - 1) / OOPS_OUTGRAD_WGS);
  pl.grid = (tiles + pl.tpw - 1) / pl.tpw;
  return pl;
}
}  // namespace

bool trimul_output_grad_supported(const oops_trimul_geometry& g) {
  return g.dtype != OOPS_F32 && g.channels == kGN && g.hidden == kGN;
}

int64_t trimul_output_grad_parts(const oops_trimul_geometry& g) {
  return trimul_output_grad_supported(g) ? grad_plan(g).grid : 0;
}

hipError_t launch_trimul_output_grad(const oops_trimul_geometry& g, const void* x, int64_t x_row, const void* w,
                                     int64_t w_row, const void* y, int64_t y_row, void* d, int64_t d_row,
                                     float* g_parts, float* s_parts, hipStream_t stream) {
  const GradPlan pl = grad_plan(g);
  if (pl.grid == 0) return hipSuccess;
  GradArgs a{};
  a.x = x, a.w = w, a.y = y, a.d = d, a.g_parts = g_parts, a.s_parts = s_parts;
  a.rows = g.groups * g.positions, a.x_row = x_row, a.w_row = w_row, a.y_row = y_row, a.d_row = d_row;
  a.tpw = pl.tpw;
  return by_half(g.dtype, [&](auto tag) -> hipError_t {
    using T = decltype(tag);
    hipLaunchKernelGGL((trimul_output_grad_kernel<T>), dim3((unsigned)pl.grid), dim3(512), 0, stream, a);
    return hipGetLastError();
  });
}

}  // namespace oops
