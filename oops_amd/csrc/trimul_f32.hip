// Triangle multiplicative update, float32 pairs: the factor projections and
// the gated output projection on the exact float32 matrix core
// (v_mfma_f32_32x32x2f32, fp32 products and sums), with the same fused
// epilogues and the same output layouts as the 16-bit kernels of trimul.hip,
// so the host pipeline (LayerNorms, contraction, weight-gradient GEMMs) is
// shared.  Reference: oops/pair/triangle_multiplication/triton/generic.py:111-200
// (the reference serves float32 through its own fused kernels as well).
//
// Both kernels: one workgroup = 4 waves x 32 tokens (128 tokens) and 64
// channels.  K runs in panels of 32 through a two-buffer LDS tile of W (rows
// padded to 36 floats); a lane holds 16 consecutive k of its token row in
// registers.  One 32x32x2 MFMA sums k = {s, 16 + s} of a panel half: lane
// half g2 supplies k = 16 g2 + s, so every operand a lane needs is contiguous
// (the order of the k sum is free, A and B use the same one).
#include "attn_fast_common.h"
#include "trimul_kernels.h"

namespace oops {

using namespace fast;

namespace {

constexpr int kTM = 128;        // tokens per workgroup
constexpr int kTK = 32;         // k per panel
constexpr int kWLD = kTK + 4;   // LDS row of a W panel (floats; the pad spreads the rows over the banks)

__device__ __forceinline__ float sigmoid32(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}
__device__ __forceinline__ f32x16 mma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// acc[t] += x . W[32 t + lq]^T over one panel: xs = this lane's 16 k of its
// row (k = 16 g2 + 0..15), wt = the panel (rows of kWLD floats), NT tiles
template <int NT>
__device__ __forceinline__ void panel_mma(f32x16 (&acc)[NT], const float* xs, const float* wt, int lq, int g2,
                                          bool x_is_a) {
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4) {
    float4 wv[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
      wv[t] = *reinterpret_cast<const float4*>(wt + (32 * t + lq) * kWLD + 16 * g2 + 4 * s4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = xs[4 * s4 + e];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float w = e == 0 ? wv[t].x : e == 1 ? wv[t].y : e == 2 ? wv[t].z : wv[t].w;
        acc[t] = x_is_a ? mma_f32(x, w, acc[t]) : mma_f32(w, x, acc[t]);
      }
    }
  }
}

struct F32FactorArgs {
  const float* xn;       // [R][c_row]
  const float* w;        // [4H][c_row]: left value, left gate, right value, right gate
  const float* bias;     // [4H] or null
  const float* mask;     // [R] or null
  float* factors;        // [2][G][H][P]
  const float* grad_factors;
  float* grad_proj;      // [4H][R]
  float* mask_parts;     // [2 cblocks][R]
  float* bias_parts;     // [token tiles][4H]
  int64_t rows, positions, groups, c_row, tiles;
  int H, cblocks;
};

// One workgroup = (token tile, factor f, 64-channel block cb): W rows 0..63 are
// the block's value channels, 64..127 its gate channels; acc[t] (t = 0, 1)
// value and acc[t + 2] gate of channel cb*64 + 32 t + lq for tokens
// r0 + 32 wave + 8 q + 4 g2 + i (element 4 q + i).
template <bool BWD>
__global__ __launch_bounds__(256) void trimul_factor_f32_kernel(F32FactorArgs a) {
  __shared__ __attribute__((aligned(16))) float w_lds[2][128 * kWLD];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, lq = lane & 31, g2 = lane >> 5;
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x, 0);
  if (tile >= a.tiles) return;
  const int nb = 2 * a.cblocks;
  const int fc = (int)(tile % nb);
  const int f = fc / a.cblocks, cb = fc - f * a.cblocks;
  const int64_t tt = tile / nb;
  const int64_t r0 = tt * kTM;
  const int H = a.H;
  const int K = (int)a.c_row;
  const int64_t R = a.rows, P = a.positions;

  // W: thread tid loads row tid / 2, floats 16 (tid % 2) .. +15 of each panel
  const int wrow = tid >> 1, whalf = tid & 1;
  const int whv = cb * 64 + (wrow & 63);
  const bool wok = whv < H;
  const float* wsrc = a.w + (int64_t)(f * 2 * H + (wrow >= 64 ? H : 0) + (wok ? whv : 0)) * K + 16 * whalf;
  auto load_w = [&](int k0, float4 (&wu)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      wu[j] = wok && k0 + 16 * whalf + 4 * j < K ? *reinterpret_cast<const float4*>(wsrc + k0 + 4 * j)
                                                  : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  auto store_w = [&](int buf, const float4 (&wu)[4]) {
    float* d = &w_lds[buf][wrow * kWLD + 16 * whalf];
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<float4*>(d + 4 * j) = wu[j];
  };
  // x: this lane's token row, floats k0 + 16 g2 .. +15
  const int64_t tok = r0 + wave * 32 + lq;
  const bool tv = tok < R;
  const float* xsrc = a.xn + (tv ? tok : 0) * a.c_row + 16 * g2;
  auto load_x = [&](int k0, float (&xs)[16]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 v = tv && k0 + 16 * g2 + 4 * j < K ? *reinterpret_cast<const float4*>(xsrc + k0 + 4 * j)
                                                       : make_float4(0.f, 0.f, 0.f, 0.f);
      xs[4 * j] = v.x, xs[4 * j + 1] = v.y, xs[4 * j + 2] = v.z, xs[4 * j + 3] = v.w;
    }
  };

  f32x16 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x16{};
  const int np = (K + kTK - 1) / kTK;
  float4 wu[4];
  float xs[16], xn[16];
  load_w(0, wu);
  load_x(0, xs);
  store_w(0, wu);
  __syncthreads();
  for (int i = 0; i < np; ++i) {
    const bool more = i + 1 < np;
    if (more) {
      load_w((i + 1) * kTK, wu);
      load_x((i + 1) * kTK, xn);
    }
    panel_mma<4>(acc, xs, w_lds[i & 1], lq, g2, true);
    if (more) store_w((i + 1) & 1, wu);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 16; ++e) xs[e] = xn[e];
  }

  // ---- epilogue
  float mp[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) mp[v] = 0.f;
  float bsum[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
  // (group, position) of the lane's first token of each q: tokens 4 apart from
  // a multiple of 4 share a group when P % 4 == 0 (one float4 per q)
  const bool vec4 = (P & 3) == 0;
  int64_t gq[4], pq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t r4 = r0 + wave * 32 + 8 * q + 4 * g2;
    gq[q] = r4 / P;
    pq[q] = r4 - gq[q] * P;
  }
  const int64_t fG = (int64_t)f * a.groups;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int hv = cb * 64 + 32 * t + lq;
    if (hv >= H) continue;
    const float bv = a.bias ? a.bias[f * 2 * H + hv] : 0.f;
    const float bg = a.bias ? a.bias[f * 2 * H + H + hv] : 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t r4 = r0 + wave * 32 + 8 * q + 4 * g2;
      if (r4 >= R) continue;
      const bool full4 = vec4 && r4 + 3 < R;
      float v[4], sg[4], keep[4];
      int64_t off[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t r = r4 + i;
        v[i] = acc[t][4 * q + i] + bv;
        sg[i] = sigmoid32(acc[t + 2][4 * q + i] + bg);
        keep[i] = a.mask && r < R ? a.mask[r] : 1.f;
        int64_t g = gq[q], p = pq[q] + i;
        if (p >= P) p -= P, ++g;  // i < 4 <= P steps at most one group
        while (p >= P) p -= P, ++g;
        off[i] = ((fG + g) * H + hv) * P + p;
      }
      if constexpr (!BWD) {
        if (full4) {
          *reinterpret_cast<float4*>(a.factors + off[0]) =
              make_float4(v[0] * sg[0] * keep[0], v[1] * sg[1] * keep[1], v[2] * sg[2] * keep[2],
                          v[3] * sg[3] * keep[3]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (r4 + i < R) a.factors[off[i]] = v[i] * sg[i] * keep[i];
        }
      } else {
        float d[4];
        if (full4) {
          const float4 u = *reinterpret_cast<const float4*>(a.grad_factors + off[0]);
          d[0] = u.x, d[1] = u.y, d[2] = u.z, d[3] = u.w;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) d[i] = r4 + i < R ? a.grad_factors[off[i]] : 0.f;
        }
        float dv[4], dg[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dv[i] = d[i] * keep[i] * sg[i];
          dg[i] = d[i] * keep[i] * v[i] * sg[i] * (1.f - sg[i]);
          mp[4 * q + i] += d[i] * v[i] * sg[i];
          bsum[t][0] += dv[i];
          bsum[t][1] += dg[i];
        }
        float* gv = a.grad_proj + (int64_t)(f * 2 * H + hv) * R + r4;
        float* gg = a.grad_proj + (int64_t)(f * 2 * H + H + hv) * R + r4;
        if (r4 + 3 < R && (R & 3) == 0) {
          *reinterpret_cast<float4*>(gv) = make_float4(dv[0], dv[1], dv[2], dv[3]);
          *reinterpret_cast<float4*>(gg) = make_float4(dg[0], dg[1], dg[2], dg[3]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (r4 + i < R) gv[i] = dv[i], gg[i] = dg[i];
        }
      }
    }
  }
  if constexpr (BWD) {
    if (a.mask_parts != nullptr) {
      // sum over the 32 channels of the half-wave (its lanes share the 16 tokens)
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
    if (a.bias_parts != nullptr) {
      // channel sums over the tile's tokens: the two half-waves, then the four waves
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
        if (hv < H)
          a.bias_parts[tt * 4 * H + f * 2 * H + k * H + hv] =
              bred[0][t][k][c] + bred[1][t][k][c] + bred[2][t][k][c] + bred[3][t][k][c];
      }
    }
  }
}

struct F32OutArgs {
  const float* nrm;   // [R][h_row]
  const float* xn;    // [R][c_row]
  const float* wo;    // [C][h_row]
  const float* wg;    // [C][c_row]
  const float* bo;
  const float* bg;
  float* out;         // [R][C]
  const float* gout;  // [R][C]
  float* gval;        // [R][c_row]
  float* ggate;       // [R][c_row]
  int64_t rows, c_row, h_row, tiles;
  int C, cblocks;
};

// One workgroup = (token tile, 64-channel block): the output channel is the
// MFMA row (A = W from LDS), the token the column (B = this lane's row), so
// acc[t] (value) and acc[2 + t] (gate logit) hold channels
// c0 + 32 t + 8 q + 4 g2 + i of token r0 + 32 wave + lq.
template <bool BWD>
__global__ __launch_bounds__(256) void trimul_output_f32_kernel(F32OutArgs a) {
  __shared__ __attribute__((aligned(16))) float w_lds[2][64 * kWLD];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, lq = lane & 31, g2 = lane >> 5;
  const int64_t tile = xcd_tile(blockIdx.x, gridDim.x, 0);
  if (tile >= a.tiles) return;
  const int cb = (int)(tile % a.cblocks);
  const int64_t r0 = (tile / a.cblocks) * kTM;
  const int c0 = cb * 64;
  const int C = a.C;
  const int64_t R = a.rows;
  const int64_t tok = r0 + wave * 32 + lq;
  const bool tv = tok < R;

  f32x16 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x16{};
#pragma unroll
  for (int phase = 0; phase < 2; ++phase) {
    const int K = (int)(phase == 0 ? a.h_row : a.c_row);
    const float* act = (phase == 0 ? a.nrm : a.xn) + (tv ? tok : 0) * K + 16 * g2;
    // W: thread tid loads row tid / 4 (channel c0 + tid / 4), floats 8 (tid % 4) .. +7
    const int wrow = tid >> 2, wq = tid & 3;
    const bool wok = c0 + wrow < C;
    const float* wsrc = (phase == 0 ? a.wo : a.wg) + (int64_t)(wok ? c0 + wrow : 0) * K + 8 * wq;
    auto load_w = [&](int k0, float4 (&wu)[2]) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        wu[j] = wok && k0 + 8 * wq + 4 * j < K ? *reinterpret_cast<const float4*>(wsrc + k0 + 4 * j)
                                               : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    auto store_w = [&](int buf, const float4 (&wu)[2]) {
      float* d = &w_lds[buf][wrow * kWLD + 8 * wq];
#pragma unroll
      for (int j = 0; j < 2; ++j) *reinterpret_cast<float4*>(d + 4 * j) = wu[j];
    };
    auto load_x = [&](int k0, float (&xs)[16]) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 v = tv && k0 + 16 * g2 + 4 * j < K ? *reinterpret_cast<const float4*>(act + k0 + 4 * j)
                                                         : make_float4(0.f, 0.f, 0.f, 0.f);
        xs[4 * j] = v.x, xs[4 * j + 1] = v.y, xs[4 * j + 2] = v.z, xs[4 * j + 3] = v.w;
      }
    };
    const int np = (K + kTK - 1) / kTK;
    float4 wu[2];
    float xs[16], xn[16];
    load_w(0, wu);
    load_x(0, xs);
    store_w(0, wu);
    __syncthreads();
    f32x16 pacc[2] = {acc[2 * phase], acc[2 * phase + 1]};
    for (int i = 0; i < np; ++i) {
      const bool more = i + 1 < np;
      if (more) {
        load_w((i + 1) * kTK, wu);
        load_x((i + 1) * kTK, xn);
      }
      panel_mma<2>(pacc, xs, w_lds[i & 1], lq, g2, false);
      if (more) store_w((i + 1) & 1, wu);
      __syncthreads();
#pragma unroll
      for (int e = 0; e < 16; ++e) xs[e] = xn[e];
    }
    acc[2 * phase] = pacc[0];
    acc[2 * phase + 1] = pacc[1];
  }

  // ---- epilogue: four consecutive channels c0 + 32 t + 8 q + 4 g2 .. +3 per (t, q)
  if (!tv) return;
  const bool vecc = (C & 3) == 0;
  const int cr = (int)a.c_row;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int ch0 = c0 + 32 * t + 8 * q + 4 * g2;
      float v[4], s[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ch = ch0 + i;
        const bool in = ch < C;
        v[i] = acc[t][4 * q + i] + (in && a.bo ? a.bo[ch] : 0.f);
        s[i] = sigmoid32(acc[2 + t][4 * q + i] + (in && a.bg ? a.bg[ch] : 0.f));
      }
      if constexpr (!BWD) {
        float* orow = a.out + tok * C;
        if (vecc && ch0 + 3 < C) {
          *reinterpret_cast<float4*>(orow + ch0) = make_float4(v[0] * s[0], v[1] * s[1], v[2] * s[2], v[3] * s[3]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (ch0 + i < C) orow[ch0 + i] = v[i] * s[i];
        }
      } else {
        const float* grow = a.gout + tok * C;
        float d[4];
        if (vecc && ch0 + 3 < C) {
          const float4 u = *reinterpret_cast<const float4*>(grow + ch0);
          d[0] = u.x, d[1] = u.y, d[2] = u.z, d[3] = u.w;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) d[i] = ch0 + i < C ? grow[ch0 + i] : 0.f;
        }
        // channels up to c_row are written (zeros past C), as the 16-bit kernel does
        if (ch0 < cr) {
          float dv[4], dg[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            dv[i] = d[i] * s[i];
            dg[i] = d[i] * v[i] * s[i] * (1.f - s[i]);
          }
          // c_row is a multiple of 8 and ch0 of 4: the four channels lie within the row
          *reinterpret_cast<float4*>(a.gval + tok * cr + ch0) = make_float4(dv[0], dv[1], dv[2], dv[3]);
          *reinterpret_cast<float4*>(a.ggate + tok * cr + ch0) = make_float4(dg[0], dg[1], dg[2], dg[3]);
        }
      }
    }
}

}  // namespace

hipError_t launch_trimul_factors_f32(const oops_trimul_geometry& g, const void* normalized, const void* weight,
                                     const float* bias, const void* mask, void* factors, const void* grad_factors,
                                     void* grad_projection, float* grad_mask_parts, float* grad_bias_parts,
                                     hipStream_t stream) {
  F32FactorArgs a{};
  a.xn = static_cast<const float*>(normalized);
  a.w = static_cast<const float*>(weight);
  a.bias = bias;
  a.mask = g.has_mask ? static_cast<const float*>(mask) : nullptr;
  a.factors = static_cast<float*>(factors);
  a.grad_factors = static_cast<const float*>(grad_factors);
  a.grad_proj = static_cast<float*>(grad_projection);
  a.mask_parts = g.has_mask ? grad_mask_parts : nullptr;
  a.bias_parts = grad_bias_parts;
  a.rows = g.groups * g.positions, a.positions = g.positions, a.groups = g.groups, a.c_row = g.c_row;
  a.H = (int)g.hidden;
  a.cblocks = (int)((g.hidden + 63) / 64);
  const int64_t token_tiles = (a.rows + kTM - 1) / kTM;
  a.tiles = token_tiles * 2 * a.cblocks;
  if (a.tiles == 0) return hipSuccess;
  const dim3 grid((unsigned)xcd_grid(a.tiles, 0));
  if (grad_factors != nullptr)
    hipLaunchKernelGGL(trimul_factor_f32_kernel<true>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(trimul_factor_f32_kernel<false>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

int64_t trimul_bias_parts_f32(const oops_trimul_geometry& g) { return (g.groups * g.positions + kTM - 1) / kTM; }

hipError_t launch_trimul_output_f32(const oops_trimul_geometry& g, const void* normalized,
                                    const void* pair_normalized, const void* output_weight, const void* gate_weight,
                                    const float* output_bias, const float* gate_bias, void* out, const void* grad_out,
                                    void* grad_value, void* grad_gate, hipStream_t stream) {
  F32OutArgs a{};
  a.nrm = static_cast<const float*>(normalized);
  a.xn = static_cast<const float*>(pair_normalized);
  a.wo = static_cast<const float*>(output_weight);
  a.wg = static_cast<const float*>(gate_weight);
  a.bo = output_bias, a.bg = gate_bias;
  a.out = static_cast<float*>(out);
  a.gout = static_cast<const float*>(grad_out);
  a.gval = static_cast<float*>(grad_value);
  a.ggate = static_cast<float*>(grad_gate);
  a.rows = g.groups * g.positions, a.c_row = g.c_row, a.h_row = g.h_row, a.C = (int)g.channels;
  a.cblocks = (int)((g.channels + 63) / 64);
  a.tiles = (a.rows + kTM - 1) / kTM * a.cblocks;
  if (a.tiles == 0) return hipSuccess;
  const dim3 grid((unsigned)xcd_grid(a.tiles, 0));
  if (grad_out != nullptr)
    hipLaunchKernelGGL(trimul_output_f32_kernel<true>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(trimul_output_f32_kernel<false>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace oops
