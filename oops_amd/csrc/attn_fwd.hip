// Flash-style forward of pair-biased attention on gfx950 MFMA.
//
// Work split: one workgroup = 4 wavefronts = one (sample, group, head) and a
// block of 128 queries; wave w owns queries w*32 .. w*32+31.  The key axis
// is walked in 32-key tiles.  Per tile the workgroup stages K (row-major),
// V (transposed, key-permuted) and the 128 x 32 bias block in LDS; each wave
// then computes its 32 x 32 score tile S^T = K Q^T with the query as the MFMA
// column, so a lane holds 16 scores of one query and the online-softmax row
// statistics need a single cross-lane exchange (lane ^ 32).  P is converted
// in registers into the k-operand of O^T += V^T P^T.
//
// Follows the semantics of the reference's _attend / online_softmax_step
// (oops/attention/triangle/triton/kernel.py:151-262,
//  oops/attention/flash/triton/kernel.py:35-50): logits are
// fma(QK, scale, bias); masked and out-of-range keys are -inf and their K/V
// rows are read as zero; the exponent reference is clamped to 0 while a row
// has seen no valid key; a fully masked row yields O = 0 and LSE = 0.  LSE is
// stored in log2 units (internal to this library).
#include "attn_kernels.h"

namespace oops {

template <typename T, typename BT, int DP>
__global__ __launch_bounds__(256) void attn_fwd_kernel(FwdArgs a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr bool kF32 = sizeof(T) == 4;
  constexpr int KPAD = kF32 ? 1 : 8;
  constexpr int KLD = DP + KPAD;        // K tile row (elements)
  constexpr int VLD = kF32 ? DP + 1 : 32 + 8;  // V tile row: natural (f32) / transposed
  constexpr int BLD = 32 + (sizeof(BT) == 4 ? 4 : 8);  // bias row (16-byte multiple)
  constexpr int NDT = DP / 32;          // 32-wide d tiles
  constexpr int NQF = DP / E::kKStep;   // k-steps of QK^T

  __shared__ __attribute__((aligned(16))) T k_lds[32 * KLD];
  __shared__ __attribute__((aligned(16))) T v_lds[kF32 ? 32 * VLD : DP * VLD];
  __shared__ __attribute__((aligned(16))) BT b_lds[128 * BLD];
  __shared__ __attribute__((aligned(16))) uint8_t m_lds[128 * 32];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int g2 = lane >> 5;

  int64_t tile = blockIdx.x;
  const Sample* tab = reinterpret_cast<const Sample*>(a.table);
  const int H = a.num_heads;
  const int s_idx = find_sample(tile, tab, a.num_samples, a.uniform_tiles,
                                [&](const Sample& s) { return s.G * H * cdiv(s.Lq, 128); });
  if (s_idx < 0) return;
  const Sample& S = tab[s_idx];
  const int64_t G = S.G;
  const int Lq = (int)S.Lq, Lk = (int)S.Lk;
  const int g = (int)(tile % G);
  const int64_t rest = tile / G;
  const int nqb = (int)cdiv(Lq, 128);
  const int qb = (int)(rest % nqb);
  const int h = (int)(rest / nqb);
  const int D = a.head_size;
  const bool vec = a.vec_ok;

  const T* qbase = a.q + S.q_off + g * S.q_sg + h * S.q_sh;
  const T* kbase = a.k + S.k_off + g * S.k_sg + h * S.k_sh;
  const T* vbase = a.v + S.v_off + g * S.v_sg + h * S.v_sh;
  const bool has_bias = a.bias != nullptr && S.b_off >= 0;
  const BT* bbase = has_bias ? a.bias + S.b_off + g * S.b_sg + h * S.b_sh : nullptr;
  const bool has_mask = a.mask != nullptr && S.m_off >= 0;
  const uint8_t* mbase = has_mask ? a.mask + S.m_off + g * S.m_sg : nullptr;
  const bool pair_mask = has_mask && S.m_si != 0;

  // ---- Q fragments (B operand: lane = query, k = head dim)
  const int q_lane = qb * 128 + wave * 32 + lq;
  Frag qf[NQF];
  {
    const bool qv = q_lane < Lq;
    const T* qrow = qbase + (int64_t)q_lane * S.q_si;
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      if constexpr (kF32) {
        const int d = s * 2 + g2;
        qf[s] = (qv && d < D) ? qrow[d] : 0.0f;
      } else {
        const uint4 u = qv ? load16(qrow, s * 16 + g2 * 8, D, vec) : make_uint4(0, 0, 0, 0);
        qf[s] = __builtin_bit_cast(Frag, u);
      }
    }
  }

  const float c1 = a.scale * kLog2e;
  float m_run = kNegInf;  // running max, log2 units
  float l_run = 0.0f;     // this lane's partial row sum
  f32x16 oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) oacc[t] = f32x16{};

  constexpr int CE = 16 / sizeof(T);      // elements per 16-byte chunk
  constexpr int CPR = DP / CE;            // chunks per K/V row
  constexpr int BCE = 16 / sizeof(BT);
  constexpr int BCPR = 32 / BCE;          // chunks per bias row

  for (int k0 = 0; k0 < Lk; k0 += 32) {
    __syncthreads();
    // ---- stage K, V
    for (int c = tid; c < 32 * CPR; c += 256) {
      const int r = c / CPR;
      const int col = (c % CPR) * CE;
      const int key = k0 + r;
      bool ok = key < Lk;
      if (ok && has_mask && !pair_mask) ok = mbase[key] != 0;
      uint4 ku = make_uint4(0, 0, 0, 0), vu = make_uint4(0, 0, 0, 0);
      if (ok) {
        ku = load16(kbase + (int64_t)key * S.k_si, col, D, vec);
        vu = load16(vbase + (int64_t)key * S.v_si, col, D, vec);
      }
      if constexpr (kF32) {
        // odd row stride (bank-conflict free column reads): scalar stores
        store_elems(&k_lds[r * KLD + col], ku);
        store_elems(&v_lds[r * VLD + col], vu);
      } else {
        *reinterpret_cast<uint4*>(&k_lds[r * KLD + col]) = ku;
        const T* ve = reinterpret_cast<const T*>(&vu);
        const int pos = perm16(r);
#pragma unroll
        for (int i = 0; i < CE; ++i) v_lds[(col + i) * VLD + pos] = ve[i];
      }
    }
    // ---- stage bias [128 queries x 32 keys], key positions permuted
    if (has_bias) {
      for (int c = tid; c < 128 * BCPR; c += 256) {
        const int r = c / BCPR;
        const int kc = (c % BCPR) * BCE;
        const int q = qb * 128 + r;
        union {
          uint4 u;
          BT e[BCE];
        } bu;
        bu.u = make_uint4(0, 0, 0, 0);
        if (q < Lq) bu.u = load16(bbase + (int64_t)q * S.b_si, k0 + kc, Lk, vec && (k0 + kc + BCE <= Lk));
#pragma unroll
        for (int i = 0; i < BCE; i += 4) {
          // 4 consecutive keys stay contiguous under perm32
          BT* dst = &b_lds[r * BLD + perm32(kc + i)];
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[e] = bu.e[i + e];
        }
      }
    }
    // ---- stage mask (keep bytes), key positions permuted
    if (has_mask) {
      const int rows = pair_mask ? 128 : 1;
      for (int c = tid; c < rows * 8; c += 256) {
        const int r = c >> 3;
        const int kc = (c & 7) * 4;
        const int q = qb * 128 + r;
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = k0 + kc + e;
          uint8_t keep = 0;
          if (key < Lk && (!pair_mask || q < Lq))
            keep = mbase[(pair_mask ? (int64_t)q * S.m_si : 0) + key] != 0;
          w |= (uint32_t)keep << (8 * e);
        }
        *reinterpret_cast<uint32_t*>(&m_lds[r * 32 + perm32(kc)]) = w;
      }
    }
    __syncthreads();

    // ---- S^T = K Q^T  (rows: keys kappa(g2, j), column: this lane's query)
    f32x16 sacc = f32x16{};
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      Frag kf;
      if constexpr (kF32) {
        kf = k_lds[lq * KLD + s * 2 + g2];
      } else {
        kf = __builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(&k_lds[lq * KLD + s * 16 + g2 * 8]));
      }
      sacc = E::mma(kf, qf[s], sacc);
    }

    float x[16];
    if (has_bias) {
      const BT* brow = &b_lds[(wave * 32 + lq) * BLD + g2 * 16];
#pragma unroll
      for (int j = 0; j < 16; ++j) x[j] = __builtin_fmaf(sacc[j], c1, Elem<BT>::to_f(brow[j]) * kLog2e);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) x[j] = sacc[j] * c1;
    }
    if (has_mask) {
      const uint8_t* mrow = &m_lds[(pair_mask ? wave * 32 + lq : 0) * 32 + g2 * 16];
#pragma unroll
      for (int j = 0; j < 16; ++j) x[j] = mrow[j] ? x[j] : kNegInf;
    } else if (k0 + 32 > Lk) {
#pragma unroll
      for (int j = 0; j < 16; ++j) x[j] = (k0 + kappa(g2, j) < Lk) ? x[j] : kNegInf;
    }

    // ---- online softmax (log2 units)
    float mx = x[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) mx = fmaxf(mx, x[j]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == kNegInf ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float p[16];
    float psum = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      p[j] = __builtin_amdgcn_exp2f(x[j] - m_use);
      psum += p[j];
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int t = 0; t < NDT; ++t) oacc[t] *= alpha;

    // ---- O^T += V^T P^T
    if constexpr (kF32) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int key = kappa(g2, j);
#pragma unroll
        for (int t = 0; t < NDT; ++t) oacc[t] = E::mma(v_lds[key * VLD + t * 32 + lq], p[j], oacc[t]);
      }
    } else {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const Frag pf = pack8<T>(&p[8 * m]);
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
          const Frag vf = __builtin_bit_cast(
              Frag, *reinterpret_cast<const uint4*>(&v_lds[(t * 32 + lq) * VLD + 16 * m + g2 * 8]));
          oacc[t] = E::mma(vf, pf, oacc[t]);
        }
      }
    }
  }

  // ---- epilogue
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / (l_tot == 0.0f ? 1.0f : l_tot);
  if (q_lane < Lq) {
    const int64_t o_row = S.o_off + g * S.o_sg + h * S.o_sh + (int64_t)q_lane * S.o_si;
    T* orow = a.out + o_row;
    T* lrow = a.out_lo != nullptr ? a.out_lo + o_row : nullptr;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = t * 32 + kappa(g2, i);
        if (d < D) {
          const float o = oacc[t][i] * inv;
          const T hi = E::from_f(o);
          orow[d] = hi;
          if (lrow) lrow[d] = E::from_f(o - E::to_f(hi));  // rounding residual of the output
        }
      }
    }
    if (g2 == 0 && a.lse != nullptr) {
      const float m_use = m_run == kNegInf ? 0.0f : m_run;
      a.lse[S.l_off + ((int64_t)g * H + h) * Lq + q_lane] = l_tot == 0.0f ? 0.0f : m_use + __log2f(l_tot);
    }
  }
}

#define OOPS_FWD_INST(T, BT, DP) template __global__ void attn_fwd_kernel<T, BT, DP>(FwdArgsT<T, BT>);
OOPS_FOR_EACH_CONFIG(OOPS_FWD_INST)

}  // namespace oops

namespace oops {

hipError_t launch_forward(const oops_attn_geometry& geo, const Plan& plan, const void* q, const void* k,
                          const void* v, const uint8_t* mask, const void* bias, void* bias_frag, void* out,
                          void* out_lo, float* lse, hipStream_t stream) {
  hipError_t err = hipSuccess;
  if (plan.bias_frag) {
    err = launch_bias_frag(geo, plan, bias, bias_frag, stream);
    if (err != hipSuccess) return err;
  }
  if (launch_forward_fast(geo, plan, q, k, v, mask, bias, plan.bias_frag ? bias_frag : nullptr, out, out_lo, lse,
                          stream, &err))
    return err;
  const bool ok = dispatch_config(geo.dtype, geo.bias_dtype, plan.dp, [&](auto t, auto bt, auto dpc) {
    using T = typename decltype(t)::type;
    using BT = typename decltype(bt)::type;
    constexpr int DP = decltype(dpc)::value;
    FwdArgsT<T, BT> a;
    a.q = static_cast<const T*>(q);
    a.k = static_cast<const T*>(k);
    a.v = static_cast<const T*>(v);
    a.bias = geo.has_bias ? static_cast<const BT*>(bias) : nullptr;
    a.mask = geo.has_mask ? mask : nullptr;
    a.out = static_cast<T*>(out);
    a.out_lo = static_cast<T*>(out_lo);
    a.lse = lse;
    a.table = geo.table_device;
    a.uniform_tiles = plan.fwd_uniform;
    a.bias_frag = nullptr;
    a.bf_sample_stride = 0;
    a.bf_nqt = a.bf_nkt = 0;
    a.num_samples = geo.num_samples;
    a.num_heads = geo.num_heads;
    a.head_size = geo.head_size;
    a.vec_ok = geo.vec_ok;
    a.scale = geo.scale;
    if (plan.fwd_tiles > 0) {
      hipLaunchKernelGGL((attn_fwd_kernel<T, BT, DP>), dim3((unsigned)plan.fwd_tiles), dim3(256), 0, stream, a);
      err = hipGetLastError();
    }
  });
  return ok ? err : hipErrorInvalidValue;
}

}  // namespace oops
