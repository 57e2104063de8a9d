// Backward of pair-biased attention on gfx950 MFMA.
//
// Four phases, one stream, no global atomics (deterministic):
//   1. attn_delta_kernel   delta[q] = sum_d O[q,d] * dO[q,d]
//   2. attn_dq_kernel      per (group, head, 128 queries): recompute P from
//                          LSE, dP^T = V dO^T, dS = P (dP - delta),
//                          dQ = scale * dS K; writes dBias = dS directly for
//                          a per-group ("full") bias.
//   3. attn_dkv_kernel     per (group, head, 128 keys): S = Q K^T with the key
//                          as MFMA column, dV^T += dO^T P, dK^T += Q^T dS.
//   4. attn_dbias_shared_kernel + attn_dbias_reduce_kernel for a bias shared
//                          by all groups: one workgroup owns a 128 x 32
//                          (query, key) block of one head and walks a range
//                          of groups, keeping the bias block in registers and
//                          accumulating sum_g dS there; ranges ("parts") are
//                          summed by the reduce kernel.
//
// Mirrors the reference's _backward_preprocess / _backward_query /
// _backward_key_value / _backward_shared_bias and softmax_backward_dscores
// (oops/attention/triangle/triton/kernel.py:375-873,
//  oops/attention/flash/triton/kernel.py:53-62,
//  oops/attention/triangle/triton/generic.py:320-536).
#include "attn_kernels.h"

namespace oops {

// ------------------------------------------------------------------ delta
template <typename T, typename BT, int DP>
__global__ __launch_bounds__(256) void attn_delta_kernel(BwdArgs a) {
  int64_t tile = blockIdx.x;
  const Sample* tab = reinterpret_cast<const Sample*>(a.table);
  const int H = a.num_heads;
  const int s_idx = find_sample(tile, tab, a.num_samples, a.uniform_tiles,
                                [&](const Sample& s) { return s.G * H * cdiv(s.Lq, 64); });
  if (s_idx < 0) return;
  const Sample& S = tab[s_idx];
  const int Lq = (int)S.Lq;
  const int nqb = (int)cdiv(Lq, 64);
  const int qb = (int)(tile % nqb);
  const int64_t gh = tile / nqb;
  const int h = (int)(gh % H);
  const int g = (int)(gh / H);
  const int q = qb * 64 + (threadIdx.x >> 2);
  const int part = threadIdx.x & 3;
  const int D = a.head_size;
  constexpr int CE = 16 / sizeof(T);
  float acc = 0.0f;
  if (q < Lq) {
    const int64_t o_row = S.o_off + g * S.o_sg + h * S.o_sh + (int64_t)q * S.o_si;
    const T* orow = a.out + o_row;
    const T* lrow = a.out_lo != nullptr ? a.out_lo + o_row : nullptr;
    const T* drow = a.dout + S.do_off + g * S.do_sg + h * S.do_sh + (int64_t)q * S.do_si;
    for (int c = part * CE; c < D; c += 4 * CE) {
      const uint4 ou = load16(orow, c, D, a.vec_ok);
      const uint4 lu = lrow ? load16(lrow, c, D, a.vec_ok) : make_uint4(0, 0, 0, 0);
      const uint4 du = load16(drow, c, D, a.vec_ok);
      const T* oe = reinterpret_cast<const T*>(&ou);
      const T* le = reinterpret_cast<const T*>(&lu);
      const T* de = reinterpret_cast<const T*>(&du);
#pragma unroll
      for (int i = 0; i < CE; ++i)
        acc += (Elem<T>::to_f(oe[i]) + Elem<T>::to_f(le[i])) * Elem<T>::to_f(de[i]);
    }
  }
  acc += __shfl_xor(acc, 1);
  acc += __shfl_xor(acc, 2);
  if (q < Lq && part == 0) a.delta[S.l_off + ((int64_t)g * H + h) * Lq + q] = acc;
}

// ------------------------------------------------------------------ dQ
template <typename T, typename BT, int DP>
__global__ __launch_bounds__(256) void attn_dq_kernel(BwdArgs a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr bool kF32 = sizeof(T) == 4;
  constexpr int KLD = DP + (kF32 ? 1 : 8);
  constexpr int TLD = 32 + 8;  // transposed K row (16-bit only)
  constexpr int BLD = 32 + (sizeof(BT) == 4 ? 4 : 8);
  constexpr int NDT = DP / 32;
  constexpr int NQF = DP / E::kKStep;

  __shared__ __attribute__((aligned(16))) T k_lds[32 * KLD];
  __shared__ __attribute__((aligned(16))) T v_lds[32 * KLD];
  __shared__ __attribute__((aligned(16))) T kt_lds[kF32 ? 1 : DP * TLD];
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

  const T* kbase = a.k + S.k_off + g * S.k_sg + h * S.k_sh;
  const T* vbase = a.v + S.v_off + g * S.v_sg + h * S.v_sh;
  const bool has_bias = a.bias != nullptr && S.b_off >= 0;
  const BT* bbase = has_bias ? a.bias + S.b_off + g * S.b_sg + h * S.b_sh : nullptr;
  const bool has_mask = a.mask != nullptr && S.m_off >= 0;
  const uint8_t* mbase = has_mask ? a.mask + S.m_off + g * S.m_sg : nullptr;
  const bool pair_mask = has_mask && S.m_si != 0;
  const bool write_full_dbias = a.dbias != nullptr && S.bias_mode == OOPS_BIAS_FULL;

  const int q_lane = qb * 128 + wave * 32 + lq;
  const bool qv = q_lane < Lq;
  Frag qf[NQF], df[NQF];
  {
    const T* qrow = a.q + S.q_off + g * S.q_sg + h * S.q_sh + (int64_t)q_lane * S.q_si;
    const T* drow = a.dout + S.do_off + g * S.do_sg + h * S.do_sh + (int64_t)q_lane * S.do_si;
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      if constexpr (kF32) {
        const int d = s * 2 + g2;
        qf[s] = (qv && d < D) ? qrow[d] : 0.0f;
        df[s] = (qv && d < D) ? drow[d] : 0.0f;
      } else {
        const uint4 z = make_uint4(0, 0, 0, 0);
        qf[s] = __builtin_bit_cast(Frag, qv ? load16(qrow, s * 16 + g2 * 8, D, vec) : z);
        df[s] = __builtin_bit_cast(Frag, qv ? load16(drow, s * 16 + g2 * 8, D, vec) : z);
      }
    }
  }
  const int64_t lidx = S.l_off + ((int64_t)g * H + h) * Lq + q_lane;
  const float lse2 = qv ? a.lse[lidx] : 0.0f;
  const float dlt = qv ? a.delta[lidx] : 0.0f;
  float* dbrow = write_full_dbias ? a.dbias + S.db_off + g * S.db_sg + h * S.db_sh + (int64_t)q_lane * S.db_si
                                  : nullptr;

  const float c1 = a.scale * kLog2e;
  f32x16 acc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) acc[t] = f32x16{};

  constexpr int CE = 16 / sizeof(T);
  constexpr int CPR = DP / CE;
  constexpr int BCE = 16 / sizeof(BT);
  constexpr int BCPR = 32 / BCE;

  for (int k0 = 0; k0 < Lk; k0 += 32) {
    __syncthreads();
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
        store_elems(&k_lds[r * KLD + col], ku);
        store_elems(&v_lds[r * KLD + col], vu);
      } else {
        *reinterpret_cast<uint4*>(&k_lds[r * KLD + col]) = ku;
        *reinterpret_cast<uint4*>(&v_lds[r * KLD + col]) = vu;
        const T* ke = reinterpret_cast<const T*>(&ku);
        const int pos = perm16(r);
#pragma unroll
        for (int i = 0; i < CE; ++i) kt_lds[(col + i) * TLD + pos] = ke[i];
      }
    }
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
          BT* dst = &b_lds[r * BLD + perm32(kc + i)];
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[e] = bu.e[i + e];
        }
      }
    }
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

    f32x16 sacc = f32x16{}, pacc = f32x16{};
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      Frag kf, vf;
      if constexpr (kF32) {
        kf = k_lds[lq * KLD + s * 2 + g2];
        vf = v_lds[lq * KLD + s * 2 + g2];
      } else {
        kf = __builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(&k_lds[lq * KLD + s * 16 + g2 * 8]));
        vf = __builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(&v_lds[lq * KLD + s * 16 + g2 * 8]));
      }
      sacc = E::mma(kf, qf[s], sacc);
      pacc = E::mma(vf, df[s], pacc);
    }

    float ds[16];
    {
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
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float p = __builtin_amdgcn_exp2f(x[j] - lse2);
        ds[j] = p * (pacc[j] - dlt);
      }
    }
    if (write_full_dbias && qv) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int key = k0 + kappa(g2, j);
        if (key < Lk) dbrow[key] = ds[j];
      }
    }
    // dQ^T += K^T dS^T
    if constexpr (kF32) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int key = kappa(g2, j);
#pragma unroll
        for (int t = 0; t < NDT; ++t) acc[t] = E::mma(k_lds[key * KLD + t * 32 + lq], ds[j], acc[t]);
      }
    } else {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const Frag sf = pack8<T>(&ds[8 * m]);
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
          const Frag kf = __builtin_bit_cast(
              Frag, *reinterpret_cast<const uint4*>(&kt_lds[(t * 32 + lq) * TLD + 16 * m + g2 * 8]));
          acc[t] = E::mma(kf, sf, acc[t]);
        }
      }
    }
  }

  if (qv && a.dq != nullptr) {
    T* row = a.dq + S.q_off + g * S.q_sg + h * S.q_sh + (int64_t)q_lane * S.q_si;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = t * 32 + kappa(g2, i);
        if (d < D) row[d] = E::from_f(acc[t][i] * a.scale);
      }
    }
  }
}

// ------------------------------------------------------------------ dK, dV
template <typename T, typename BT, int DP>
__global__ __launch_bounds__(256) void attn_dkv_kernel(BwdArgs a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr bool kF32 = sizeof(T) == 4;
  constexpr int KLD = DP + (kF32 ? 1 : 8);
  constexpr int TLD = 32 + 8;
  constexpr int BLD = 32 + (sizeof(BT) == 4 ? 4 : 8);  // transposed bias: [key][query]
  constexpr int NDT = DP / 32;
  constexpr int NQF = DP / E::kKStep;

  __shared__ __attribute__((aligned(16))) T q_lds[32 * KLD];
  __shared__ __attribute__((aligned(16))) T do_lds[32 * KLD];
  __shared__ __attribute__((aligned(16))) T qt_lds[kF32 ? 1 : DP * TLD];
  __shared__ __attribute__((aligned(16))) T dot_lds[kF32 ? 1 : DP * TLD];
  __shared__ __attribute__((aligned(16))) BT bt_lds[128 * BLD];
  __shared__ __attribute__((aligned(16))) uint8_t mt_lds[128 * 32];
  __shared__ __attribute__((aligned(16))) float lse_lds[32];
  __shared__ __attribute__((aligned(16))) float dlt_lds[32];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int g2 = lane >> 5;

  int64_t tile = blockIdx.x;
  const Sample* tab = reinterpret_cast<const Sample*>(a.table);
  const int H = a.num_heads;
  const int s_idx = find_sample(tile, tab, a.num_samples, a.uniform_tiles,
                                [&](const Sample& s) { return s.G * H * cdiv(s.Lk, 128); });
  if (s_idx < 0) return;
  const Sample& S = tab[s_idx];
  const int64_t G = S.G;
  const int Lq = (int)S.Lq, Lk = (int)S.Lk;
  const int g = (int)(tile % G);
  const int64_t rest = tile / G;
  const int nkb = (int)cdiv(Lk, 128);
  const int kb = (int)(rest % nkb);
  const int h = (int)(rest / nkb);
  const int D = a.head_size;
  const bool vec = a.vec_ok;

  const T* qbase = a.q + S.q_off + g * S.q_sg + h * S.q_sh;
  const T* dobase = a.dout + S.do_off + g * S.do_sg + h * S.do_sh;
  const bool has_bias = a.bias != nullptr && S.b_off >= 0;
  const BT* bbase = has_bias ? a.bias + S.b_off + g * S.b_sg + h * S.b_sh : nullptr;
  const bool has_mask = a.mask != nullptr && S.m_off >= 0;
  const uint8_t* mbase = has_mask ? a.mask + S.m_off + g * S.m_sg : nullptr;
  const bool pair_mask = has_mask && S.m_si != 0;
  const float* lse_row = a.lse + S.l_off + ((int64_t)g * H + h) * Lq;
  const float* dlt_row = a.delta + S.l_off + ((int64_t)g * H + h) * Lq;

  // this lane's key: K, V as B operands (lane = key, k = head dim)
  const int key_lane = kb * 128 + wave * 32 + lq;
  bool kvalid = key_lane < Lk;
  if (kvalid && has_mask && !pair_mask) kvalid = mbase[key_lane] != 0;
  Frag kf[NQF], vf[NQF];
  {
    const T* krow = a.k + S.k_off + g * S.k_sg + h * S.k_sh + (int64_t)key_lane * S.k_si;
    const T* vrow = a.v + S.v_off + g * S.v_sg + h * S.v_sh + (int64_t)key_lane * S.v_si;
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      if constexpr (kF32) {
        const int d = s * 2 + g2;
        kf[s] = (kvalid && d < D) ? krow[d] : 0.0f;
        vf[s] = (kvalid && d < D) ? vrow[d] : 0.0f;
      } else {
        const uint4 z = make_uint4(0, 0, 0, 0);
        kf[s] = __builtin_bit_cast(Frag, kvalid ? load16(krow, s * 16 + g2 * 8, D, vec) : z);
        vf[s] = __builtin_bit_cast(Frag, kvalid ? load16(vrow, s * 16 + g2 * 8, D, vec) : z);
      }
    }
  }

  const float c1 = a.scale * kLog2e;
  f32x16 dk[NDT], dv[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) dk[t] = dv[t] = f32x16{};

  constexpr int CE = 16 / sizeof(T);
  constexpr int CPR = DP / CE;
  constexpr int BCE = 16 / sizeof(BT);

  for (int q0 = 0; q0 < Lq; q0 += 32) {
    __syncthreads();
    for (int c = tid; c < 32 * CPR; c += 256) {
      const int r = c / CPR;
      const int col = (c % CPR) * CE;
      const int q = q0 + r;
      uint4 qu = make_uint4(0, 0, 0, 0), du = make_uint4(0, 0, 0, 0);
      if (q < Lq) {
        qu = load16(qbase + (int64_t)q * S.q_si, col, D, vec);
        du = load16(dobase + (int64_t)q * S.do_si, col, D, vec);
      }
      if constexpr (kF32) {
        store_elems(&q_lds[r * KLD + col], qu);
        store_elems(&do_lds[r * KLD + col], du);
      } else {
        *reinterpret_cast<uint4*>(&q_lds[r * KLD + col]) = qu;
        *reinterpret_cast<uint4*>(&do_lds[r * KLD + col]) = du;
        const T* qe = reinterpret_cast<const T*>(&qu);
        const T* de = reinterpret_cast<const T*>(&du);
        const int pos = perm16(r);
#pragma unroll
        for (int i = 0; i < CE; ++i) {
          qt_lds[(col + i) * TLD + pos] = qe[i];
          dot_lds[(col + i) * TLD + pos] = de[i];
        }
      }
    }
    if (tid < 32) {
      const int q = q0 + tid;
      // out-of-range queries: P = exp2(x - inf) = 0, delta = 0
      lse_lds[perm32(tid)] = q < Lq ? lse_row[q] : __builtin_huge_valf();
      dlt_lds[perm32(tid)] = q < Lq ? dlt_row[q] : 0.0f;
    }
    if (has_bias) {
      // bias[q][key] for 32 queries x 128 keys, stored transposed [key][perm32(q)]
      constexpr int KCPR = 128 / BCE;
      for (int c = tid; c < 32 * KCPR; c += 256) {
        const int r = c / KCPR;  // query
        const int kc = (c % KCPR) * BCE;
        const int q = q0 + r;
        const int key0 = kb * 128 + kc;
        union {
          uint4 u;
          BT e[BCE];
        } bu;
        bu.u = make_uint4(0, 0, 0, 0);
        if (q < Lq) bu.u = load16(bbase + (int64_t)q * S.b_si, key0, Lk, vec && (key0 + BCE <= Lk));
        const int pos = perm32(r);
#pragma unroll
        for (int e = 0; e < BCE; ++e) bt_lds[(kc + e) * BLD + pos] = bu.e[e];
      }
    }
    if (pair_mask) {
      for (int c = tid; c < 32 * 128; c += 256) {
        const int r = c >> 7;  // query
        const int kk = c & 127;
        const int q = q0 + r, key = kb * 128 + kk;
        uint8_t keep = 0;
        if (q < Lq && key < Lk) keep = mbase[(int64_t)q * S.m_si + key] != 0;
        mt_lds[kk * 32 + perm32(r)] = keep;
      }
    }
    __syncthreads();

    // S = Q K^T, dP = dO V^T  (rows: queries kappa(g2, i), column: this lane's key)
    f32x16 sacc = f32x16{}, pacc = f32x16{};
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      Frag qa, da;
      if constexpr (kF32) {
        qa = q_lds[lq * KLD + s * 2 + g2];
        da = do_lds[lq * KLD + s * 2 + g2];
      } else {
        qa = __builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(&q_lds[lq * KLD + s * 16 + g2 * 8]));
        da = __builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(&do_lds[lq * KLD + s * 16 + g2 * 8]));
      }
      sacc = E::mma(qa, kf[s], sacc);
      pacc = E::mma(da, vf[s], pacc);
    }
    float p[16], ds[16];
    {
      const float* lrow = &lse_lds[g2 * 16];
      const float* drow = &dlt_lds[g2 * 16];
      const int krow = wave * 32 + lq;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float x = has_bias ? __builtin_fmaf(sacc[i], c1, Elem<BT>::to_f(bt_lds[krow * BLD + g2 * 16 + i]) * kLog2e)
                           : sacc[i] * c1;
        bool keep = kvalid;
        if (pair_mask) keep = keep && mt_lds[krow * 32 + g2 * 16 + i] != 0;
        x = keep ? x : kNegInf;
        p[i] = __builtin_amdgcn_exp2f(x - lrow[i]);
        ds[i] = p[i] * (pacc[i] - drow[i]);
      }
    }
    // dV^T += dO^T P ; dK^T += Q^T dS   (k = query)
    if constexpr (kF32) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int q = kappa(g2, i);
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
          dv[t] = E::mma(do_lds[q * KLD + t * 32 + lq], p[i], dv[t]);
          dk[t] = E::mma(q_lds[q * KLD + t * 32 + lq], ds[i], dk[t]);
        }
      }
    } else {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const Frag pf = pack8<T>(&p[8 * m]);
        const Frag sf = pack8<T>(&ds[8 * m]);
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
          const int off = (t * 32 + lq) * TLD + 16 * m + g2 * 8;
          const Frag da = __builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(&dot_lds[off]));
          const Frag qa = __builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(&qt_lds[off]));
          dv[t] = E::mma(da, pf, dv[t]);
          dk[t] = E::mma(qa, sf, dk[t]);
        }
      }
    }
  }

  if (key_lane < Lk) {
    T* krow = a.dk ? a.dk + S.k_off + g * S.k_sg + h * S.k_sh + (int64_t)key_lane * S.k_si : nullptr;
    T* vrow = a.dv ? a.dv + S.v_off + g * S.v_sg + h * S.v_sh + (int64_t)key_lane * S.v_si : nullptr;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = t * 32 + kappa(g2, i);
        if (d < D) {
          if (krow) krow[d] = E::from_f(kvalid ? dk[t][i] * a.scale : 0.0f);
          if (vrow) vrow[d] = E::from_f(kvalid ? dv[t][i] : 0.0f);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ shared dBias
template <typename T, typename BT, int DP>
__global__ __launch_bounds__(256) void attn_dbias_shared_kernel(BwdArgs a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr bool kF32 = sizeof(T) == 4;
  constexpr int KLD = DP + (kF32 ? 1 : 8);
  constexpr int NQF = DP / E::kKStep;

  __shared__ __attribute__((aligned(16))) T k_lds[32 * KLD];
  __shared__ __attribute__((aligned(16))) T v_lds[32 * KLD];
  __shared__ __attribute__((aligned(16))) uint8_t m_lds[128 * 32];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int g2 = lane >> 5;
  const int P = a.parts;

  int64_t tile = blockIdx.x;
  const Sample* tab = reinterpret_cast<const Sample*>(a.table);
  const int H = a.num_heads;
  const int s_idx = find_sample(tile, tab, a.num_samples, a.uniform_tiles, [&](const Sample& s) {
    return s.bias_mode == OOPS_BIAS_SHARED ? H * cdiv(s.Lq, 128) * cdiv(s.Lk, 32) * P : (int64_t)0;
  });
  if (s_idx < 0) return;
  const Sample& S = tab[s_idx];
  const int64_t G = S.G;
  const int Lq = (int)S.Lq, Lk = (int)S.Lk;
  const int nkb = (int)cdiv(Lk, 32);
  const int nqb = (int)cdiv(Lq, 128);
  const int kb = (int)(tile % nkb);
  int64_t rest = tile / nkb;
  const int qb = (int)(rest % nqb);
  rest /= nqb;
  const int h = (int)(rest % H);
  const int part = (int)(rest / H);
  const int64_t g_begin = G * part / P, g_end = G * (part + 1) / P;
  const int D = a.head_size;
  const bool vec = a.vec_ok;
  const bool has_mask = a.mask != nullptr && S.m_off >= 0;
  const bool pair_mask = has_mask && S.m_si != 0;

  const int q_lane = qb * 128 + wave * 32 + lq;
  const bool qv = q_lane < Lq;
  const int k0 = kb * 32;
  const float c1 = a.scale * kLog2e;

  // bias block, shared by every group: lane's query x keys kappa(g2, j)
  float xb[16];
  {
    const BT* brow = a.bias + S.b_off + h * S.b_sh + (int64_t)q_lane * S.b_si;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int key = k0 + kappa(g2, j);
      xb[j] = (qv && key < Lk) ? Elem<BT>::to_f(brow[key]) * kLog2e : 0.0f;
    }
  }
  float acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.0f;

  constexpr int CE = 16 / sizeof(T);
  constexpr int CPR = DP / CE;

  for (int64_t g = g_begin; g < g_end; ++g) {
    const uint8_t* mbase = has_mask ? a.mask + S.m_off + g * S.m_sg : nullptr;
    __syncthreads();
    {
      const T* kbase = a.k + S.k_off + g * S.k_sg + h * S.k_sh;
      const T* vbase = a.v + S.v_off + g * S.v_sg + h * S.v_sh;
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
          store_elems(&k_lds[r * KLD + col], ku);
          store_elems(&v_lds[r * KLD + col], vu);
        } else {
          *reinterpret_cast<uint4*>(&k_lds[r * KLD + col]) = ku;
          *reinterpret_cast<uint4*>(&v_lds[r * KLD + col]) = vu;
        }
      }
      if (has_mask) {
        const int rows = pair_mask ? 128 : 1;
        for (int c = tid; c < rows * 32; c += 256) {
          const int r = c >> 5;
          const int kk = c & 31;
          const int q = qb * 128 + r, key = k0 + kk;
          uint8_t keep = 0;
          if (key < Lk && (!pair_mask || q < Lq))
            keep = mbase[(pair_mask ? (int64_t)q * S.m_si : 0) + key] != 0;
          m_lds[r * 32 + perm32(kk)] = keep;
        }
      }
    }
    Frag qf[NQF], df[NQF];
    {
      const T* qrow = a.q + S.q_off + g * S.q_sg + h * S.q_sh + (int64_t)q_lane * S.q_si;
      const T* drow = a.dout + S.do_off + g * S.do_sg + h * S.do_sh + (int64_t)q_lane * S.do_si;
#pragma unroll
      for (int s = 0; s < NQF; ++s) {
        if constexpr (kF32) {
          const int d = s * 2 + g2;
          qf[s] = (qv && d < D) ? qrow[d] : 0.0f;
          df[s] = (qv && d < D) ? drow[d] : 0.0f;
        } else {
          const uint4 z = make_uint4(0, 0, 0, 0);
          qf[s] = __builtin_bit_cast(Frag, qv ? load16(qrow, s * 16 + g2 * 8, D, vec) : z);
          df[s] = __builtin_bit_cast(Frag, qv ? load16(drow, s * 16 + g2 * 8, D, vec) : z);
        }
      }
    }
    const int64_t lidx = S.l_off + (g * H + h) * Lq + q_lane;
    const float lse2 = qv ? a.lse[lidx] : __builtin_huge_valf();
    const float dlt = qv ? a.delta[lidx] : 0.0f;
    __syncthreads();

    f32x16 sacc = f32x16{}, pacc = f32x16{};
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      Frag kf, vf;
      if constexpr (kF32) {
        kf = k_lds[lq * KLD + s * 2 + g2];
        vf = v_lds[lq * KLD + s * 2 + g2];
      } else {
        kf = __builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(&k_lds[lq * KLD + s * 16 + g2 * 8]));
        vf = __builtin_bit_cast(Frag, *reinterpret_cast<const uint4*>(&v_lds[lq * KLD + s * 16 + g2 * 8]));
      }
      sacc = E::mma(kf, qf[s], sacc);
      pacc = E::mma(vf, df[s], pacc);
    }
    const uint8_t* mrow = &m_lds[(pair_mask ? wave * 32 + lq : 0) * 32 + g2 * 16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float x = __builtin_fmaf(sacc[j], c1, xb[j]);
      bool keep = k0 + kappa(g2, j) < Lk;
      if (has_mask) keep = keep && mrow[j] != 0;
      x = keep ? x : kNegInf;
      const float p = __builtin_amdgcn_exp2f(x - lse2);
      acc[j] += p * (pacc[j] - dlt);
    }
  }

  if (qv) {
    float* dst = P == 1 ? a.dbias : a.dbias_part + (int64_t)part * a.dbias_extent;
    float* row = dst + S.db_off + h * S.db_sh + (int64_t)q_lane * S.db_si;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int key = k0 + kappa(g2, j);
      if (key < Lk) row[key] = acc[j];
    }
  }
}

// sum of the per-part slabs into dBias (shared-bias samples only)
template <typename T, typename BT, int DP>
__global__ __launch_bounds__(256) void attn_dbias_reduce_kernel(BwdArgs a) {
  int64_t tile = blockIdx.x;
  const Sample* tab = reinterpret_cast<const Sample*>(a.table);
  const int H = a.num_heads;
  const int s_idx = find_sample(tile, tab, a.num_samples, a.uniform_tiles, [&](const Sample& s) {
    return s.bias_mode == OOPS_BIAS_SHARED ? cdiv(H * s.Lq * s.Lk, 256) : (int64_t)0;
  });
  if (s_idx < 0) return;
  const Sample& S = tab[s_idx];
  const int64_t e = tile * 256 + threadIdx.x;
  const int64_t Lk = S.Lk, Lq = S.Lq;
  if (e >= H * Lq * Lk) return;
  // a contiguous [h][q][k] slab (the usual case) needs no index arithmetic
  int64_t off = S.db_off + e;
  if (S.db_si != Lk || S.db_sh != Lq * Lk) {
    const int64_t key = e % Lk;
    const int64_t q = (e / Lk) % Lq;
    const int64_t h = e / (Lk * Lq);
    off = S.db_off + h * S.db_sh + q * S.db_si + key;
  }
  // per-sample parts (fast path): a sample with one part wrote dBias directly.  In a split batch the
  // samples longer than fused_max_lq had the separate dBias kernel and its parts
  const int parts = a.fused_max_lq > 0 && S.Lq > a.fused_max_lq ? parts_for(S.G, a.part_groups_rest, a.parts_rest)
                    : a.part_groups > 0                        ? parts_for(S.G, a.part_groups, a.parts)
                                                               : a.parts;
  if (parts < 2) return;
  // the parts in order, eight loads in flight at a time
  const float* src = a.dbias_part + off;
  float acc = 0.0f;
  int p = 0;
  for (; p + 8 <= parts; p += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = src[(int64_t)(p + j) * a.dbias_extent];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += v[j];
  }
  for (; p < parts; ++p) acc += src[(int64_t)p * a.dbias_extent];
  a.dbias[off] = acc;
}

#define OOPS_BWD_INST(T, BT, DP)                                                \
  template __global__ void attn_delta_kernel<T, BT, DP>(BwdArgsT<T, BT>);               \
  template __global__ void attn_dq_kernel<T, BT, DP>(BwdArgsT<T, BT>);                  \
  template __global__ void attn_dkv_kernel<T, BT, DP>(BwdArgsT<T, BT>);                 \
  template __global__ void attn_dbias_shared_kernel<T, BT, DP>(BwdArgsT<T, BT>);        \
  template __global__ void attn_dbias_reduce_kernel<T, BT, DP>(BwdArgsT<T, BT>);
OOPS_FOR_EACH_CONFIG(OOPS_BWD_INST)

}  // namespace oops

namespace oops {

int head_group_of(const oops_attn_geometry& geo) { return head_group(geo); }

hipError_t launch_backward(const oops_attn_geometry& geo, const Plan& plan, const void* q, const void* k,
                           const void* v, const uint8_t* mask, const void* bias, const void* out,
                           const void* out_lo, const float* lse, const void* dout, void* dq, void* dk, void* dv,
                           float* dbias, float* delta, float* ld_pack, void* qdo_compact, float* dbias_part,
                           void* bias_frag, hipStream_t stream) {
  const bool fast = backward_fast_ok(geo, plan);
  const int phases = geo.phases == 0 ? 0xF : geo.phases;
  hipError_t err = hipSuccess;
  // the fragment-major bias copy feeds the fast dQ and dK/dV kernels
  const bool use_bf = fast && plan.bias_frag && (phases & (OOPS_PHASE_DQ | OOPS_PHASE_DKV));
  if (use_bf) {
    err = launch_bias_frag(geo, plan, bias, bias_frag, stream);
    if (err != hipSuccess) return err;
  }
  // the fast dQ kernel writes the LSE/delta pack and the compact Q / dO of the
  // fused dK/dV + dBias kernel
  const bool fusable = fast && ld_pack != nullptr && qdo_compact != nullptr && dkvb_fused_ok(geo, plan);
  const size_t compact_elems = (size_t)plan.lse_extent * kCompactRow;
  void* qc = fusable ? qdo_compact : nullptr;
  void* dc = fusable ? static_cast<char*>(qdo_compact) + compact_elems * 2 : nullptr;
  const BwdLaunch L{q, k, v, out, out_lo, dout, bias, mask, lse, delta, fusable ? ld_pack : nullptr, qc, dc, dq, dk,
                    dv, dbias, dbias_part, use_bf ? bias_frag : nullptr};
  const bool ok = dispatch_config(geo.dtype, geo.bias_dtype, plan.dp, [&](auto t, auto bt, auto dpc) {
    using T = typename decltype(t)::type;
    using BT = typename decltype(bt)::type;
    constexpr int DP = decltype(dpc)::value;
    BwdArgsT<T, BT> a;
    fill_bwd_args(a, geo, plan, L);
    const dim3 block(256);
    auto check = [&]() {
      if (err == hipSuccess) err = hipGetLastError();
    };
    const bool need_dq = dq != nullptr || (a.dbias != nullptr && plan.any_full);
    const bool run_dq = (phases & OOPS_PHASE_DQ) && need_dq && plan.fwd_tiles > 0;
    // the fast dQ kernel computes delta itself when it runs first
    const bool fused_delta = fast && run_dq;
    if ((phases & OOPS_PHASE_DELTA) && !fused_delta) {
      a.uniform_tiles = plan.delta_uniform;
      hipLaunchKernelGGL((attn_delta_kernel<T, BT, DP>), dim3((unsigned)plan.delta_tiles), block, 0, stream, a);
      check();
    }
    if (run_dq) {
      if (fast) {
        if (err == hipSuccess) err = launch_dq_fast(geo, plan, L, fused_delta, stream);
      } else {
        a.uniform_tiles = plan.fwd_uniform;
        hipLaunchKernelGGL((attn_dq_kernel<T, BT, DP>), dim3((unsigned)plan.fwd_tiles), block, 0, stream, a);
        check();
      }
    }
    // dK, dV and the shared dBias in one kernel when it serves the geometry and
    // the pack is ready: the fast dQ kernel has just written it, or (a call
    // without the dQ and delta phases) a previous call's did
    const bool pack_ready = (fast && run_dq) || !(phases & (OOPS_PHASE_DQ | OOPS_PHASE_DELTA));
    const bool fused = fusable && pack_ready && (phases & OOPS_PHASE_DKV) && (phases & OOPS_PHASE_DBIAS) &&
                       a.dbias != nullptr;
    if (fused) {
      if (err == hipSuccess) err = launch_dkvb_fused(geo, plan, L, stream);
      // a split batch: the samples too long for the fused kernel take the separate kernels
      if (plan.fused_split) {
        if (err == hipSuccess) err = launch_dkv_fast(geo, plan, L, stream, true);
        if (err == hipSuccess) err = launch_dbias_fast(geo, plan, L, stream, true);
        a.fused_max_lq = kFusedMaxLen;
        a.parts_rest = plan.fast_parts;
        a.part_groups_rest = plan.fast_part_groups;
      }
      a.parts = plan.fused_parts;
      a.part_groups = plan.fused_part_groups;
      if (a.parts > 1 || (plan.fused_split && plan.fast_parts > 1)) {
        a.uniform_tiles = plan.sred_uniform;
        hipLaunchKernelGGL((attn_dbias_reduce_kernel<T, BT, DP>), dim3((unsigned)plan.sred_tiles), block, 0,
                           stream, a);
        check();
      }
      return;
    }
    if ((phases & OOPS_PHASE_DKV) && (dk != nullptr || dv != nullptr) && plan.dkv_tiles > 0) {
      if (fast) {
        if (err == hipSuccess) err = launch_dkv_fast(geo, plan, L, stream);
      } else {
        a.uniform_tiles = plan.dkv_uniform;
        hipLaunchKernelGGL((attn_dkv_kernel<T, BT, DP>), dim3((unsigned)plan.dkv_tiles), block, 0, stream, a);
        check();
      }
    }
    if ((phases & OOPS_PHASE_DBIAS) && a.dbias != nullptr && plan.any_shared && plan.sbias_tiles > 0) {
      if (fast) {
        if (err == hipSuccess) err = launch_dbias_fast(geo, plan, L, stream);
        a.parts = plan.fast_parts;
        a.part_groups = plan.fast_part_groups;
      } else {
        a.uniform_tiles = plan.sbias_uniform;
        hipLaunchKernelGGL((attn_dbias_shared_kernel<T, BT, DP>), dim3((unsigned)plan.sbias_tiles), block, 0,
                           stream, a);
        check();
      }
      if (a.parts > 1) {
        a.uniform_tiles = plan.sred_uniform;
        hipLaunchKernelGGL((attn_dbias_reduce_kernel<T, BT, DP>), dim3((unsigned)plan.sred_tiles), block, 0,
                           stream, a);
        check();
      }
    }
  });
  return ok ? err : hipErrorInvalidValue;
}

}  // namespace oops
