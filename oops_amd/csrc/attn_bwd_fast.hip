// Backward fast path for 16-bit Q/K/V (bias in the same dtype or absent),
// head size <= 64 and a multiple of 8.
//
// attn_dkv_fast_kernel: one workgroup = 4 wavefronts = 128 keys of one
// (sample, group, head); wave w owns keys w*32 .. w*32+31 and keeps their K
// and V fragments in registers.  The query axis is walked in steps of 64.
// Per step the workgroup stages Q, dO (row-major) and -LSE, -delta in a
// 3-buffer LDS ring; each wave computes, for two 32-query row tiles,
//   S  = Q K^T              (+ bias through an identity MFMA: the bias rows
//                            are the A operand, I(1/scale) the B operand),
//   dP = dO V^T - delta     (-delta is the accumulator input of the MFMA),
//   P  = exp2(S * scale * log2 e - LSE),  dS = P * dP,
//   dV^T += dO^T P,  dK^T += Q^T dS      (dO^T, Q^T by LDS transpose reads),
// with the key as MFMA column, so P and dS go from accumulators straight into
// the next MFMA's k-operand.
//
// Semantics: the reference's _backward_key_value
// (oops/attention/triangle/triton/kernel.py:569-717) with
// softmax_backward_dscores (oops/attention/flash/triton/kernel.py:53-62):
// masked keys get dK = dV = 0; rows with no valid key carry LSE = 0 and
// contribute nothing.
#include "attn_fast_common.h"

namespace oops {

using namespace fast;

template <typename T, int DP, bool HAS_BIAS>
__global__ __launch_bounds__(256, 2) void attn_dkv_fast_kernel(BwdArgsT<T, T> a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int LD = DP + 8;        // Q / dO tile row (elements)
  constexpr int TBUF = 64 * LD;     // elements per tile buffer
  constexpr int NDT = DP / 32;
  constexpr int NQF = DP / 16;
  constexpr int NCH = DP / 32;      // 16-byte chunks of Q (and dO) per thread per step

  __shared__ __attribute__((aligned(16))) T q_lds[3 * TBUF];
  __shared__ __attribute__((aligned(16))) T do_lds[3 * TBUF];
  __shared__ __attribute__((aligned(16))) float nlse_lds[3 * 64];  // -LSE, rows permuted
  __shared__ __attribute__((aligned(16))) float ndlt_lds[3 * 64];  // -delta, rows permuted

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int g2 = lane >> 5;

  // XCD-aware order (see attn_fwd_fast.hip): logical (head group, g, head, key block)
  int64_t tile = xcd_tile(blockIdx.x, gridDim.x);
  if (tile >= a.total_tiles) return;
  const Sample* tab = reinterpret_cast<const Sample*>(a.table);
  const int H = a.num_heads;
  const int s_idx = find_sample(tile, tab, a.num_samples, a.uniform_tiles,
                                [&](const Sample& s) { return s.G * H * cdiv(s.Lk, 128); });
  if (s_idx < 0) return;
  const Sample& S = tab[__builtin_amdgcn_readfirstlane(s_idx)];
  const int64_t G = S.G;
  const int Lq = (int)S.Lq, Lk = (int)S.Lk;
  const int nkb = (int)cdiv(Lk, 128);
  const int HG = a.head_group;
  const int kb = (int)(tile % nkb);
  int64_t rest = tile / nkb;
  const int hh = (int)(rest % HG);
  rest /= HG;
  const int g = (int)(rest % G);
  const int h = (int)(rest / G) * HG + hh;
  const int D = a.head_size;
  const int q_si = (int)S.q_si, do_si = (int)S.do_si, b_si = (int)S.b_si;
  const int nsteps = (Lq + 63) >> 6;

  // ---- this lane's key: K, V fragments (B operands: lane = key, k = head dim)
  const int key = kb * 128 + wave * 32 + lq;
  bool kvalid = key < Lk;
  const bool has_mask = a.mask != nullptr && S.m_off >= 0;
  if (kvalid && has_mask) kvalid = a.mask[S.m_off + g * S.m_sg + key] != 0;
  const bool wave_masked = __any(!kvalid);
  Frag kf[NQF], vf[NQF];
  {
    const T* kbase = a.k + S.k_off + g * S.k_sg + h * S.k_sh;
    const T* vbase = a.v + S.v_off + g * S.v_sg + h * S.v_sh;
    const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc(kbase, (uint32_t)(((int64_t)(Lk - 1) * S.k_si + D) * 2));
    const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc(vbase, (uint32_t)(((int64_t)(Lk - 1) * S.v_si + D) * 2));
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      const int col = s * 16 + g2 * 8;
      const bool ok = kvalid && col < D;
      kf[s] = __builtin_bit_cast(Frag, buffer_load16(k_rsrc, ok ? (uint32_t)((key * (int)S.k_si + col) * 2) : kOut));
      vf[s] = __builtin_bit_cast(Frag, buffer_load16(v_rsrc, ok ? (uint32_t)((key * (int)S.v_si + col) * 2) : kOut));
    }
  }
  Frag ident[2];
  identity_frags<T>(ident, 1.0f / a.scale, lane);

  // ---- per-thread staging offsets (bytes); the step adds q0 * stride via soffset
  const T* qbase = a.q + S.q_off + g * S.q_sg + h * S.q_sh;
  const T* dobase = a.dout + S.do_off + g * S.do_sg + h * S.do_sh;
  const __amdgpu_buffer_rsrc_t q_rsrc = make_rsrc(qbase, (uint32_t)(((int64_t)(Lq - 1) * q_si + D) * 2));
  const __amdgpu_buffer_rsrc_t do_rsrc = make_rsrc(dobase, (uint32_t)(((int64_t)(Lq - 1) * do_si + D) * 2));
  uint32_t st_row[NCH], q_off[NCH], do_off[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = tid + 256 * i;
    const int r = c / (DP / 8);
    const int col = (c % (DP / 8)) * 8;
    st_row[i] = r;
    q_off[i] = col < D ? (uint32_t)((r * q_si + col) * 2) : kOut;
    do_off[i] = col < D ? (uint32_t)((r * do_si + col) * 2) : kOut;
  }
  const float* lse_row = a.lse + S.l_off + ((int64_t)g * H + h) * Lq;
  const float* dlt_row = a.delta + S.l_off + ((int64_t)g * H + h) * Lq;
  // bias rows of this wave's keys: A fragments (lane = query, 8 consecutive keys)
  const T* bbase = HAS_BIAS ? a.bias + S.b_off + g * S.b_sg + h * S.b_sh : a.q;
  const __amdgpu_buffer_rsrc_t b_rsrc =
      make_rsrc(bbase, HAS_BIAS ? (uint32_t)(((int64_t)(Lq - 1) * b_si + Lk) * 2) : 0u);
  const int kw = kb * 128 + wave * 32;  // first key of this wave

  struct Stage {
    uint4 q[NCH], d[NCH];
    float lse, dlt;
  };
  auto load_stage = [&](int step, Stage& st) {
    const int q0 = step * 64;
    const uint32_t qs = (uint32_t)(q0 * q_si * 2), ds = (uint32_t)(q0 * do_si * 2);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const bool ok = q0 + (int)st_row[i] < Lq;
      st.q[i] = buffer_load16_s(q_rsrc, ok ? q_off[i] : kOut, qs);
      st.d[i] = buffer_load16_s(do_rsrc, ok ? do_off[i] : kOut, ds);
    }
    if (tid < 64) {
      const int q = q0 + tid;
      // rows past Lq: P = exp2(x - inf) = 0 and delta = 0
      st.lse = q < Lq ? lse_row[q] : __builtin_huge_valf();
      st.dlt = q < Lq ? dlt_row[q] : 0.0f;
    }
  };
  auto store_stage = [&](int buf, const Stage& st) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + 256 * i;
      const int r = c / (DP / 8);
      const int col = (c % (DP / 8)) * 8;
      *reinterpret_cast<uint4*>(&q_lds[buf * TBUF + r * LD + col]) = st.q[i];
      *reinterpret_cast<uint4*>(&do_lds[buf * TBUF + r * LD + col]) = st.d[i];
    }
    if (tid < 64) {
      const int pos = (tid & 32) + perm32(tid & 31);
      nlse_lds[buf * 64 + pos] = -st.lse;
      ndlt_lds[buf * 64 + pos] = -st.dlt;
    }
  };

  const float c1 = a.scale * kLog2e;
  f32x16 dk[NDT], dv[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) dk[t] = dv[t] = f32x16{};

  // one step: two 32-query row tiles of LDS buffer buf against this wave's keys
  auto compute = [&](int buf, int q0, const uint4 (&bias)[2][2]) {
    const T* qt = &q_lds[buf * TBUF];
    const T* dt = &do_lds[buf * TBUF];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      f32x16 sacc;
      if constexpr (HAS_BIAS) {
        sacc = E::mma(__builtin_bit_cast(Frag, bias[r][0]), ident[0], f32x16{});
        sacc = E::mma(__builtin_bit_cast(Frag, bias[r][1]), ident[1], sacc);
      } else {
        sacc = f32x16{};
      }
      f32x16 pacc = *reinterpret_cast<const f32x16*>(&ndlt_lds[buf * 64 + 32 * r + g2 * 16]);
#pragma unroll
      for (int s = 0; s < NQF; ++s) {
        sacc = E::mma(lds_frag<T>(qt + (32 * r + lq) * LD + s * 16 + g2 * 8), kf[s], sacc);
        pacc = E::mma(lds_frag<T>(dt + (32 * r + lq) * LD + s * 16 + g2 * 8), vf[s], pacc);
      }
      const f32x16 nlse = *reinterpret_cast<const f32x16*>(&nlse_lds[buf * 64 + 32 * r + g2 * 16]);
      float p[16], ds[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        p[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j], c1, nlse[j]));
        if (wave_masked) p[j] = kvalid ? p[j] : 0.0f;
        ds[j] = p[j] * pacc[j];
      }
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const Frag pf = pack8<T>(&p[8 * m]);
        const Frag sf = pack8<T>(&ds[8 * m]);
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
          dv[t] = E::mma(lds_read_tr_frag<T>(dt, LD, 32 * r + 16 * m, 32 * t, lane), pf, dv[t]);
          dk[t] = E::mma(lds_read_tr_frag<T>(qt, LD, 32 * r + 16 * m, 32 * t, lane), sf, dk[t]);
        }
      }
    }
  };
  auto load_bias = [&](int step, uint4 (&bias)[2][2]) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int q = step * 64 + 32 * r + lq;
#pragma unroll
      for (int c = 0; c < 2; ++c)
        bias[r][c] = buffer_load16_s(
            b_rsrc, q < Lq ? (uint32_t)((q * b_si + kw + 16 * c + g2 * 8) * 2) : kOut, 0);
    }
  };

  // ---- pipeline: step i computes buffer i % 3; the stage of step i+2
  // (loaded during step i-1) is written at the top of step i.
  Stage stg;
  uint4 bias_a[2][2], bias_b[2][2];
  if (nsteps > 0) {
    load_stage(0, stg);
    if constexpr (HAS_BIAS) load_bias(0, bias_a);
    store_stage(0, stg);
  }
  if (nsteps > 1) {
    load_stage(1, stg);
    if constexpr (HAS_BIAS) load_bias(1, bias_b);
    store_stage(1, stg);
  }
  if (nsteps > 2) load_stage(2, stg);
  vmem_wait_all();
  __syncthreads();
  int buf = 0;
  auto step = [&](int i, uint4 (&bias_cur)[2][2]) {
    const int b1 = buf == 2 ? 0 : buf + 1;
    const int b2 = b1 == 2 ? 0 : b1 + 1;
    if (i + 2 < nsteps) store_stage(b2, stg);
    if (i + 3 < nsteps) load_stage(i + 3, stg);
    compute(buf, i * 64, bias_cur);
    if constexpr (HAS_BIAS)
      if (i + 2 < nsteps) load_bias(i + 2, bias_cur);
    lds_barrier();
    buf = b1;
  };
  for (int i = 0; i < nsteps; i += 2) {
    step(i, bias_a);
    if (i + 1 >= nsteps) break;
    step(i + 1, bias_b);
  }

  // ---- write dK = scale * dK^T^T, dV (zero for masked keys)
  if (key < Lk) {
    T* krow = a.dk ? a.dk + S.k_off + g * S.k_sg + h * S.k_sh + (int64_t)key * S.k_si : nullptr;
    T* vrow = a.dv ? a.dv + S.v_off + g * S.v_sg + h * S.v_sh + (int64_t)key * S.v_si : nullptr;
    const float ks = kvalid ? a.scale : 0.0f, vs = kvalid ? 1.0f : 0.0f;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        const int d = t * 32 + kappa(g2, i);
        if (d < D) {
          if (krow) store4<T>(krow, d, dk[t][i] * ks, dk[t][i + 1] * ks, dk[t][i + 2] * ks, dk[t][i + 3] * ks);
          if (vrow) store4<T>(vrow, d, dv[t][i] * vs, dv[t][i + 1] * vs, dv[t][i + 2] * vs, dv[t][i + 3] * vs);
        }
      }
    }
  }
}

#define OOPS_BWD_FAST_INST(T, DP)                                                \
  template __global__ void attn_dkv_fast_kernel<T, DP, true>(BwdArgsT<T, T>);  \
  template __global__ void attn_dkv_fast_kernel<T, DP, false>(BwdArgsT<T, T>);
OOPS_BWD_FAST_INST(__bf16, 32)
OOPS_BWD_FAST_INST(__bf16, 64)
OOPS_BWD_FAST_INST(_Float16, 32)
OOPS_BWD_FAST_INST(_Float16, 64)

bool backward_fast_ok(const oops_attn_geometry& geo, const Plan& plan) {
  if (geo.force_generic) return false;
  if (geo.dtype == OOPS_F32 || plan.dp > 64 || plan.any_pair_mask || !geo.vec_ok || geo.head_size % 8 != 0 ||
      !plan.offsets_32bit)
    return false;
  return !(geo.has_bias && geo.bias_dtype != geo.dtype);
}

hipError_t launch_dkv_fast(const oops_attn_geometry& geo, const Plan& plan, const BwdLaunch& L, hipStream_t stream) {
  hipError_t err = hipSuccess;
  auto go = [&](auto tag, auto dpc) {
    using T = typename decltype(tag)::type;
    constexpr int DP = decltype(dpc)::value;
    BwdArgsT<T, T> a;
    fill_bwd_args(a, geo, plan, L);
    a.uniform_tiles = plan.dkv_uniform;
    a.total_tiles = plan.dkv_tiles;
    const dim3 grid((unsigned)xcd_grid(plan.dkv_tiles));
    if (a.bias != nullptr)
      hipLaunchKernelGGL((attn_dkv_fast_kernel<T, DP, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((attn_dkv_fast_kernel<T, DP, false>), grid, dim3(256), 0, stream, a);
    err = hipGetLastError();
  };
  if (geo.dtype == OOPS_BF16) {
    if (plan.dp == 32) go(Tag<__bf16>{}, std::integral_constant<int, 32>{});
    else go(Tag<__bf16>{}, std::integral_constant<int, 64>{});
  } else {
    if (plan.dp == 32) go(Tag<_Float16>{}, std::integral_constant<int, 32>{});
    else go(Tag<_Float16>{}, std::integral_constant<int, 64>{});
  }
  return err;
}

}  // namespace oops
