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

template <typename T, int DP, bool HAS_BIAS, int R>
__global__ __launch_bounds__(256, OOPS_DKV_OCC) void attn_dkv_fast_kernel(BwdArgsT<T, T> a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int TBUF = 64 * DP;     // elements per tile buffer (64 swizzled rows, see swz)
  constexpr int NDT = DP / 32;
  constexpr int NQF = DP / 16;
  constexpr int NCH = DP / 32;      // 16-byte chunks of Q (and dO) per thread per step

  __shared__ __attribute__((aligned(16))) T q_lds[3 * R * TBUF];
  __shared__ __attribute__((aligned(16))) T do_lds[3 * R * TBUF];
  __shared__ __attribute__((aligned(16))) float nlse_lds[3 * R * 64];  // -LSE / c1, rows permuted
  __shared__ __attribute__((aligned(16))) float ndlt_lds[3 * R * 64];  // -delta, rows permuted

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int g2 = lane >> 5;

  // XCD-aware order (see attn_fwd_fast.hip): logical (head group, row block,
  // head, key block); a row block is R consecutive groups g that share the
  // bias, so each bias fragment loaded serves R rows
  int64_t tile = xcd_tile(blockIdx.x, gridDim.x, xcd_chunk(a.uniform_tiles));
  if (tile >= a.total_tiles) return;
  const Sample* tab = reinterpret_cast<const Sample*>(a.table);
  const int H = a.num_heads;
  // (a split batch: the samples the fused dK/dV + dBias kernel does not serve)
  const int s_idx = find_sample(tile, tab, a.num_samples, a.uniform_tiles, [&](const Sample& s) {
    return a.fused_max_lq > 0 && s.Lq <= a.fused_max_lq ? (int64_t)0 : cdiv(s.G, R) * H * cdiv(s.Lk, 128);
  });
  if (s_idx < 0) return;
  const Sample& S = tab[__builtin_amdgcn_readfirstlane(s_idx)];
  const int64_t G = S.G;
  const int64_t GB = cdiv(G, R);
  const int Lq = (int)S.Lq, Lk = (int)S.Lk;
  const int nkb = (int)cdiv(Lk, 128);
  const int HG = a.head_group;
  const int kb = __builtin_amdgcn_readfirstlane((int)((uint32_t)tile % (uint32_t)nkb));
  uint32_t rest = (uint32_t)tile / (uint32_t)nkb;
  const int hh = __builtin_amdgcn_readfirstlane((int)(rest % (uint32_t)HG));
  rest /= (uint32_t)HG;
  const int g0 = __builtin_amdgcn_readfirstlane((int)(rest % (uint32_t)GB) * R);
  const int h = __builtin_amdgcn_readfirstlane((int)(rest / (uint32_t)GB) * HG + hh);
  const int D = a.head_size;
  const int q_si = (int)S.q_si, do_si = (int)S.do_si, b_si = (int)S.b_si;
  const int nsteps = (Lq + 63) >> 6;
  bool row_ok[R];
#pragma unroll
  for (int r = 0; r < R; ++r) row_ok[r] = g0 + r < G;

  // ---- this lane's key: K, V fragments of each row (B operands: lane = key, k = head dim)
  const int key = kb * 128 + wave * 32 + lq;
  const bool has_mask = a.mask != nullptr && S.m_off >= 0;
  bool kvalid[R], wave_masked[R];
  Frag kf[R][NQF], vf[R][NQF];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int g = g0 + r;
    bool kv = row_ok[r] && key < Lk;
    if (kv && has_mask) kv = a.mask[S.m_off + g * S.m_sg + key] != 0;
    kvalid[r] = kv;
    wave_masked[r] = __any(!kv);
    const T* kbase = a.k + S.k_off + (row_ok[r] ? g : g0) * S.k_sg + h * S.k_sh;
    const T* vbase = a.v + S.v_off + (row_ok[r] ? g : g0) * S.v_sg + h * S.v_sh;
    const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc(kbase, (uint32_t)(((int64_t)(Lk - 1) * S.k_si + D) * 2));
    const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc(vbase, (uint32_t)(((int64_t)(Lk - 1) * S.v_si + D) * 2));
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      const int col = s * 16 + g2 * 8;
      const bool ok = kv && col < D;
      kf[r][s] = __builtin_bit_cast(Frag, buffer_load16(k_rsrc, ok ? (uint32_t)((key * (int)S.k_si + col) * 2) : kOut));
      vf[r][s] = __builtin_bit_cast(Frag, buffer_load16(v_rsrc, ok ? (uint32_t)((key * (int)S.v_si + col) * 2) : kOut));
    }
  }
  Frag ident[2];
  identity_frags<T>(ident, 1.0f / a.scale, lane);

  // ---- per-thread staging offsets (bytes); the step adds q0 * stride via soffset
  __amdgpu_buffer_rsrc_t q_rsrc[R], do_rsrc[R], l_rsrc[R], d_rsrc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    // a row past G (odd G) reads nothing: empty ranges
    const int g = row_ok[r] ? g0 + r : g0;
    const uint32_t live = row_ok[r] ? 1u : 0u;
    q_rsrc[r] = make_rsrc(a.q + S.q_off + g * S.q_sg + h * S.q_sh, live * (uint32_t)(((int64_t)(Lq - 1) * q_si + D) * 2));
    do_rsrc[r] =
        make_rsrc(a.dout + S.do_off + g * S.do_sg + h * S.do_sh, live * (uint32_t)(((int64_t)(Lq - 1) * do_si + D) * 2));
    // LSE / delta rows: rows past Lq read 0; they contribute nothing because
    // their dO (and Q) rows read as zero, so dS = P * (0 - 0) = 0
    l_rsrc[r] = make_rsrc(a.lse + S.l_off + ((int64_t)g * H + h) * Lq, live * (uint32_t)(Lq * 4));
    d_rsrc[r] = make_rsrc(a.delta + S.l_off + ((int64_t)g * H + h) * Lq, live * (uint32_t)(Lq * 4));
  }
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
  // bias rows of this wave's keys: A fragments (lane = query, 8 consecutive
  // keys), from the fragment-major copy of a shared bias (one contiguous
  // 1 KB load per fragment) or from the bias rows themselves; with R > 1 the
  // bias is shared by the rows (the host picks R > 1 only then)
  const int kw = kb * 128 + wave * 32;  // first key of this wave
  const bool use_bf = HAS_BIAS && a.bias_frag != nullptr && S.bias_mode == OOPS_BIAS_SHARED;
  __amdgpu_buffer_rsrc_t b_rsrc;
  if (use_bf) {
    const int kt = kw >> 5;
    const bool in = kt < a.bf_nkt;  // a wave wholly past Lk: empty range
    b_rsrc = make_rsrc(a.bias_frag + s_idx * a.bf_sample_stride + (int64_t)h * a.bf_nqt * a.bf_nkt * 1024 +
                           (in ? kt : 0) * 1024,
                       in ? (uint32_t)(((int64_t)a.bf_nqt * a.bf_nkt - (in ? kt : 0)) * 2048) : 0u);
  } else {
    const T* bbase = HAS_BIAS ? a.bias + S.b_off + g0 * S.b_sg + h * S.b_sh : a.q;
    b_rsrc = make_rsrc(bbase, HAS_BIAS ? (uint32_t)(((int64_t)(Lq - 1) * b_si + Lk) * 2) : 0u);
  }

  struct Stage {
    uint4 q[R][NCH], d[R][NCH];
    float lse[R], dlt[R];
  };
  auto load_stage = [&](int step, Stage& st) {
    const int q0 = step * 64;
    const uint32_t qs = (uint32_t)(q0 * q_si * 2), ds = (uint32_t)(q0 * do_si * 2);
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const bool ok = q0 + (int)st_row[i] < Lq;
        st.q[r][i] = buffer_load16_s(q_rsrc[r], ok ? q_off[i] : kOut, qs);
        st.d[r][i] = buffer_load16_s(do_rsrc[r], ok ? do_off[i] : kOut, ds);
      }
      if (tid < 64) {
        const uint32_t off = (uint32_t)((q0 + tid) * 4);  // range-checked: rows past Lq read 0
        st.lse[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(l_rsrc[r], off, 0, 0));
        st.dlt[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(d_rsrc[r], off, 0, 0));
      }
    }
  };
  // -LSE is the S accumulator's input, in units of the unscaled scores
  const float inv_c1 = 1.0f / (a.scale * kLog2e);
  auto store_stage = [&](int buf, const Stage& st) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int c = tid + 256 * i;
        const int row = c / (DP / 8);
        const int col = (c % (DP / 8)) * 8;
        *reinterpret_cast<uint4*>(&q_lds[(buf * R + r) * TBUF + swz_off<DP>(row, col)]) = st.q[r][i];
        *reinterpret_cast<uint4*>(&do_lds[(buf * R + r) * TBUF + swz_off<DP>(row, col)]) = st.d[r][i];
      }
      if (tid < 64) {
        const int pos = (tid & 32) + perm32(tid & 31);
        nlse_lds[(buf * R + r) * 64 + pos] = -st.lse[r] * inv_c1;
        ndlt_lds[(buf * R + r) * 64 + pos] = -st.dlt[r];
      }
    }
  };

  const float c1 = a.scale * kLog2e;
  f32x16 dk[R][NDT], dv[R][NDT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < NDT; ++t) dk[r][t] = dv[r][t] = f32x16{};

  TrLane trl[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) trl[t] = tr_lane<DP>(lane, 32 * t);
  // one step: for each row, two 32-query tiles of LDS buffer buf against this wave's keys
  auto compute = [&](int buf, const uint4 (&bias)[2][2]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (!row_ok[r]) continue;
      const T* qt = &q_lds[(buf * R + r) * TBUF];
      const T* dt = &do_lds[(buf * R + r) * TBUF];
#pragma unroll
      for (int qr = 0; qr < 2; ++qr) {
        // S - LSE / c1: the accumulator starts from -LSE / c1
        f32x16 sacc = *reinterpret_cast<const f32x16*>(&nlse_lds[(buf * R + r) * 64 + 32 * qr + g2 * 16]);
        if constexpr (HAS_BIAS) {
          sacc = E::mma(__builtin_bit_cast(Frag, bias[qr][0]), ident[0], sacc);
          sacc = E::mma(__builtin_bit_cast(Frag, bias[qr][1]), ident[1], sacc);
        }
        f32x16 pacc = *reinterpret_cast<const f32x16*>(&ndlt_lds[(buf * R + r) * 64 + 32 * qr + g2 * 16]);
#pragma unroll
        for (int s = 0; s < NQF; ++s) {
          sacc = E::mma(lds_frag<T>(qt + swz_off<DP>(32 * qr + lq, s * 16 + g2 * 8)), kf[r][s], sacc);
          pacc = E::mma(lds_frag<T>(dt + swz_off<DP>(32 * qr + lq, s * 16 + g2 * 8)), vf[r][s], pacc);
        }
        float p[16], ds[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          p[j] = __builtin_amdgcn_exp2f(sacc[j] * c1);
          if (wave_masked[r]) p[j] = kvalid[r] ? p[j] : 0.0f;
          ds[j] = p[j] * pacc[j];
        }
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const Frag pf = pack8<T>(&p[8 * m]);
          const Frag sf = pack8<T>(&ds[8 * m]);
#pragma unroll
          for (int t = 0; t < NDT; ++t) {
            const int at = (32 * qr + 16 * m) * DP + 32 * t;
            dv[r][t] = E::mma(lds_read_tr_frag_sw<T>(dt + at, trl[t]), pf, dv[r][t]);
            dk[r][t] = E::mma(lds_read_tr_frag_sw<T>(qt + at, trl[t]), sf, dk[r][t]);
          }
        }
      }
    }
  };
  auto load_bias = [&](int step, uint4 (&bias)[2][2]) {
#pragma unroll
    for (int qr = 0; qr < 2; ++qr) {
      const int q = step * 64 + 32 * qr + lq;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        // fragment copy: tile row qt = 2 step + qr, entry (c, lane); rows past the copy read 0
        const uint32_t off = use_bf ? (uint32_t)((((2 * step + qr) * a.bf_nkt * 2 + c) * 64 + lane) * 16)
                                    : (q < Lq ? (uint32_t)((q * b_si + kw + 16 * c + g2 * 8) * 2) : kOut);
        bias[qr][c] = buffer_load16_s(b_rsrc, off, 0);
        if (!use_bf) bias[qr][c] = finite16<T>(bias[qr][c]);  // (the copy holds finite values already)
      }
    }
  };

  // ---- pipeline: step i computes buffer i % 3; the stage of step i+2
  // (loaded during step i-1) is written at the top of step i.
  Stage stg;
  uint4 bias_r[2][2];
  if (nsteps > 0) {
    load_stage(0, stg);
    if constexpr (HAS_BIAS) load_bias(0, bias_r);
    store_stage(0, stg);
  }
  if (nsteps > 1) {
    load_stage(1, stg);
    store_stage(1, stg);
  }
  load_stage(2, stg);
  vmem_wait_all();
  __syncthreads();
  int buf = 0;
  for (int i = 0; i < nsteps; ++i) {
    const int b1 = buf == 2 ? 0 : buf + 1;
    const int b2 = b1 == 2 ? 0 : b1 + 1;
    if (i + 2 < nsteps) store_stage(b2, stg);
    load_stage(i + 3, stg);
    compute(buf, bias_r);
    if constexpr (HAS_BIAS)
      load_bias(i + 1, bias_r);  // one register set: the next step's bias
    lds_barrier();
    buf = b1;
  }

  // ---- write dK = scale * dK^T^T, dV (zero for masked keys)
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (!row_ok[r] || key >= Lk) continue;
    const int g = g0 + r;
    T* krow = a.dk ? a.dk + S.k_off + g * S.k_sg + h * S.k_sh + (int64_t)key * S.k_si : nullptr;
    T* vrow = a.dv ? a.dv + S.v_off + g * S.v_sg + h * S.v_sh + (int64_t)key * S.v_si : nullptr;
    const float ks = kvalid[r] ? a.scale : 0.0f, vs = kvalid[r] ? 1.0f : 0.0f;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      if (krow) store_tile<T>(krow, t * 32, D, g2, dk[r][t], ks);
      if (vrow) store_tile<T>(vrow, t * 32, D, g2, dv[r][t], vs);
    }
  }
}

// attn_dq_fast_kernel: one workgroup = 4 wavefronts x 32 queries of one
// (sample, group, head), the query as MFMA column (as in the forward).  Per
// 64-key step: S^T = bias (identity MFMA) + K Q^T, dP^T = V dO^T - delta
// (-delta is a constant accumulator input), P = exp2(S * scale * log2 e -
// LSE), dS = P dP, dQ^T += K^T dS^T (K^T by LDS transpose reads).  A
// per-group ("full") bias gets dBias = dS written from registers.
// Reference: _backward_query (oops/attention/triangle/triton/kernel.py:428-565).
// MASKED_TILES: the geometry may have 64-key tiles with masked or
// out-of-range keys (else only the unmasked tile code is compiled);
// FULL_DBIAS: some sample has a per-group bias whose dBias = dS is written
// here.  Both only add code that costs registers when compiled in.  FOLD
// (bf16, bias, at most kFoldTiles key tiles): the key masks are folded into
// the bias fragments (fold_bias) instead of selected per score.
// The lean instances (D <= 32, no per-score mask code, no full dBias) start
// dP from a register tile of -delta instead of zero (one VALU add less per
// score) and are built for four waves per SIMD, which the extra 16 registers
// still fit.
template <int DP, bool MASKED_TILES, bool FULL_DBIAS, bool FOLD>
constexpr bool kLeanDq = DP == 32 && (!MASKED_TILES || FOLD) && !FULL_DBIAS;
template <typename T, int DP, bool HAS_BIAS, bool MASKED_TILES, bool FULL_DBIAS, bool FOLD>
__global__ __launch_bounds__(256, (kLeanDq<DP, MASKED_TILES, FULL_DBIAS, FOLD> ? 4 : OOPS_DQ_OCC)) void attn_dq_fast_kernel(
    BwdArgsT<T, T> a) {
  constexpr bool LEAN = kLeanDq<DP, MASKED_TILES, FULL_DBIAS, FOLD>;
  static_assert(!FOLD || (MASKED_TILES && HAS_BIAS && sizeof(T) == 2), "fold: masked bf16 tiles with a bias");
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int LD = DP + 8;
  constexpr int TBUF = 64 * LD;
  constexpr int NDT = DP / 32;
  constexpr int NQF = DP / 16;
  constexpr int NCH = DP / 32;

  __shared__ __attribute__((aligned(16))) T k_lds[3 * TBUF];
  __shared__ __attribute__((aligned(16))) T v_lds[3 * TBUF];
  __shared__ uint64_t keep_lds[kMaxKeyTiles];
  __shared__ float dl_lds[4 * 32];
  __shared__ __attribute__((aligned(16))) uint32_t fold_lds[FOLD ? kFoldTiles * 32 : 4];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int g2 = lane >> 5;

  int64_t tile = xcd_tile(blockIdx.x, gridDim.x, xcd_chunk(a.uniform_tiles));
  if (tile >= a.total_tiles) return;
  const Sample* tab = reinterpret_cast<const Sample*>(a.table);
  const int H = a.num_heads;
  const int s_idx = find_sample(tile, tab, a.num_samples, a.uniform_tiles,
                                [&](const Sample& s) { return s.G * H * cdiv(s.Lq, 128); });
  if (s_idx < 0) return;
  const Sample& S = tab[__builtin_amdgcn_readfirstlane(s_idx)];
  const int64_t G = S.G;
  const int Lq = (int)S.Lq, Lk = (int)S.Lk;
  const int nqb = (int)cdiv(Lq, 128);
  const int HG = a.head_group;
  // (launch grids stay below 2^31 workgroups: 32-bit division)
  const int qb = __builtin_amdgcn_readfirstlane((int)((uint32_t)tile % (uint32_t)nqb));
  uint32_t rest = (uint32_t)tile / (uint32_t)nqb;
  const int hh = __builtin_amdgcn_readfirstlane((int)(rest % (uint32_t)HG));
  rest /= (uint32_t)HG;
  const int g = __builtin_amdgcn_readfirstlane((int)(rest % (uint32_t)G));
  const int h = __builtin_amdgcn_readfirstlane((int)(rest / (uint32_t)G) * HG + hh);
  const int D = a.head_size;
  const int ntiles = (Lk + 63) >> 6;
  const int k_si = (int)S.k_si, v_si = (int)S.v_si, b_si = (int)S.b_si;
  const bool has_mask = a.mask != nullptr && S.m_off >= 0;
  const uint8_t* mbase = has_mask ? a.mask + S.m_off + g * S.m_sg : nullptr;
  const bool write_dbias = FULL_DBIAS && a.dbias != nullptr && S.bias_mode == OOPS_BIAS_FULL;

  // keep bitmaps; without mixed tiles (no mask, Lk a multiple of 64) every tile is whole
  if constexpr (MASKED_TILES) for (int t = wave; t < ntiles; t += 4) {
    const int key = t * 64 + lane;
    bool keep = key < Lk;
    if (keep && has_mask) keep = mbase[key] != 0;
    const uint64_t bits = __ballot(keep);
    if (lane == 0) keep_lds[t] = bits;
  }

  const int q_lane = qb * 128 + wave * 32 + lq;
  const bool qv = q_lane < Lq;
  const int64_t lidx = S.l_off + ((int64_t)g * H + h) * Lq + q_lane;
  const float neg_lse = qv ? -a.lse[lidx] : 0.0f;
  Frag qf[NQF], df[NQF];
  float ndelta;  // -delta of this lane's query (subtracted from dP in the VALU)
  {
    // The wave's 32 query rows of Q and dO are read whole (DP/8 lanes per
    // row, 16-byte chunks), staged through a wave-private region of the K/V
    // ring (free until the ring's first store, after the barrier below) and
    // read back as MFMA fragments.
    constexpr int NQR = DP / 16;
    constexpr int LPR = DP / 8;
    const int q0w = qb * 128 + wave * 32;
    const int64_t gh_q = S.q_off + g * S.q_sg + h * S.q_sh;
    const int64_t gh_d = S.do_off + g * S.do_sg + h * S.do_sh;
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q + gh_q, (uint32_t)(((int64_t)(Lq - 1) * S.q_si + D) * 2));
    const __amdgpu_buffer_rsrc_t dr = make_rsrc(a.dout + gh_d, (uint32_t)(((int64_t)(Lq - 1) * S.do_si + D) * 2));
    int q_row[NQR], q_col[NQR];
    bool ok[NQR];
    uint4 qu[NQR], du[NQR];
#pragma unroll
    for (int i = 0; i < NQR; ++i) {
      const int c = i * 64 + lane;
      q_row[i] = c / LPR;
      q_col[i] = (c % LPR) * 8;
      ok[i] = q0w + q_row[i] < Lq && q_col[i] < D;
      qu[i] = buffer_load16(qr, ok[i] ? (uint32_t)(((q0w + q_row[i]) * (int)S.q_si + q_col[i]) * 2) : kOut);
      du[i] = buffer_load16(dr, ok[i] ? (uint32_t)(((q0w + q_row[i]) * (int)S.do_si + q_col[i]) * 2) : kOut);
    }
    if constexpr (DP == kCompactRow) {
      // compact copies of these Q and dO rows for the fused dK/dV + dBias kernel
      if (a.qc != nullptr && (a.fused_max_lq == 0 || Lq <= a.fused_max_lq)) {
        const int64_t row0 = S.l_off + ((int64_t)g * H + h) * Lq + q0w;
#pragma unroll
        for (int i = 0; i < NQR; ++i)
          if (ok[i]) {
            const int64_t e = (row0 + q_row[i]) * kCompactRow + q_col[i];
            *reinterpret_cast<uint4*>(a.qc + e) = qu[i];
            *reinterpret_cast<uint4*>(a.dc + e) = du[i];
          }
      }
    }
    float dl;
    if (a.delta_in_dq) {
      // delta = rowsum((O + O_lo) * dO): partial sums over this lane's
      // chunks, reduced over the row's lanes, gathered through LDS
      const int64_t gh_o = S.o_off + g * S.o_sg + h * S.o_sh;
      const uint32_t o_bytes = (uint32_t)(((int64_t)(Lq - 1) * S.o_si + D) * 2);
      const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.out + gh_o, o_bytes);
      const __amdgpu_buffer_rsrc_t lrr = make_rsrc(a.out_lo != nullptr ? a.out_lo + gh_o : a.out,
                                                   a.out_lo != nullptr ? o_bytes : 0u);
      float part[NQR];
#pragma unroll
      for (int i = 0; i < NQR; ++i) {
        const uint32_t off = ok[i] ? (uint32_t)(((q0w + q_row[i]) * (int)S.o_si + q_col[i]) * 2) : kOut;
        const uint4 ou = buffer_load16(orr, off);
        const uint4 lu = buffer_load16(lrr, off);
        const T* oe = reinterpret_cast<const T*>(&ou);
        const T* le = reinterpret_cast<const T*>(&lu);
        const T* de = reinterpret_cast<const T*>(&du[i]);
        // O dO + O_lo dO, two products per v_dot2 on the packed 16-bit pairs
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          typename Pair<T>::v2 op, lp, dp;
          op[0] = oe[e], op[1] = oe[e + 1];
          lp[0] = le[e], lp[1] = le[e + 1];
          dp[0] = de[e], dp[1] = de[e + 1];
          s = Pair<T>::dot(lp, dp, Pair<T>::dot(op, dp, s));
        }
#pragma unroll
        for (int m = 1; m < LPR; m <<= 1) s += __shfl_xor(s, m);
        part[i] = s;
      }
#pragma unroll
      for (int i = 0; i < NQR; ++i)
        if (lane % LPR == 0) {
          dl_lds[wave * 32 + q_row[i]] = part[i];
          if (q0w + q_row[i] < Lq) a.delta[lidx - lq + q_row[i]] = part[i];
        }
    }
    T* const q_w = &k_lds[wave * 32 * LD];
    T* const d_w = &v_lds[wave * 32 * LD];
#pragma unroll
    for (int i = 0; i < NQR; ++i) {
      *reinterpret_cast<uint4*>(&q_w[q_row[i] * LD + q_col[i]]) = qu[i];
      *reinterpret_cast<uint4*>(&d_w[q_row[i] * LD + q_col[i]]) = du[i];
    }
    // other lanes of this wave read what was just written (LDS operations
    // of one wave complete in order; the fences keep the compiler's order)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      qf[s] = lds_frag<T>(&q_w[lq * LD + s * 16 + g2 * 8]);
      df[s] = lds_frag<T>(&d_w[lq * LD + s * 16 + g2 * 8]);
    }
    if (a.delta_in_dq) {
      dl = dl_lds[wave * 32 + lq];
      dl = qv ? dl : 0.0f;
    } else {
      dl = qv ? a.delta[lidx] : 0.0f;
    }
    ndelta = -dl;
  }
  // the pack of the fused dK/dV + dBias kernel: per (g, h) row, -LSE / c of
  // the Lq queries (lanes 0..31), then -delta (lanes 32..63)
  if (a.ld_pack != nullptr && qv) {
    float* const pk_row = a.ld_pack + 2 * (lidx - q_lane);
    pk_row[g2 * Lq + q_lane] = g2 ? ndelta : neg_lse * (1.0f / (a.scale * kLog2e));
  }
  Frag ident[2];
  identity_frags<T>(ident, 1.0f / a.scale, lane);

  const T* kbase = a.k + S.k_off + g * S.k_sg + h * S.k_sh;
  const T* vbase = a.v + S.v_off + g * S.v_sg + h * S.v_sh;
  const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc(kbase, (uint32_t)(((int64_t)(Lk - 1) * k_si + D) * 2));
  const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc(vbase, (uint32_t)(((int64_t)(Lk - 1) * v_si + D) * 2));
  // empty ranges: the loads of an absent tile (t >= ntiles) read zeros and make no memory request
  const __amdgpu_buffer_rsrc_t k_none = make_rsrc(kbase, 0u), v_none = make_rsrc(vbase, 0u);
  uint32_t kv_row[NCH], k_off[NCH], v_off[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = tid + 256 * i;
    const int r = c / (DP / 8);
    const int col = (c % (DP / 8)) * 8;
    kv_row[i] = r;
    k_off[i] = col < D ? (uint32_t)((r * k_si + col) * 2) : kOut;
    v_off[i] = col < D ? (uint32_t)((r * v_si + col) * 2) : kOut;
  }
  // bias fragments: from the fragment-major copy of a shared bias (one
  // contiguous 1 KB load per fragment), else from the bias rows themselves
  const bool use_bf = HAS_BIAS && a.bias_frag != nullptr && S.bias_mode == OOPS_BIAS_SHARED;
  __amdgpu_buffer_rsrc_t b_rsrc, b_none;
  uint32_t b_off[2][2], b_step;
  if (use_bf) {
    const int qt = qb * 4 + wave;
    const bool in = qt < a.bf_nqt;  // a wave wholly past Lq: empty range
    b_rsrc = make_rsrc(a.bias_frag + s_idx * a.bf_sample_stride +
                           (((int64_t)h * a.bf_nqt + (in ? qt : 0)) * a.bf_nkt) * 1024,
                       in ? (uint32_t)(a.bf_nkt * 2048) : 0u);
    b_none = make_rsrc(a.bias_frag, 0u);
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int c = 0; c < 2; ++c) b_off[t2][c] = (uint32_t)(((t2 * 2 + c) * 64 + lane) * 16);
    b_step = 4096;
  } else {
    const T* bbase = HAS_BIAS ? a.bias + S.b_off + g * S.b_sg + h * S.b_sh : a.q;
    b_rsrc = make_rsrc(bbase, HAS_BIAS ? (uint32_t)(((int64_t)(Lq - 1) * b_si + Lk) * 2) : 0u);
    b_none = make_rsrc(bbase, 0u);
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int c = 0; c < 2; ++c)
        b_off[t2][c] = qv ? (uint32_t)((q_lane * b_si + 32 * t2 + 16 * c + g2 * 8) * 2) : kOut;
    b_step = 128;
  }
  float* dbrow = write_dbias && qv ? a.dbias + S.db_off + g * S.db_sg + h * S.db_sh + (int64_t)q_lane * S.db_si
                                   : nullptr;

  // An absent tile (t >= ntiles) issues its loads with out-of-range offsets:
  // no memory traffic, and no branch, so the compiler can count outstanding
  // loads exactly and never has to wait for all of them.
  auto load_kv = [&](int t, uint4 (&ku)[NCH], uint4 (&vu)[NCH]) {
    const uint32_t ks = (uint32_t)(t * 64 * k_si * 2), vs = (uint32_t)(t * 64 * v_si * 2);
    if constexpr (!MASKED_TILES) {
      // whole tiles: fixed per-lane offsets, an absent tile takes the empty ranges
      const bool live = t < ntiles;
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        ku[i] = buffer_load16_s(live ? k_rsrc : k_none, k_off[i], ks);
        vu[i] = buffer_load16_s(live ? v_rsrc : v_none, v_off[i], vs);
      }
      return;
    }
    const uint64_t bits = t < ntiles ? keep_lds[t < ntiles ? t : 0] : 0;
    const bool full = bits == ~uint64_t(0);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const bool ok = full || ((bits >> kv_row[i]) & 1);
      ku[i] = buffer_load16_s(k_rsrc, ok ? k_off[i] : kOut, ks);
      vu[i] = buffer_load16_s(v_rsrc, ok ? v_off[i] : kOut, vs);
    }
  };
  auto store_kv = [&](int buf, const uint4 (&ku)[NCH], const uint4 (&vu)[NCH]) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + 256 * i;
      const int r = c / (DP / 8);
      const int col = (c % (DP / 8)) * 8;
      *reinterpret_cast<uint4*>(&k_lds[buf * TBUF + r * LD + col]) = ku[i];
      *reinterpret_cast<uint4*>(&v_lds[buf * TBUF + r * LD + col]) = vu[i];
    }
  };
  auto load_bias = [&](int t, uint4 (&bf)[2][2]) {
    const uint32_t s = (uint32_t)t * b_step;
    if (!MASKED_TILES && use_bf) {
      // whole tiles of the fragment-major copy: the tile offset is a scalar
      // offset (every tile lies inside the range), an absent tile reads the empty range
      const __amdgpu_buffer_rsrc_t r = t < ntiles ? b_rsrc : b_none;
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int c = 0; c < 2; ++c) bf[t2][c] = buffer_load16_s(r, b_off[t2][c], s);
      return;
    }
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int c = 0; c < 2; ++c) bf[t2][c] = buffer_load16_s(b_rsrc, t < ntiles ? b_off[t2][c] + s : kOut, 0);
    // bias rows read directly (not the fragment-major copy, which holds finite values already)
    if (!use_bf) {
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int c = 0; c < 2; ++c) bf[t2][c] = finite16<T>(bf[t2][c]);
    }
  };

  __syncthreads();
  // (the fold table is read after the barrier that ends the prologue)
  if constexpr (FOLD) build_fold_table(fold_lds, keep_lds, ntiles, tid, 256);
  auto next_tile = [&](int t) {
    if constexpr (!MASKED_TILES) return t + 1 < ntiles ? t + 1 : ntiles;
    if (t >= ntiles) return ntiles;
    ++t;
    while (t < ntiles && keep_lds[t] == 0) ++t;
    return t;
  };

  const float c1 = a.scale * kLog2e;
  f32x16 nd_tile;  // LEAN: the dP accumulator's starting value
#pragma unroll
  for (int j = 0; j < 16; ++j) nd_tile[j] = LEAN ? ndelta : 0.0f;
  f32x16 acc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) acc[t] = f32x16{};

  // MASKED: a tile with masked or out-of-range keys (P selected per score);
  // fully kept tiles run the variant without any per-score mask work
  auto compute = [&](auto masked, int buf, int t, uint64_t bits, const uint4 (&bf)[2][2]) {
    constexpr bool MASKED = decltype(masked)::value;
    const T* kt = &k_lds[buf * TBUF];
    const T* vt = &v_lds[buf * TBUF];
    const uint64_t lb = bits >> (g2 * 4);
    const uint4* fm = reinterpret_cast<const uint4*>(&fold_lds[FOLD ? (t * 2 + g2) * 16 : 0]);
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      f32x16 sacc;
      if constexpr (HAS_BIAS) {
        const uint4 b0 = FOLD ? fold_bias(bf[t2][0], fm[t2 * 2]) : bf[t2][0];
        const uint4 b1 = FOLD ? fold_bias(bf[t2][1], fm[t2 * 2 + 1]) : bf[t2][1];
        sacc = E::mma(ident[0], __builtin_bit_cast(Frag, b0), f32x16{});
        sacc = E::mma(ident[1], __builtin_bit_cast(Frag, b1), sacc);
      } else {
        sacc = f32x16{};
      }
      f32x16 pacc = LEAN ? nd_tile : f32x16{};
#pragma unroll
      for (int s = 0; s < NQF; ++s) {
        sacc = E::mma(lds_frag<T>(kt + (32 * t2 + lq) * LD + s * 16 + g2 * 8), qf[s], sacc);
        pacc = E::mma(lds_frag<T>(vt + (32 * t2 + lq) * LD + s * 16 + g2 * 8), df[s], pacc);
      }
      float ds[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j], c1, neg_lse));
        if constexpr (MASKED) {
          const int kk = 32 * t2 + ((j >> 2) << 3) + (j & 3);
          p = ((lb >> kk) & 1) ? p : 0.0f;
        }
        ds[j] = LEAN ? p * pacc[j] : p * (pacc[j] + ndelta);
      }
      if (FULL_DBIAS && dbrow) {
        const int k0 = t * 64 + 32 * t2;
#pragma unroll
        for (int j = 0; j < 16; j += 4) {
          const int key = k0 + kappa(g2, j);
          if (key + 3 < Lk) {
            *reinterpret_cast<float4*>(dbrow + key) = make_float4(ds[j], ds[j + 1], ds[j + 2], ds[j + 3]);
          } else {
            for (int e = 0; e < 4; ++e)
              if (key + e < Lk) dbrow[key + e] = ds[j + e];
          }
        }
      }
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const Frag sf = pack8<T>(&ds[8 * m]);
#pragma unroll
        for (int d = 0; d < NDT; ++d)
          acc[d] = E::mma(lds_read_tr_frag<T>(kt, LD, 32 * t2 + 16 * m, 32 * d, lane), sf, acc[d]);
      }
    }
  };

  uint4 ku[NCH], vu[NCH];
  uint4 bias_a[2][2];
  int t0 = next_tile(-1);
  int t1 = next_tile(t0);
  int t2 = next_tile(t1);
  if (t0 < ntiles) {
    load_kv(t0, ku, vu);
    if constexpr (HAS_BIAS) load_bias(t0, bias_a);
    store_kv(0, ku, vu);
  }
  if (t1 < ntiles) {
    load_kv(t1, ku, vu);
    store_kv(1, ku, vu);
  }
  load_kv(t2, ku, vu);
  vmem_wait_all();
  __syncthreads();
  int buf = 0;
  while (t0 < ntiles) {
    const int t3 = next_tile(t2);
    const uint64_t bits = MASKED_TILES ? uniform64(keep_lds[t0]) : ~uint64_t(0);
    const int b1 = buf == 2 ? 0 : buf + 1;
    const int b2 = b1 == 2 ? 0 : b1 + 1;
    if (t2 < ntiles) store_kv(b2, ku, vu);
    load_kv(t3, ku, vu);
    if (!MASKED_TILES || FOLD || bits == ~uint64_t(0))
      compute(std::false_type{}, buf, t0, bits, bias_a);
    else if constexpr (MASKED_TILES && !FOLD)
      compute(std::true_type{}, buf, t0, bits, bias_a);
    if constexpr (HAS_BIAS)
      load_bias(t1, bias_a);  // one register set: the next tile's bias
    lds_barrier();
    buf = b1;
    t0 = t1;
    t1 = t2;
    t2 = t3;
  }

  // the lane's query, recomputed from the lane id here (an opaque read, so
  // that the compiler does not keep the epilogue's per-lane addresses live
  // through the loop, where the lean instances have no registers to spare)
  uint32_t ln;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
  const int q_end = qb * 128 + wave * 32 + (int)(ln & 31);
  if (q_end < Lq && a.dq != nullptr) {
    T* row = a.dq + S.q_off + g * S.q_sg + h * S.q_sh + (int64_t)q_end * S.q_si;
#pragma unroll
    for (int t = 0; t < NDT; ++t) store_tile<T>(row, t * 32, D, (int)(ln >> 5), acc[t], a.scale);
  }
}

// attn_dbias_fast_kernel: dBias[h, q, k] = sum over groups g of dS for a
// bias shared by all groups.  One workgroup = 4 waves x 32 queries and 64
// keys of one head, walking the groups g of one part.  The bias block's MFMA
// contribution is computed once and is the accumulator input of every
// group's S^T; K/V tiles of each group go through a 3-buffer LDS ring; the
// dS block accumulates in registers (no atomics).  Partial sums per part are
// added by attn_dbias_reduce_kernel.
// Reference: _backward_shared_bias (oops/attention/triangle/triton/kernel.py:721-873).
// MASKED_TILES: as in attn_dq_fast_kernel.
template <typename T, int DP, bool MASKED_TILES>
__global__ __launch_bounds__(256, OOPS_DBIAS_OCC) void attn_dbias_fast_kernel(BwdArgsT<T, T> a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int LD = DP + 8;
  constexpr int TBUF = 64 * LD;
  constexpr int NQF = DP / 16;
  constexpr int NCH = DP / 32;

  // query side (Q, dO of the wave's 32 queries): loaded with whole-row
  // coalesced loads, then turned into MFMA fragments through a per-wave LDS
  // region (written and read by that wave only)
  constexpr int QLD = DP + 8;
  constexpr int NQR = DP / 16;  // 16-byte chunks per lane for 32 rows
  __shared__ __attribute__((aligned(16))) T k_lds[3 * TBUF];
  __shared__ __attribute__((aligned(16))) T v_lds[3 * TBUF];
  __shared__ __attribute__((aligned(16))) T qw_lds[4 * 2 * 32 * QLD];
  __shared__ uint64_t keep_lds[3];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int g2 = lane >> 5;
  T* const q_w = &qw_lds[wave * 2 * 32 * QLD];
  T* const d_w = q_w + 32 * QLD;

  int64_t tile = xcd_tile(blockIdx.x, gridDim.x, xcd_chunk(a.uniform_tiles));
  if (tile >= a.total_tiles) return;
  const Sample* tab = reinterpret_cast<const Sample*>(a.table);
  const int H = a.num_heads;
  const int s_idx = find_sample(tile, tab, a.num_samples, a.uniform_tiles, [&](const Sample& s) {
    return s.bias_mode == OOPS_BIAS_SHARED && !(a.fused_max_lq > 0 && s.Lq <= a.fused_max_lq)
               ? H * cdiv(s.Lq, 128) * cdiv(s.Lk, 64) * parts_for(s.G, a.part_groups, a.parts)
               : (int64_t)0;
  });
  if (s_idx < 0) return;
  const Sample& S = tab[__builtin_amdgcn_readfirstlane(s_idx)];
  const int64_t G = S.G;
  const int P = parts_for(G, a.part_groups, a.parts);  // this sample's group ranges
  const int Lq = (int)S.Lq, Lk = (int)S.Lk;
  const int nkb = (int)cdiv(Lk, 64);
  const int nqb = (int)cdiv(Lq, 128);
  // logical order (head, part, q block, key block): neighbours share the bias block rows
  const int kb = __builtin_amdgcn_readfirstlane((int)((uint32_t)tile % (uint32_t)nkb));
  uint32_t rest = (uint32_t)tile / (uint32_t)nkb;
  const int qb = __builtin_amdgcn_readfirstlane((int)(rest % (uint32_t)nqb));
  rest /= (uint32_t)nqb;
  const int part = __builtin_amdgcn_readfirstlane((int)(rest % (uint32_t)P));
  const int h = __builtin_amdgcn_readfirstlane((int)(rest / (uint32_t)P));
  const int64_t g_begin = G * part / P, g_end = G * (part + 1) / P;
  const int D = a.head_size;
  const int k0 = kb * 64;
  const int k_si = (int)S.k_si, v_si = (int)S.v_si;
  const bool has_mask = a.mask != nullptr && S.m_off >= 0;

  const int q_lane = qb * 128 + wave * 32 + lq;
  const bool qv = q_lane < Lq;
  const float c1 = a.scale * kLog2e;

  // bias contribution of this (query, key) block, shared by every group
  f32x16 bacc[2];
  {
    Frag ident[2];
    identity_frags<T>(ident, 1.0f / a.scale, lane);
    const T* brow = a.bias + S.b_off + h * S.b_sh + (int64_t)q_lane * S.b_si;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      bacc[t2] = f32x16{};
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int key = k0 + 32 * t2 + 16 * c + g2 * 8;
        uint4 u = make_uint4(0, 0, 0, 0);
        if (qv) {
          if (key + 8 <= Lk) u = *reinterpret_cast<const uint4*>(brow + key);
          else u = load16(brow, key, Lk, false);
        }
        bacc[t2] = E::mma(ident[c], __builtin_bit_cast(Frag, finite16<T>(u)), bacc[t2]);
      }
    }
  }
  f32x16 acc[2];
  acc[0] = acc[1] = f32x16{};

  // per-group K/V tile of the block (64 keys), LDS ring like the other kernels
  uint32_t kv_row[NCH], k_col[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = tid + 256 * i;
    kv_row[i] = c / (DP / 8);
    k_col[i] = (c % (DP / 8)) * 8;
  }
  struct Stage {
    uint4 k[NCH], v[NCH];
    uint64_t bits;
  };
  // row-invariant bases: group g adds g * (group stride)
  const T* k_h = a.k + S.k_off + h * S.k_sh;
  const T* v_h = a.v + S.v_off + h * S.v_sh;
  // (buffer resources must be wave-uniform: lane-dependent parts go in the offsets)
  const T* q_h = a.q + S.q_off + h * S.q_sh;
  const T* do_h = a.dout + S.do_off + h * S.do_sh;
  const uint32_t q_bytes_all = (uint32_t)(((int64_t)(Lq - 1) * S.q_si + D) * 2);
  const uint32_t do_bytes_all = (uint32_t)(((int64_t)(Lq - 1) * S.do_si + D) * 2);
  // chunk i of this lane: row q_row[i] of the wave's 32 queries, columns q_col[i] .. +8
  const int q0w = qb * 128 + wave * 32;
  uint32_t q_ck_off[NQR], do_ck_off[NQR];
  int q_row[NQR], q_col[NQR];
#pragma unroll
  for (int i = 0; i < NQR; ++i) {
    const int c = i * 64 + lane;
    q_row[i] = c / (DP / 8);
    q_col[i] = (c % (DP / 8)) * 8;
    const bool ok = q0w + q_row[i] < Lq && q_col[i] < D;
    q_ck_off[i] = ok ? (uint32_t)(((q0w + q_row[i]) * (int)S.q_si + q_col[i]) * 2) : kOut;
    do_ck_off[i] = ok ? (uint32_t)(((q0w + q_row[i]) * (int)S.do_si + q_col[i]) * 2) : kOut;
  }
  const int64_t k_sg = S.k_sg, v_sg = S.v_sg, q_sg = S.q_sg, do_sg = S.do_sg;
  const float* l_h = a.lse + S.l_off + (int64_t)h * Lq;
  const float* d_h = a.delta + S.l_off + (int64_t)h * Lq;
  const int64_t l_sg = (int64_t)H * Lq;
  const uint8_t* m_h = has_mask ? a.mask + S.m_off : nullptr;
  const int64_t m_sg = S.m_sg;
  const uint32_t kv_bytes_k = (uint32_t)(((int64_t)(Lk - 1) * k_si + D) * 2);
  const uint32_t kv_bytes_v = (uint32_t)(((int64_t)(Lk - 1) * v_si + D) * 2);
  auto load_stage = [&](int64_t g, Stage& st) {
    const bool live = g < g_end;  // past the part: zero-traffic loads, no branch
    const int64_t gg = live ? g : g_begin;
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(k_h + gg * k_sg, kv_bytes_k);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(v_h + gg * v_sg, kv_bytes_v);
    const int key = k0 + lane;
    bool keep = live && key < Lk;
    if (keep && m_h) keep = m_h[gg * m_sg + key] != 0;
    st.bits = __ballot(keep);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const bool ok = ((st.bits >> kv_row[i]) & 1) && (int)k_col[i] < D;
      const int kk = k0 + kv_row[i];
      st.k[i] = buffer_load16(kr, ok ? (uint32_t)((kk * k_si + k_col[i]) * 2) : kOut);
      st.v[i] = buffer_load16(vr, ok ? (uint32_t)((kk * v_si + k_col[i]) * 2) : kOut);
    }
  };
  auto store_stage = [&](int buf, const Stage& st) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      *reinterpret_cast<uint4*>(&k_lds[buf * TBUF + kv_row[i] * LD + k_col[i]]) = st.k[i];
      *reinterpret_cast<uint4*>(&v_lds[buf * TBUF + kv_row[i] * LD + k_col[i]]) = st.v[i];
    }
    if (tid == 0) keep_lds[buf] = st.bits;
  };
  // per-group query-side operands of this lane (registers)
  // Raw loads only: any arithmetic on a loaded value here would make the
  // wave wait for the load at once.  Queries past Lq read zeros (their
  // scores then contribute P * (0 - 0) = 0 and are never written).
  struct QStage {
    uint4 q[NQR], d[NQR];
    float lse, dlt;
  };
  auto load_q = [&](int64_t g, QStage& qs) {
    const bool live = g < g_end;
    const int64_t gg = live ? g : g_begin;
    const __amdgpu_buffer_rsrc_t qrs = make_rsrc(q_h + gg * q_sg, q_bytes_all);
    const __amdgpu_buffer_rsrc_t drs = make_rsrc(do_h + gg * do_sg, do_bytes_all);
#pragma unroll
    for (int i = 0; i < NQR; ++i) {
      qs.q[i] = buffer_load16(qrs, live ? q_ck_off[i] : kOut);
      qs.d[i] = buffer_load16(drs, live ? do_ck_off[i] : kOut);
    }
    const __amdgpu_buffer_rsrc_t lr = make_rsrc(l_h + gg * l_sg, (uint32_t)(Lq * 4));
    const __amdgpu_buffer_rsrc_t drr = make_rsrc(d_h + gg * l_sg, (uint32_t)(Lq * 4));
    const uint32_t loff = live && qv ? (uint32_t)(q_lane * 4) : kOut;
    qs.lse = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(lr, loff, 0, 0));
    qs.dlt = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(drr, loff, 0, 0));
  };
  // the wave's rows into its LDS region, then this lane's fragments back
  // (LDS operations of one wave complete in order, so the region is free
  // again once the fragments have been read)
  auto q_frags = [&](const QStage& qs, Frag (&qf)[NQF], Frag (&df)[NQF]) {
#pragma unroll
    for (int i = 0; i < NQR; ++i) {
      *reinterpret_cast<uint4*>(&q_w[q_row[i] * QLD + q_col[i]]) = qs.q[i];
      *reinterpret_cast<uint4*>(&d_w[q_row[i] * QLD + q_col[i]]) = qs.d[i];
    }
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      qf[s] = lds_frag<T>(&q_w[lq * QLD + s * 16 + g2 * 8]);
      df[s] = lds_frag<T>(&d_w[lq * QLD + s * 16 + g2 * 8]);
    }
  };

  const int64_t ng = g_end - g_begin;
  Stage stg;
  QStage qc;
  if (ng > 0) {
    load_stage(g_begin, stg);
    store_stage(0, stg);
  }
  if (ng > 1) {
    load_stage(g_begin + 1, stg);
    store_stage(1, stg);
  }
  load_q(g_begin, qc);
  load_stage(g_begin + 2, stg);
  vmem_wait_all();
  __syncthreads();
  int buf = 0;
  for (int64_t i = 0; i < ng; ++i) {
    const int b1 = buf == 2 ? 0 : buf + 1;
    const int b2 = b1 == 2 ? 0 : b1 + 1;
    if (i + 2 < ng) store_stage(b2, stg);
    load_stage(g_begin + i + 3, stg);
    const T* kt = &k_lds[buf * TBUF];
    const T* vt = &v_lds[buf * TBUF];
    const uint64_t bits = uniform64(keep_lds[buf]);
    const uint64_t lb = bits >> (g2 * 4);
    Frag qf[NQF], df[NQF];
    q_frags(qc, qf, df);
    const float ndlt = -qc.dlt, nlse = -qc.lse;
    // one set of query-side registers: the next group's rows are loaded as
    // soon as this group's have gone through LDS
    load_q(g_begin + i + 1, qc);
    f32x16 nd;
#pragma unroll
    for (int j = 0; j < 16; ++j) nd[j] = ndlt;
    // fully kept tiles take the variant without per-score mask work
    auto tile = [&](auto masked) {
      constexpr bool MASKED = decltype(masked)::value;
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        f32x16 sacc = bacc[t2];
        f32x16 pacc = nd;
#pragma unroll
        for (int s = 0; s < NQF; ++s) {
          sacc = E::mma(lds_frag<T>(kt + (32 * t2 + lq) * LD + s * 16 + g2 * 8), qf[s], sacc);
          pacc = E::mma(lds_frag<T>(vt + (32 * t2 + lq) * LD + s * 16 + g2 * 8), df[s], pacc);
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j], c1, nlse));
          if constexpr (MASKED) {
            const int kk = 32 * t2 + ((j >> 2) << 3) + (j & 3);
            p = ((lb >> kk) & 1) ? p : 0.0f;
          }
          acc[t2][j] = __builtin_fmaf(p, pacc[j], acc[t2][j]);
        }
      }
    };
    if (!MASKED_TILES || bits == ~uint64_t(0))
      tile(std::false_type{});
    else if constexpr (MASKED_TILES)
      tile(std::true_type{});
    lds_barrier();
    buf = b1;
  }

  if (qv) {
    float* dst = P == 1 ? a.dbias : a.dbias_part + (int64_t)part * a.dbias_extent;
    float* row = dst + S.db_off + h * S.db_sh + (int64_t)q_lane * S.db_si;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int j = 0; j < 16; j += 4) {
        const int key = k0 + 32 * t2 + kappa(g2, j);
        if (key + 3 < Lk) {
          *reinterpret_cast<float4*>(row + key) = make_float4(acc[t2][j], acc[t2][j + 1], acc[t2][j + 2], acc[t2][j + 3]);
        } else {
          for (int e = 0; e < 4; ++e)
            if (key + e < Lk) row[key + e] = acc[t2][j + e];
        }
      }
  }
}

#define OOPS_DQ_FAST_INST(T, DP, B)                                                                \
  template __global__ void attn_dq_fast_kernel<T, DP, B, false, false, false>(BwdArgsT<T, T>); \
  template __global__ void attn_dq_fast_kernel<T, DP, B, true, false, false>(BwdArgsT<T, T>);  \
  template __global__ void attn_dq_fast_kernel<T, DP, B, false, true, false>(BwdArgsT<T, T>);  \
  template __global__ void attn_dq_fast_kernel<T, DP, B, true, true, false>(BwdArgsT<T, T>);
#define OOPS_BWD_FAST_INST(T, DP)                                                \
  template __global__ void attn_dkv_fast_kernel<T, DP, true, 1>(BwdArgsT<T, T>);  \
  template __global__ void attn_dkv_fast_kernel<T, DP, true, 2>(BwdArgsT<T, T>);  \
  template __global__ void attn_dkv_fast_kernel<T, DP, false, 1>(BwdArgsT<T, T>); \
  OOPS_DQ_FAST_INST(T, DP, true)                                                 \
  OOPS_DQ_FAST_INST(T, DP, false)                                                \
  template __global__ void attn_dbias_fast_kernel<T, DP, false>(BwdArgsT<T, T>);     \
  template __global__ void attn_dbias_fast_kernel<T, DP, true>(BwdArgsT<T, T>);
OOPS_BWD_FAST_INST(__bf16, 32)
OOPS_BWD_FAST_INST(__bf16, 64)
template __global__ void attn_dq_fast_kernel<__bf16, 32, true, true, false, true>(BwdArgsT<__bf16, __bf16>);
template __global__ void attn_dq_fast_kernel<__bf16, 64, true, true, false, true>(BwdArgsT<__bf16, __bf16>);
OOPS_BWD_FAST_INST(_Float16, 32)
OOPS_BWD_FAST_INST(_Float16, 64)

bool backward_fast_ok(const oops_attn_geometry& geo, const Plan& plan) { return fast_path_ok(geo, plan); }

template <typename F>
hipError_t dispatch_fast(const oops_attn_geometry& geo, const Plan& plan, F&& f) {
  hipError_t err = hipSuccess;
  auto go = [&](auto tag, auto dpc) { err = f(tag, dpc); };
  if (geo.dtype == OOPS_BF16) {
    if (plan.dp == 32) go(Tag<__bf16>{}, std::integral_constant<int, 32>{});
    else go(Tag<__bf16>{}, std::integral_constant<int, 64>{});
  } else {
    if (plan.dp == 32) go(Tag<_Float16>{}, std::integral_constant<int, 32>{});
    else go(Tag<_Float16>{}, std::integral_constant<int, 64>{});
  }
  return err;
}

hipError_t launch_dkv_fast(const oops_attn_geometry& geo, const Plan& plan, const BwdLaunch& L, hipStream_t stream,
                           bool rest) {
  return dispatch_fast(geo, plan, [&](auto tag, auto dpc) {
    using T = typename decltype(tag)::type;
    constexpr int DP = decltype(dpc)::value;
    BwdArgsT<T, T> a;
    fill_bwd_args(a, geo, plan, L);
    // OOPS_DKV_ROWS=2: two rows per workgroup share each bias fragment (row-shared
    // biases only); it costs a wave of occupancy and measured slower at the headline shape
    const bool pair = !rest && OOPS_DKV_ROWS == 2 && a.bias != nullptr && !plan.any_full && plan.dkv_tiles_r2 > 0;
    a.uniform_tiles = pair ? plan.dkv_uniform_r2 : plan.dkv_uniform;
    a.total_tiles = pair ? plan.dkv_tiles_r2 : plan.dkv_tiles;
    if (rest) {
      a.fused_max_lq = kFusedMaxLen;
      a.uniform_tiles = 0;
      a.total_tiles = plan.dkv_rest_tiles;
    }
    if (a.total_tiles == 0) return hipSuccess;
    const dim3 grid((unsigned)xcd_grid(a.total_tiles, xcd_chunk(a.uniform_tiles)));
    if (pair)
      hipLaunchKernelGGL((attn_dkv_fast_kernel<T, DP, true, 2>), grid, dim3(256), 0, stream, a);
    else if (a.bias != nullptr)
      hipLaunchKernelGGL((attn_dkv_fast_kernel<T, DP, true, 1>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((attn_dkv_fast_kernel<T, DP, false, 1>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
  });
}

hipError_t launch_dq_fast(const oops_attn_geometry& geo, const Plan& plan, const BwdLaunch& L, bool delta_in_dq,
                          hipStream_t stream) {
  return dispatch_fast(geo, plan, [&](auto tag, auto dpc) {
    using T = typename decltype(tag)::type;
    constexpr int DP = decltype(dpc)::value;
    BwdArgsT<T, T> a;
    fill_bwd_args(a, geo, plan, L);
    a.uniform_tiles = plan.fwd_uniform;
    a.total_tiles = plan.fwd_tiles;
    a.delta_in_dq = delta_in_dq ? 1 : 0;
    // a split batch: compact copies only of the rows the fused kernel reads
    a.fused_max_lq = L.qc != nullptr && plan.fused_split ? kFusedMaxLen : 0;
    const dim3 grid((unsigned)xcd_grid(plan.fwd_tiles, xcd_chunk(plan.fwd_uniform)));
    const bool full = a.dbias != nullptr && plan.any_full;
    auto go = [&](auto has_bias, auto masked, auto full_db, auto fold) {
      hipLaunchKernelGGL((attn_dq_fast_kernel<T, DP, decltype(has_bias)::value, decltype(masked)::value,
                                              decltype(full_db)::value, decltype(fold)::value>),
                         grid, dim3(256), 0, stream, a);
    };
    auto by_full = [&](auto has_bias, auto masked) {
      if constexpr (decltype(has_bias)::value && decltype(masked)::value && std::is_same_v<T, __bf16>) {
        if (!full && fold_masks_ok(plan)) return go(has_bias, masked, std::false_type{}, std::true_type{});
      }
      if (full) go(has_bias, masked, std::true_type{}, std::false_type{});
      else go(has_bias, masked, std::false_type{}, std::false_type{});
    };
    auto by_mask = [&](auto has_bias) {
      if (plan.masked_tiles) by_full(has_bias, std::true_type{});
      else by_full(has_bias, std::false_type{});
    };
    if (a.bias != nullptr) by_mask(std::true_type{});
    else by_mask(std::false_type{});
    return hipGetLastError();
  });
}

hipError_t launch_dbias_fast(const oops_attn_geometry& geo, const Plan& plan, const BwdLaunch& L,
                             hipStream_t stream, bool rest) {
  return dispatch_fast(geo, plan, [&](auto tag, auto dpc) {
    using T = typename decltype(tag)::type;
    constexpr int DP = decltype(dpc)::value;
    BwdArgsT<T, T> a;
    fill_bwd_args(a, geo, plan, L);
    a.parts = plan.fast_parts;
    a.part_groups = plan.fast_part_groups;
    a.uniform_tiles = rest ? 0 : plan.fast_sbias_uniform;
    a.total_tiles = rest ? plan.fast_sbias_rest_tiles : plan.fast_sbias_tiles;
    if (rest) a.fused_max_lq = kFusedMaxLen;
    if (a.total_tiles == 0) return hipSuccess;
    const dim3 grid((unsigned)xcd_grid(a.total_tiles, xcd_chunk(a.uniform_tiles)));
    if (plan.masked_tiles)
      hipLaunchKernelGGL((attn_dbias_fast_kernel<T, DP, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((attn_dbias_fast_kernel<T, DP, false>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
  });
}

}  // namespace oops
