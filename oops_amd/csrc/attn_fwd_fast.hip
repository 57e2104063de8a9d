// Forward fast path for 16-bit Q/K/V (bias in the same dtype or absent),
// head size <= 64 and a multiple of 8: the configuration of the headline
// workload.
//
// At head size 32 every score costs only 128 MFMA flops, so the per-score
// vector work (scale, bias, exponent, row statistics, conversion) bounds the
// kernel, not the matrix cores.  The kernel therefore
//   * adds the bias on the matrix core: acc += I(1/scale) x bias, with a
//     constant identity A-fragment and the bias rows (natural layout, one
//     16-byte load per fragment) as the B-fragment, so a logit costs one FMA
//     (x = acc * scale * log2 e - m) before its exponent;
//   * raises the running max lazily (only when it grows by more than 2^8),
//     so the O rescale is skipped on almost every step;
//   * sums the row with v_dot2 on the packed probabilities that also feed
//     the PV MFMA;
//   * resolves masks per 64-key tile from a bitmap built once per
//     workgroup: fully kept tiles do no mask work, fully masked tiles are
//     skipped, only mixed tiles select per score;
//   * writes O and its rounding residual with whole 64-byte row segments.
// Work split: 4 wavefronts x 32 queries per workgroup, 64 keys per step.
// K and V tiles go from global memory straight into a 4-buffer LDS ring
// (buffer_load ... lds, issued three steps ahead, one barrier per step); K
// rows are XOR-swizzled in 16-byte chunks so the fragment reads are free of
// bank conflicts, and the PV MFMA reads V^T fragments with the gfx950 LDS
// transpose read.  Bias fragments are loaded from global memory straight
// into registers one step ahead.  All loads use range-checked buffer
// resources; a tile past the end reads at an out-of-range offset (zeros, no
// memory traffic) so every load is unconditional and the wait counts stay
// exact.
//
// Semantics are those of the generic forward (attn_fwd.hip), i.e. of the
// reference's _attend (oops/attention/triangle/triton/kernel.py:151-262):
// masked keys read as -inf logits with zero K/V, fully masked rows give
// O = 0 and LSE = 0.  The bias weight 1/scale is rounded to the input dtype
// (relative error <= 2^-9 for bf16), below the rounding of P itself.
#include "attn_fast_common.h"


namespace oops {

using namespace fast;

constexpr int kRing = 4;  // K/V tile buffers in LDS


// MASKED_TILES: the geometry may have 64-key tiles with masked or
// out-of-range keys; without it the per-score mask code is not compiled
// (it costs registers even when never executed).  FOLD (bf16, bias, at most
// kFoldTiles key tiles): the masks are folded into the bias fragments
// instead of selected per score.
template <typename T, int DP, bool HAS_BIAS, bool MASKED_TILES, bool FOLD>
__global__ __launch_bounds__(256, OOPS_FWD_OCC) void attn_fwd_fast_kernel(FwdArgsT<T, T> a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  using P2 = typename Pair<T>::v2;
  constexpr int NDT = DP / 32;
  constexpr int NQF = DP / 16;
  constexpr int KT = 64 * DP;        // elements per K (or V) tile: 64 swizzled rows
  constexpr int CPR = DP / 8;        // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;      // rows per direct-to-LDS load of a wave
  constexpr int IPW = 16 / RPI;      // loads per wave per tile and tensor (16 rows per wave)
  constexpr int NDMA = 2 * IPW;      // K and V loads per wave per tile

  // The ring position is a compile-time constant wherever a buffer is
  // addressed (the loop is unrolled over the ring): buffer offsets become
  // instruction immediates, and the compiler can tell that the loads into
  // one buffer do not overlap the reads of another.  The waits for the
  // direct-to-LDS loads are explicit (before each step's barrier).
  __shared__ __attribute__((aligned(16))) T k_lds[kRing * KT];
  __shared__ __attribute__((aligned(16))) T v_lds[kRing * KT];
  auto kbuf = [&](auto bc) -> T* { return k_lds + decltype(bc)::value * KT; };
  auto vbuf = [&](auto bc) -> T* { return v_lds + decltype(bc)::value * KT; };
  __shared__ uint64_t keep_lds[kMaxKeyTiles];
  __shared__ __attribute__((aligned(16))) uint32_t fold_lds[FOLD ? kFoldTiles * 32 : 4];
  static_assert(!FOLD || (MASKED_TILES && HAS_BIAS && sizeof(T) == 2), "fold: masked bf16 tiles with a bias");

  const int tid = threadIdx.x;
  // wave-uniform (scalar); & 3 lets the compiler bound LDS addresses
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6) & 3;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int g2 = lane >> 5;

  // XCD-aware order: the dispatcher deals workgroups round-robin to the 8
  // XCDs, so workgroup b runs on XCD b % 8; each XCD gets one contiguous
  // range of logical tiles.  Within a sample the logical order is
  // (head group, group g, head in group, query block): the query blocks of
  // one (g, head group) share K/V in one L2, and each XCD sees the bias of
  // only its head group.
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

  const T* kbase = a.k + S.k_off + g * S.k_sg + h * S.k_sh;
  const T* vbase = a.v + S.v_off + g * S.v_sg + h * S.v_sh;
  const bool has_mask = a.mask != nullptr && S.m_off >= 0;
  const uint8_t* mbase = has_mask ? a.mask + S.m_off + g * S.m_sg : nullptr;

  // ---- per 64-key tile keep bitmaps (bit i: key 64t+i in range and kept);
  // without mixed tiles (no mask, Lk a multiple of 64) every tile is whole
  if constexpr (MASKED_TILES) for (int t = wave; t < ntiles; t += 4) {
    const int key = t * 64 + lane;
    bool keep = key < Lk;
    if (keep && has_mask) keep = mbase[key] != 0;
    const uint64_t bits = __ballot(keep);
    if (lane == 0) keep_lds[t] = bits;
  }

  const int q_lane = qb * 128 + wave * 32 + lq;
  const bool qv = q_lane < Lq;
  Frag qf[NQF];
  {
    const T* qrow = a.q + S.q_off + g * S.q_sg + h * S.q_sh + (int64_t)q_lane * S.q_si;
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
      const int col = s * 16 + g2 * 8;
      qf[s] = __builtin_bit_cast(
          Frag, qv && col < D ? *reinterpret_cast<const uint4*>(qrow + col) : make_uint4(0, 0, 0, 0));
    }
  }
  // identity A-fragments carrying the bias weight 1/scale: MFMA c adds bias keys 16c..16c+15
  Frag ident[2];
  identity_frags<T>(ident, 1.0f / a.scale, lane);

  // ---- fixed per-lane offsets (bytes) of the direct-to-LDS tile loads:
  // wave w fills rows 16w .. 16w+15 of the K and V tiles; lane l writes slot
  // l of its load, i.e. row l / CPR, slot l % CPR, which holds the logical
  // chunk (l % CPR) ^ swz(row).  The step adds k0 * stride via soffset.
  const __amdgpu_buffer_rsrc_t k_rsrc = make_rsrc(kbase, (uint32_t)(((int64_t)(Lk - 1) * k_si + D) * 2));
  const __amdgpu_buffer_rsrc_t v_rsrc = make_rsrc(vbase, (uint32_t)(((int64_t)(Lk - 1) * v_si + D) * 2));
  // empty ranges: the loads of an absent tile (t >= ntiles) read zeros and make no memory request
  const __amdgpu_buffer_rsrc_t k_none = make_rsrc(kbase, 0u), v_none = make_rsrc(vbase, 0u);
  int d_row[IPW];
  uint32_t k_off[IPW], v_off[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int r = 16 * wave + i * RPI + lane / CPR;
    const int col = ((lane % CPR) ^ swz<DP>(r)) * 8;  // K: swizzled rows
    const int vcol = (lane % CPR) * 8;                // V: plain rows
    d_row[i] = r;
    k_off[i] = col < D ? (uint32_t)((r * k_si + col) * 2) : kOut;
    v_off[i] = vcol < D ? (uint32_t)((r * v_si + vcol) * 2) : kOut;
  }
  // bias fragments: from the fragment-major copy of a shared bias (one
  // contiguous 1 KB load per fragment), else from the bias rows themselves
  const bool use_bf = HAS_BIAS && a.bias_frag != nullptr && S.bias_mode == OOPS_BIAS_SHARED;
  __amdgpu_buffer_rsrc_t b_rsrc, b_none;
  uint32_t b_off[2][2], b_step;
  if (use_bf) {
    const int qt = qb * 4 + wave;
    // a wave wholly past Lq may index a tile row beyond the copy: empty range
    const bool in = qt < a.bf_nqt;
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

  // tile -> registers (K, V chunks of this thread; masked keys read zeros)
  // An absent tile (t >= ntiles) issues its loads with out-of-range offsets:
  // no memory traffic, and no branch, so the compiler can count outstanding
  // loads exactly and never has to wait for all of them.
  auto load_kv = [&](int t, auto bc) {
    const uint32_t ks = (uint32_t)(t * 64 * k_si * 2), vs = (uint32_t)(t * 64 * v_si * 2);
    if constexpr (!MASKED_TILES) {
      // whole tiles: the per-lane offsets are fixed, an absent tile takes the empty ranges
      const bool live = t < ntiles;
#pragma unroll
      for (int i = 0; i < IPW; ++i) {
        const int r0 = 16 * wave + i * RPI;
        dma16(live ? k_rsrc : k_none, kbuf(bc) + r0 * DP, k_off[i], ks);
        dma16(live ? v_rsrc : v_none, vbuf(bc) + r0 * DP, v_off[i], vs);
      }
      return;
    }
    const uint64_t bits = t < ntiles ? keep_lds[t < ntiles ? t : 0] : 0;
    const bool full = bits == ~uint64_t(0);
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const bool ok = full || ((bits >> d_row[i]) & 1);
      const int r0 = 16 * wave + i * RPI;
      dma16(k_rsrc, kbuf(bc) + r0 * DP, ok ? k_off[i] : kOut, ks);
      dma16(v_rsrc, vbuf(bc) + r0 * DP, ok ? v_off[i] : kOut, vs);
    }
  };
  // bias B-fragments of a tile: keys past Lk fall in the next row or past the
  // resource; both are masked (mixed tile) or read as zero
  // (the tile offset goes into the vector offset: the hardware range check
  // covers the vector offset, which keeps the last row's tail in bounds)
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
  };
  // S^T of a tile (bias by identity MFMA, then Q K^T) from LDS buffer buf
  auto scores = [&](auto bc, int t, const uint4 (&bf)[2][2], f32x16 (&sacc)[2]) {
    const uint4* fm = reinterpret_cast<const uint4*>(&fold_lds[FOLD ? (t * 2 + g2) * 16 : 0]);
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      if constexpr (HAS_BIAS) {
        // (bias rows read directly are made finite here; the fragment-major copy holds finite values)
        const uint4 r0 = use_bf ? bf[t2][0] : finite16<T>(bf[t2][0]);
        const uint4 r1 = use_bf ? bf[t2][1] : finite16<T>(bf[t2][1]);
        const uint4 b0 = FOLD ? fold_bias(r0, fm[t2 * 2]) : r0;
        const uint4 b1 = FOLD ? fold_bias(r1, fm[t2 * 2 + 1]) : r1;
        sacc[t2] = E::mma(ident[0], __builtin_bit_cast(Frag, b0), f32x16{});
        sacc[t2] = E::mma(ident[1], __builtin_bit_cast(Frag, b1), sacc[t2]);
      } else {
        sacc[t2] = f32x16{};
      }
#pragma unroll
      for (int s = 0; s < NQF; ++s) {
        const Frag kf = __builtin_bit_cast(
            Frag, *reinterpret_cast<const uint4*>(kbuf(bc) + swz_off<DP>(32 * t2 + lq, s * 16 + g2 * 8)));
        sacc[t2] = E::mma(kf, qf[s], sacc[t2]);
      }
    }
  };

  if constexpr (MASKED_TILES) __syncthreads();  // keep bitmaps visible
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
  float m_run = kNegInf;  // reference max (log2 units), raised lazily
  float neg_m = 0.0f;     // -m_run (0 while no key has been seen)
  float l_run = 0.0f;     // this lane's partial row sum
  f32x16 oacc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) oacc[t] = f32x16{};
  P2 ones;
  ones[0] = (T)1.0f;
  ones[1] = (T)1.0f;

  // softmax of one tile's scores + O^T += V^T P^T from LDS buffer buf
  auto attend = [&](auto bc, uint64_t bits, f32x16 (&sacc)[2]) {
    if (MASKED_TILES && !FOLD && bits != ~uint64_t(0)) {
      // mixed tile: masked / out-of-range keys get -inf
      const uint64_t lb = bits >> (g2 * 4);
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int kk = 32 * t2 + ((j >> 2) << 3) + (j & 3);
          sacc[t2][j] = ((lb >> kk) & 1) ? sacc[t2][j] : kNegInf;
        }
    }
    // tile max: two chains of three-operand maxima (v_max3, two new values
    // per operation: 17 operations for 32 values), then across the halves
    float mc[2];
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      float x = fmaxf(fmaxf(sacc[t2][0], sacc[t2][1]), sacc[t2][2]);
#pragma unroll
      for (int j = 3; j < 15; j += 2) x = fmaxf(fmaxf(x, sacc[t2][j]), sacc[t2][j + 1]);
      mc[t2] = fmaxf(x, sacc[t2][15]);
    }
    float mx = max_halves(fmaxf(mc[0], mc[1])) * c1;
    const bool grow = mx > m_run + kLazyRescale;
    if (__any(grow)) {
      const float m_new = grow ? mx : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      neg_m = m_run == kNegInf ? 0.0f : -m_run;
      l_run *= alpha;
#pragma unroll
      for (int t = 0; t < NDT; ++t) oacc[t] *= alpha;
    }
    // the row sum: one v_dot2 chain into l_run (the exponentials between its
    // links hide their latency; no chain registers to clear or add up)
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        Frag pf;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          P2 pr;
          pr[0] = (T)__builtin_amdgcn_exp2f(__builtin_fmaf(sacc[t2][8 * m + e], c1, neg_m));
          pr[1] = (T)__builtin_amdgcn_exp2f(__builtin_fmaf(sacc[t2][8 * m + e + 1], c1, neg_m));
          l_run = Pair<T>::dot(pr, ones, l_run);
          pf[e] = pr[0];
          pf[e + 1] = pr[1];
        }
#pragma unroll
        for (int t = 0; t < NDT; ++t) {
          const Frag vf = lds_read_tr_frag<T>(vbuf(bc), DP, 32 * t2 + 16 * m, t * 32, lane);
          oacc[t] = E::mma(vf, pf, oacc[t]);
        }
      }
  };

  // ---- pipeline.  Step i computes tile t0 from ring buffer i % kRing.  It
  // first issues the direct-to-LDS loads of the tile kRing - 1 steps ahead
  // (into the buffer the previous step released), then S of t0 (its bias
  // fragments were loaded one step ahead), then the bias loads of t1, then
  // the softmax and PV of t0.  Before the step's barrier, the loads of the
  // next step's tile must have landed: issued two steps earlier, they are
  // followed by 2 * NDMA tile loads and 3 x 4 bias loads.
  static_assert(kRing == 4, "the wait count below assumes a 4-buffer ring");
  uint4 bias_a[2][2];
  f32x16 sacc[2];
  int t0 = next_tile(-1);
  int t1 = next_tile(t0);
  int t2 = next_tile(t1);
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  using B2 = std::integral_constant<int, 2>;
  using B3 = std::integral_constant<int, 3>;
  load_kv(t0, B0{});
  load_kv(t1, B1{});
  load_kv(t2, B2{});
  if constexpr (HAS_BIAS) load_bias(t0, bias_a);
  // drain every prologue load (Q included) so that only the loads issued
  // in the loop are ever in flight there
  vmem_wait_all();
  __syncthreads();
  // the ring position is a compile-time constant in each of four unrolled steps
  auto step = [&](auto bc, auto bc_load) {
    const int t3 = next_tile(t2);
    const uint64_t bits = MASKED_TILES ? keep_lds[t0] : ~uint64_t(0);
    load_kv(t3, bc_load);
    scores(bc, t0, bias_a, sacc);
    if constexpr (HAS_BIAS) load_bias(t1, bias_a);
    attend(bc, bits, sacc);
    vmem_wait<2 * NDMA + (HAS_BIAS ? 12 : 0)>();
    lds_barrier();
    t0 = t1;
    t1 = t2;
    t2 = t3;
  };
  while (t0 < ntiles) {
    step(B0{}, B3{});
    if (t0 >= ntiles) break;
    step(B1{}, B0{});
    if (t0 >= ntiles) break;
    step(B2{}, B1{});
    if (t0 >= ntiles) break;
    step(B3{}, B2{});
  }

  // ---- epilogue
  const float l_tot = sum_halves(l_run);
  const float inv = 1.0f / (l_tot == 0.0f ? 1.0f : l_tot);
  if (qv) {
    const int64_t o_row = S.o_off + g * S.o_sg + h * S.o_sh + (int64_t)q_lane * S.o_si;
    T* orow = a.out + o_row;
    T* lrow = a.out_lo != nullptr ? a.out_lo + o_row : nullptr;
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      float o[16], r[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        o[e] = oacc[t][e] * inv;
        r[e] = o[e] - E::to_f(E::from_f(o[e]));  // rounding residual of the output
      }
      store_tile<T>(orow, t * 32, D, g2, o, 1.0f);
      if (lrow) store_tile<T>(lrow, t * 32, D, g2, r, 1.0f);
    }
    if (g2 == 0 && a.lse != nullptr) {
      const float m_use = m_run == kNegInf ? 0.0f : m_run;
      a.lse[S.l_off + ((int64_t)g * H + h) * Lq + q_lane] = l_tot == 0.0f ? 0.0f : m_use + __log2f(l_tot);
    }
  }
}

#define OOPS_FWD_FAST_INST(T, DP)                                                       \
  template __global__ void attn_fwd_fast_kernel<T, DP, true, false, false>(FwdArgsT<T, T>);  \
  template __global__ void attn_fwd_fast_kernel<T, DP, true, true, false>(FwdArgsT<T, T>);   \
  template __global__ void attn_fwd_fast_kernel<T, DP, false, false, false>(FwdArgsT<T, T>); \
  template __global__ void attn_fwd_fast_kernel<T, DP, false, true, false>(FwdArgsT<T, T>);
OOPS_FWD_FAST_INST(__bf16, 32)
template __global__ void attn_fwd_fast_kernel<__bf16, 32, true, true, true>(FwdArgsT<__bf16, __bf16>);
template __global__ void attn_fwd_fast_kernel<__bf16, 64, true, true, true>(FwdArgsT<__bf16, __bf16>);
OOPS_FWD_FAST_INST(__bf16, 64)
OOPS_FWD_FAST_INST(_Float16, 32)
OOPS_FWD_FAST_INST(_Float16, 64)

bool fold_masks_ok(const Plan& plan) { return plan.max_len_k <= 64 * kFoldTiles; }

bool fast_path_ok(const oops_attn_geometry& geo, const Plan& plan) {
  if (geo.force_generic == 1) return false;
  if (geo.dtype == OOPS_F32 || plan.dp > 64 || plan.max_len_k > 64 * kMaxKeyTiles || plan.any_pair_mask ||
      !geo.vec_ok || geo.head_size % 8 != 0 || !plan.offsets_32bit)
    return false;
  return !(geo.has_bias && geo.bias_dtype != geo.dtype);
}

// attn_bias_frag_kernel: the fragment-major copy of every shared bias.  For
// sample s, head h, 32-query tile qt and 32-key tile kt the copy holds
// 2 x 64 entries of 8 elements: entry (c, lane) = bias[qt*32 + lane%32]
// [kt*32 + 16c + 8*(lane/32) .. +8], zero outside the sample.  These are
// exactly the bias fragments of the fast kernels' identity MFMAs, so a wave
// reads a fragment with one contiguous 1 KB load instead of 32 rows of
// 32 bytes (which the L1 serves one row at a time).  One thread per entry.
template <typename T>
__global__ __launch_bounds__(256) void attn_bias_frag_kernel(const T* __restrict__ bias, T* __restrict__ bf,
                                                             const int64_t* table, int num_samples, int H,
                                                             int nqt, int nkt, int64_t sample_stride) {
  const int64_t per_sample = (int64_t)H * nqt * nkt * 128;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= per_sample * num_samples) return;
  const int s = (int)(i / per_sample);
  int64_t r = i - (int64_t)s * per_sample;
  const int lane = (int)(r & 63);
  r >>= 6;
  const int c = (int)(r & 1);
  r >>= 1;
  const int kt = (int)(r % nkt);
  r /= nkt;
  const int qt = (int)(r % nqt);
  const int h = (int)(r / nqt);
  const Sample& S = reinterpret_cast<const Sample*>(table)[s];
  uint4 v = make_uint4(0, 0, 0, 0);
  const int q = qt * 32 + (lane & 31);
  const int k = kt * 32 + 16 * c + 8 * (lane >> 5);
  if (S.bias_mode == OOPS_BIAS_SHARED && S.b_off >= 0 && q < S.Lq && k < S.Lk) {
    const T* row = bias + S.b_off + h * S.b_sh + (int64_t)q * S.b_si;
    if (k + 8 <= S.Lk) {
      v = *reinterpret_cast<const uint4*>(row + k);
    } else {
      T e[8];
      for (int j = 0; j < 8; ++j) e[j] = k + j < S.Lk ? row[k + j] : (T)0.0f;
      v = __builtin_bit_cast(uint4, e);
    }
    v = fast::finite16<T>(v);  // (non-finite elements read as +-max: see finite2)
  }
  const int64_t dst = (int64_t)s * sample_stride + ((((int64_t)h * nqt + qt) * nkt + kt) * 2 + c) * 512 + lane * 8;
  *reinterpret_cast<uint4*>(bf + dst) = v;
}

hipError_t launch_bias_frag(const oops_attn_geometry& geo, const Plan& plan, const void* bias, void* bf,
                            hipStream_t stream) {
  const int64_t n = (int64_t)geo.num_samples * geo.num_heads * plan.bf_nqt * plan.bf_nkt * 128;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (geo.dtype == OOPS_BF16)
    hipLaunchKernelGGL(attn_bias_frag_kernel<__bf16>, grid, dim3(256), 0, stream, static_cast<const __bf16*>(bias),
                       static_cast<__bf16*>(bf), geo.table_device, geo.num_samples, geo.num_heads, plan.bf_nqt,
                       plan.bf_nkt, plan.bf_sample_stride);
  else
    hipLaunchKernelGGL(attn_bias_frag_kernel<_Float16>, grid, dim3(256), 0, stream,
                       static_cast<const _Float16*>(bias), static_cast<_Float16*>(bf), geo.table_device,
                       geo.num_samples, geo.num_heads, plan.bf_nqt, plan.bf_nkt, plan.bf_sample_stride);
  return hipGetLastError();
}

bool launch_forward_fast(const oops_attn_geometry& geo, const Plan& plan, const void* q, const void* k,
                         const void* v, const uint8_t* mask, const void* bias, const void* bias_frag, void* out,
                         void* out_lo, float* lse, hipStream_t stream, hipError_t* err) {
  if (!fast_path_ok(geo, plan)) return false;
  auto go = [&](auto tag, auto dpc) {
    using T = typename decltype(tag)::type;
    constexpr int DP = decltype(dpc)::value;
    FwdArgsT<T, T> a;
    a.q = static_cast<const T*>(q);
    a.k = static_cast<const T*>(k);
    a.v = static_cast<const T*>(v);
    a.bias = geo.has_bias ? static_cast<const T*>(bias) : nullptr;
    a.mask = geo.has_mask ? mask : nullptr;
    a.out = static_cast<T*>(out);
    a.out_lo = static_cast<T*>(out_lo);
    a.lse = lse;
    a.table = geo.table_device;
    a.uniform_tiles = plan.fwd_uniform;
    a.num_samples = geo.num_samples;
    a.num_heads = geo.num_heads;
    a.head_size = geo.head_size;
    a.vec_ok = geo.vec_ok;
    a.scale = geo.scale;
    a.total_tiles = plan.fwd_tiles;
    a.head_group = head_group(geo);
    a.bias_frag = static_cast<const T*>(bias_frag);
    a.bf_sample_stride = plan.bf_sample_stride;
    a.bf_nqt = plan.bf_nqt;
    a.bf_nkt = plan.bf_nkt;
    const dim3 grid((unsigned)xcd_grid(plan.fwd_tiles, xcd_chunk(plan.fwd_uniform)));
    auto go = [&](auto has_bias, auto masked, auto fold) {
      hipLaunchKernelGGL((attn_fwd_fast_kernel<T, DP, decltype(has_bias)::value, decltype(masked)::value,
                                               decltype(fold)::value>),
                         grid, dim3(256), 0, stream, a);
    };
    auto by_mask = [&](auto has_bias) {
      if constexpr (decltype(has_bias)::value && std::is_same_v<T, __bf16>) {
        if (plan.masked_tiles && fold_masks_ok(plan)) return go(has_bias, std::true_type{}, std::true_type{});
      }
      if (plan.masked_tiles) go(has_bias, std::true_type{}, std::false_type{});
      else go(has_bias, std::false_type{}, std::false_type{});
    };
    if (a.bias != nullptr) by_mask(std::true_type{});
    else by_mask(std::false_type{});
    *err = hipGetLastError();
  };
  if (plan.fwd_tiles == 0) {
    *err = hipSuccess;
    return true;
  }
  if (geo.dtype == OOPS_BF16) {
    if (plan.dp == 32) go(Tag<__bf16>{}, std::integral_constant<int, 32>{});
    else go(Tag<__bf16>{}, std::integral_constant<int, 64>{});
  } else {
    if (plan.dp == 32) go(Tag<_Float16>{}, std::integral_constant<int, 32>{});
    else go(Tag<_Float16>{}, std::integral_constant<int, 64>{});
  }
  return true;
}

}  // namespace oops
