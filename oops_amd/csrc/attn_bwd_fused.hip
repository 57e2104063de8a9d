// Fused dK, dV and row-shared dBias for 16-bit Q/K/V, head size <= 32.
//
// The backward of attention over G groups (rows of the pair representation)
// with one bias shared by every group needs three reductions along three
// different axes: dQ sums over keys, dK and dV over queries, and the shared
// dBias over groups.  The dQ kernel (attn_dq_fast_kernel, which also writes
// delta) owns the first; this kernel owns the other two, so each score's P
// and dS are formed once for dK, dV and dBias together instead of once in a
// dK/dV kernel and again in a dBias kernel.
//
// One workgroup = 8 wavefronts = 32 keys of one (sample, head) and one range
// ("part") of the groups.  The waves form groups of RW: with RW = 4 two
// groups work on two rows (groups g, g + 1) at a time, wave w of a group
// taking the 32-query tiles w, w + 4, w + 8, ... (at most six, Lq <= 768);
// with RW = 8 all eight waves work on one row, wave w taking the tiles w,
// w + 8, w + 16, w + 24 (Lq <= 1024).  Every lane owns one key (the MFMA
// column).  Per step a wave computes, for one query tile,
//   S  = Q K^T (+ bias by an identity MFMA, - LSE as the accumulator input),
//   dP = dO V^T - delta,   P = exp2(S * scale * log2 e),   dS = P * dP,
//   dV^T += dO^T P,  dK^T += Q^T dS,  region[step] += dS.
// The dBias region of a wave (32 keys x its query tiles) stays in registers
// for the whole part.  At the end of each row its group's partials of dK and
// dV are summed in a fixed order through LDS and stored, whole 64-byte key
// rows at a time; at the end of the part the regions go to the part's dBias
// slab (with two groups, the second group's through LDS to the first's), and
// attn_dbias_reduce_kernel sums the slabs.  No atomics: results are
// bit-identical from run to run.
//
// Data movement: every load of the main loop goes straight from global
// memory to LDS (buffer_load ... lds, issued through inline assembly and
// ordered by explicit vmcnt waits).  Q and dO come from the head-major
// compact copies the dQ kernel writes (2 KB contiguous per tile), -LSE/c and
// -delta from the pack it writes beside them.  Each wave has its own LDS
// ring (3 stages with RW = 4, 2 with RW = 8) of Q and dO tiles with
// XOR-swizzled rows, -LSE/c and -delta, filled one or two steps ahead, so
// the steps need no workgroup barrier; each group's K/V block and keep bytes
// go into one slot per group, loaded during the previous row; the bias of
// the workgroup's 32 keys and all query tiles (identity-MFMA fragments, from
// the fragment-major copy made by attn_bias_frag_kernel) is loaded into LDS
// once per part.  Two barriers per tensor at each row's end, around the
// dK/dV sum, which reuses the ring stage just read.
//
// Semantics: the reference's _backward_key_value and _backward_shared_bias
// (oops/attention/triangle/triton/kernel.py:569-873, generic.py:484-534) with
// softmax_backward_dscores (oops/attention/flash/triton/kernel.py:53-62).
// Masked keys get dK = dV = 0 and contribute nothing to dBias.
#include "attn_fast_common.h"

namespace oops {

using namespace fast;

namespace {

constexpr int kFusedWaves = 8;
// Two geometries of the workgroup: RW = 4 waves per group and two groups (two
// rows) in flight, up to 6 query tiles per wave (Lq <= 768), with a 3-stage
// ring; or RW = 8, all eight waves on one row, up to 4 query tiles per wave
// (Lq <= 1024), with a 2-stage ring so that the 64 KB bias region still fits.
constexpr int kFusedMaxSteps = 6;
static_assert(4 * kFusedMaxSteps * 32 == kFusedMaxLen, "the plan's length limit is the kernel's");
static_assert(8 * 4 * 32 == kFusedLongMaxLen, "the plan's long-sample limit is the kernel's");
template <int RW>
constexpr int kStages = RW == 4 ? 3 : 2;
constexpr int kQT = 32 * 32;       // elements of one 32 x 32 tile

// LDS byte address of p (a __shared__ object), as a wave-uniform value: the
// M0 operand of the direct-to-LDS loads below.  The kernel takes the
// addresses of its LDS arrays once and steps them with constant offsets.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)(p));
}
// Direct-to-LDS loads through inline assembly (see dma16_asm): 16, 4 or 1
// byte(s) per lane into 64 consecutive slots at LDS address m0 (bytes, 1
// byte into a zero-extended dword).  Every load of the main loop goes
// straight to LDS: none leaves a register waiting for its data, which the
// compiler, not knowing the load, could copy too early.
__device__ __forceinline__ void dma16_m0(const u32x4& r, uint32_t m0, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0),
      "v"(voff), "s"(r)
      : "memory", "m0");
}
__device__ __forceinline__ void dma4_m0(const u32x4& r, uint32_t m0, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dword %1, %2, 0 offen lds" ::"s"(m0),
      "v"(voff), "s"(r)
      : "memory", "m0");
}
__device__ __forceinline__ void dma_u8_m0(const u32x4& r, uint32_t m0, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_ubyte %1, %2, 0 offen lds" ::"s"(m0),
      "v"(voff), "s"(r)
      : "memory", "m0");
}
// s_waitcnt vmcnt(N): all but the last N loads have landed in LDS (the
// memory clobber keeps later LDS reads after it)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// LDS of one wave's ring stage: Q tile, dO tile (swizzled rows), -LSE/c, -delta
struct RingStage {
  uint16_t q[kQT];
  uint16_t d[kQT];
  float ld[64];  // -LSE / c of the 32 queries, then -delta
};

template <typename T, bool MASKED, int NS, int RW>
__global__ __launch_bounds__(512, 1) void attn_dkvb_fast_kernel(BwdArgsT<T, T> a) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  static_assert(sizeof(T) == 2, "16-bit operands");
  static_assert(RW == 2 || RW == 4 || RW == 8, "waves per group");
  static_assert(NS >= 1 && NS <= (RW == 8 ? 4 : kFusedMaxSteps), "query tiles per wave and group");
  constexpr int kRowWaves = RW;
  constexpr int kKvLoads = RW == 2 ? 2 : 1;  // K/V block loads per wave and row
  constexpr int kItems = RW == 2 ? 2 : 1;    // (key, four dims) items each reader thread sums and stores
  constexpr int kGroups = kFusedWaves / RW;  // groups (rows) in flight
  constexpr int NST = kStages<RW>;           // ring stages

  // per-wave ring of NST stages (NST - 1 in flight while one is read); at a
  // pair's end a wave's just-read stage holds its dK/dV partials
  __shared__ __attribute__((aligned(16))) RingStage ring_lds[NST][kFusedWaves];
  // K / V blocks of the groups in flight: [group][K, V][32 keys][32]
  __shared__ __attribute__((aligned(16))) T kv_lds[kGroups * 2 * 32 * 32];
  // the workgroup's bias region, identity-MFMA fragments of its 32 keys for
  // every query tile: [query tile][chunk c][64 lanes][8], loaded once per part
  __shared__ __attribute__((aligned(16))) T bias_lds[NS * kRowWaves * 2 * 64 * 8];
  // keep bytes of the 32 keys of the groups in flight, per lane (lanes 32..63
  // repeat 0..31): [group][64]
  __shared__ uint32_t keep_lds[kGroups][64];

  const int tid = threadIdx.x;
  // (readfirstlane: the wave index, and everything derived from it, is
  // wave-uniform and lives in scalar registers, e.g. the LDS base of the
  // direct-to-LDS loads, which must be a scalar)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rs = wave / RW;  // group (of the rows in flight) this wave works on
  const int wq = wave % RW;  // its share of the query tiles
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int g2 = lane >> 5;

  // LDS byte addresses (M0 of the direct-to-LDS loads): this wave's ring
  // stage 0 (stage s adds s * kStageStride), its K/V rows, its keep bytes
  constexpr uint32_t kStageStride = kFusedWaves * sizeof(RingStage);
  const uint32_t ring_m0 = lds_addr(&ring_lds[0][wave]);
  const uint32_t keep_m0 = lds_addr(keep_lds) + (uint32_t)(rs * 64 * 4);
  const uint32_t bias_m0 = lds_addr(bias_lds);

  int64_t tile = xcd_tile(blockIdx.x, gridDim.x, xcd_chunk(a.uniform_tiles));
  if (tile >= a.total_tiles) return;
  const Sample* tab = reinterpret_cast<const Sample*>(a.table);
  const int H = a.num_heads;
  const int s_idx = find_sample(tile, tab, a.num_samples, a.uniform_tiles, [&](const Sample& s) {
    // (a split batch: only the samples this kernel serves)
    const bool mine = (a.fused_max_lq == 0 || s.Lq <= a.fused_max_lq) && s.Lq > a.fused_min_lq;
    return mine ? (int64_t)H * cdiv(s.Lk, 32) * parts_for(s.G, a.part_groups, a.parts) : (int64_t)0;
  });
  if (s_idx < 0) return;
  const Sample& S = tab[__builtin_amdgcn_readfirstlane(s_idx)];
  // every table field the loop needs, read once into (scalar) registers: the
  // barriers are compiler memory fences, after which fields read through S
  // would be fetched from global memory again
  auto u64 = [](int64_t x) { return (int64_t)uniform64((uint64_t)x); };
  auto uptr = [](auto* p) { return reinterpret_cast<decltype(p)>(uniform64(reinterpret_cast<uint64_t>(p))); };
  const int64_t G = u64(S.G);
  const int P = parts_for(G, a.part_groups, a.parts);
  const int Lq = __builtin_amdgcn_readfirstlane((int)S.Lq), Lk = __builtin_amdgcn_readfirstlane((int)S.Lk);
  const int nkb = (int)cdiv(Lk, 32);
  // logical order (head, part, key block): the key blocks of one (head, part)
  // read the same Q / dO rows and run next to each other on one XCD
  // (launch grids stay below 2^31 workgroups: 32-bit division)
  const int kb = (int)((uint32_t)tile % (uint32_t)nkb);
  const uint32_t rest = (uint32_t)tile / (uint32_t)nkb;
  const int part = (int)(rest % (uint32_t)P);
  const int h = (int)(rest / (uint32_t)P);
  const int g_begin = __builtin_amdgcn_readfirstlane((int)(G * part / P));
  const int g_end = __builtin_amdgcn_readfirstlane((int)(G * (part + 1) / P));
  const int D = a.head_size;
  const int nqt = (Lq + 31) >> 5;  // <= NS * 4 (the launch picks NS for the longest sample)
  const float c1 = a.scale * kLog2e;
  const int key = kb * 32 + lq;  // this lane's key
  const bool has_mask = MASKED && a.mask != nullptr && S.m_off >= 0;

  // Q and dO rows come from the dQ kernel's compact copies: row
  // l_off + (g H + h) Lq + q of kCompactRow elements
  const int64_t row_h = S.l_off + (int64_t)h * Lq;
  const T* const q_h = uptr(a.qc + row_h * kCompactRow);
  const T* const do_h = uptr(a.dc + row_h * kCompactRow);
  const int64_t q_sg = (int64_t)H * Lq * kCompactRow, do_sg = q_sg;
  // the (g, h) row of the dQ kernel's pack: -LSE / c of the Lq queries, then -delta
  const float* const pk_h = uptr(a.ld_pack + 2 * row_h);
  const int64_t pk_sg = 2 * (int64_t)H * Lq;
  const uint8_t* const m_h = has_mask ? uptr(a.mask + S.m_off) : nullptr;
  const int64_t m_sg = has_mask ? u64(S.m_sg) : 0;

  // ---- per-lane DMA offsets (bytes) of the Q / dO tile rows of step 0
  // (query tile wq) within the (g, h) block of the compact copies, which are
  // the same for Q and dO; step i (query tile RW i + wq) adds i kStepQD.
  // Load r (0, 1) of a tile covers rows 16 r .. 16 r + 15; lane l writes
  // slot l = row 16 r + l / 4, physical chunk l % 4, which holds logical
  // chunk (l % 4) ^ swz(row).  Rows past Lq fall past the block's range and
  // chunks past D get an offset past every range: they read 0.
  constexpr uint32_t kStepQD = (uint32_t)(kRowWaves * 32 * kCompactRow * 2);
  uint32_t tile_off0[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int row = 16 * r + (lane >> 2);
    const int col = ((lane & 3) ^ swz<32>(row)) * 8;
    tile_off0[r] = col < D ? (uint32_t)(((wq * 32 + row) * kCompactRow + col) * 2) : kOut;
  }
  // pack offsets of step i: lane l reads query (RW i + wq) * 32 + ld_q,
  // lanes 32..63 from the -delta half, so that ring position l holds the
  // query the accumulator layout puts there (ld_q inverts perm32); a query
  // past Lq gets 2^31 added (out of range: it reads 0)
  const int ld_q0 = wq * 32 + kappa(lq >> 4, lq & 15);
  // K/V block DMA of a group: its four loads (K rows 0..15, K rows 16..31, V
  // rows 0..15, V rows 16..31) spread over the group's waves, load u = (kKvLoads
  // wq + j) % 4 (with eight waves per group, waves 4..7 load the same bytes as
  // waves 0..3)
  uint32_t kv_m0[kKvLoads], kv_lane_off[kKvLoads], kv_bytes[kKvLoads];
  int64_t kv_sg[kKvLoads];
  const T* kv_h[kKvLoads];
#pragma unroll
  for (int j = 0; j < kKvLoads; ++j) {
    const int u = (kKvLoads * wq + j) & 3;
    const int t = u >> 1;
    const int row = 16 * (u & 1) + (lane >> 2);
    const int col = (lane & 3) * 8;
    kv_m0[j] = lds_addr(kv_lds) + (uint32_t)(((rs * 2 + t) * 32 * 32 + 16 * (u & 1) * 32) * sizeof(T));
    const int64_t si = u64(t ? S.v_si : S.k_si);
    kv_sg[j] = u64(t ? S.v_sg : S.k_sg);
    kv_h[j] = uptr(t ? a.v + S.v_off + h * S.v_sh : a.k + S.k_off + h * S.k_sh);
    kv_bytes[j] = (uint32_t)(((int64_t)(Lk - 1) * si + D) * 2);
    const int key_ = kb * 32 + row;
    kv_lane_off[j] = key_ < Lk && col < D ? (uint32_t)((key_ * si + col) * 2) : kOut;
  }
  // bias fragments (A operand, lane = query): the fragment-major copy of the
  // shared bias; the 1 KB block of (query tile, chunk c) sits at a uniform offset
  const bool bf_in = kb < a.bf_nkt;
  const u32x4 b_rsrc =
      rsrc_words(a.bias_frag + s_idx * a.bf_sample_stride + (int64_t)h * a.bf_nqt * a.bf_nkt * 1024 +
                    (bf_in ? kb : 0) * 1024,
                bf_in ? (uint32_t)(((int64_t)a.bf_nqt * a.bf_nkt - kb) * 2048) : 0u);
  const uint32_t b_lane = (uint32_t)lane * 16;
  const int bf_step = a.bf_nkt * 2 * 1024;  // bytes per query tile
  float* const db_col = (P == 1 ? a.dbias : a.dbias_part + (int64_t)part * a.dbias_extent) + S.db_off +
                        h * S.db_sh + key;
  const int64_t db_si = S.db_si;

  Frag ident[2];
  identity_frags<T>(ident, 1.0f / a.scale, lane);
  const TrLane trl = tr_lane<32>(lane, 0);

  // The resources of group g's (g, h) blocks of the compact Q and dO copies
  // and of the pack, built once per group (the loads of a step differ only in
  // their per-lane offsets); a group past the part gets empty ranges (reads 0)
  struct GroupDesc {
    u32x4 q, d, pk;
  };
  const uint32_t qd_bytes = (uint32_t)(((Lq - 1) * kCompactRow + D) * 2);
  auto group_desc = [&](int g) {
    const bool live = g < g_end;
    const int64_t gg = live ? g : g_begin;
    GroupDesc gd;
    gd.q = rsrc_words(q_h + gg * q_sg, live ? qd_bytes : 0u);
    gd.d = rsrc_words(do_h + gg * do_sg, live ? qd_bytes : 0u);
    gd.pk = rsrc_words(pk_h + gg * pk_sg, live ? (uint32_t)(Lq * 8) : 0u);
    return gd;
  };
  // stage (the group of gd, step i: query tile 4 i + wq) into ring stage st
  // of this wave: the pack (1 load) and the Q / dO tiles (4); every stage
  // issues all five
  auto dma_stage = [&](const GroupDesc& gd, auto ic, int st) {
    constexpr int i = decltype(ic)::value;
    const uint32_t m0 = ring_m0 + (uint32_t)st * kStageStride;
    const int q = ld_q0 + kRowWaves * 32 * i;
    dma4_m0(gd.pk, m0 + offsetof(RingStage, ld), (uint32_t)((q + g2 * Lq) * 4) | ((uint32_t)(q >= Lq) << 31));
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t off = tile_off0[r] + (uint32_t)i * kStepQD;
      dma16_m0(gd.q, m0 + offsetof(RingStage, q) + 16 * r * 32 * 2, off);
      dma16_m0(gd.d, m0 + offsetof(RingStage, d) + 16 * r * 32 * 2, off);
    }
  };
  // K/V block of this wave's group g into its slot of kv_lds (kKvLoads DMA loads)
  auto dma_kv = [&](int g) {
    const bool live = g < g_end;
    const int64_t gg = live ? g : g_begin;
#pragma unroll
    for (int j = 0; j < kKvLoads; ++j) {
      const u32x4 r = rsrc_words(kv_h[j] + gg * kv_sg[j], live ? kv_bytes[j] : 0u);
      dma16_m0(r, kv_m0[j], kv_lane_off[j]);
    }
  };
  // keep bytes of group g's keys into keep_lds[rs] (one load)
  auto dma_keep = [&](int g) {
    const bool live = g < g_end;
    const int64_t gg = live ? g : g_begin;
    const u32x4 r = rsrc_words(has_mask ? m_h + gg * m_sg : nullptr, has_mask && live ? (uint32_t)Lk : 0u);
    dma_u8_m0(r, keep_m0, (uint32_t)key);
  };
  // whether key kb * 32 + k of this wave's group g is attended (its keep bytes have landed)
  auto kv_keep = [&](int g, int k) {
    return g < g_end && kb * 32 + k < Lk && (!has_mask || keep_lds[rs][k] != 0);
  };

  // Row end: each group's waves' dK (then dV) partials are summed through
  // LDS and stored.  The reader threads of a group are its own waves (with
  // eight waves per group, the first four); item t of them owns dims 4 red_q
  // .. 4 red_q + 3 of key red_key (red_q = 2 c + g2 for chunk c and lane half
  // g2 of the accumulator layout), so eight consecutive lanes write one whole
  // 64-byte key row: scattered 4-byte stores into rows 196 KB apart (the
  // ending-node layout) cost the kernel a third of its time.  256 items per
  // group: one per thread, two with two waves per group.
  int red_key[kItems], red_src[kItems];
  bool red_live[kItems];
  int64_t red_k[kItems], red_v[kItems];
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int red_t = tid % (kRowWaves * 64) + it * kRowWaves * 64;
    red_key[it] = (red_t >> 3) & 31;
    const int red_q = red_t & 7, red_c = red_q >> 1, red_g = red_q & 1;
    const int red_gkey = kb * 32 + red_key[it];
    red_live[it] = red_gkey < Lk && 4 * red_q < D;
    red_k[it] = S.k_off + h * S.k_sh + (int64_t)red_gkey * S.k_si + 4 * red_q;
    red_v[it] = S.v_off + h * S.v_sh + (int64_t)red_gkey * S.v_si + 4 * red_q;
    // (see the layout of the partials below)
    red_src[it] = 64 * red_c + ((red_key[it] + 32 * red_g) ^ (4 * red_c));
  }
  const int64_t k_sg = S.k_sg, v_sg = S.v_sg;
  constexpr int kStageF4 = (int)(sizeof(RingStage) / 16);
  static_assert(sizeof(RingStage) % 16 == 0 && 16 * 64 <= 4 * kStageF4, "a wave's partials fit its ring stage");
  // one tensor's partials (acc) -> each wave's ring stage `slot` (read
  // already), barrier, the fixed-order sum of the group's four partials by
  // its waves, scaled, stored; barrier (partials read before that LDS is
  // written again).  Lane L's registers 4 c .. 4 c + 3 (dims 8 c + 4 g2
  // .. + 3 of its key) sit at float4 64 c + (L ^ 4 c) of its wave's block:
  // the writes of a wave are a permutation of consecutive 16-byte slots, and
  // the reads of eight consecutive lanes (one key, four c, two g2) fall into
  // four bank groups, two lanes each.
  // (a masked key's rows are written as zeros; a dead group writes nothing)
  auto reduce_store = [&](int slot, const f32x16& acc, T* dst, const int64_t (&off)[kItems], int64_t goff, float sc,
                          bool live, const bool (&ok)[kItems]) {
    float4* const red = reinterpret_cast<float4*>(&ring_lds[slot][0]);
    float4* const rw = red + wave * kStageF4;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      rw[64 * c + (lane ^ (4 * c))] = make_float4(acc[4 * c], acc[4 * c + 1], acc[4 * c + 2], acc[4 * c + 3]);
    __syncthreads();
    if (RW != 8 || wq < 4) {
#pragma unroll
      for (int it = 0; it < kItems; ++it) {
        const float4* src = red + kRowWaves * rs * kStageF4 + red_src[it];
        float4 o = src[0];
#pragma unroll
        for (int w = 1; w < kRowWaves; ++w) {
          const float4 x = src[w * kStageF4];
          o.x += x.x;
          o.y += x.y;
          o.z += x.z;
          o.w += x.w;
        }
        if (dst != nullptr && red_live[it] && live) {
          const float f = ok[it] ? sc : 0.0f;
          *reinterpret_cast<uint2*>(dst + off[it] + goff) =
              make_uint2(pack2<T>(o.x * f, o.y * f), pack2<T>(o.z * f, o.w * f));
        }
      }
    }
    __syncthreads();
  };

  float region[NS][16];
#pragma unroll
  for (int i = 0; i < NS; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) region[i][j] = 0.0f;
  f32x16 dk = f32x16{}, dv = f32x16{};
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;

  // ---- prologue: K/V and keep bytes of the first rows, the first NST - 1
  // stages, the bias region
  dma_kv(g_begin + rs);
  if constexpr (MASKED) dma_keep(g_begin + rs);
  // (gd: the resources of the group whose stage was issued last)
  GroupDesc gd = group_desc(g_begin + rs);
  dma_stage(gd, I0{}, 0);
  if constexpr (NST == 3) {
    if constexpr (NS == 1) {
      gd = group_desc(g_begin + kGroups + rs);
      dma_stage(gd, I0{}, 1);
    } else {
      dma_stage(gd, I1{}, 1);
    }
  }
  // the bias region: wave w loads query tiles RW i + w % RW (both chunks;
  // with two groups, the groups' waves write the same bytes); query tiles
  // past Lq, which ghost steps read, are zeros
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int qt = kRowWaves * i + wq;
    const bool in = qt < nqt && qt < a.bf_nqt;
#pragma unroll
    for (int c = 0; c < 2; ++c)
      dma16_m0(b_rsrc, bias_m0 + (uint32_t)((qt * 2 + c) * 64 * 8 * sizeof(T)),
               in ? b_lane + (uint32_t)(qt * bf_step + c * 1024) : kOut);
  }
  wait_vm<0>();
  __syncthreads();

  // Loads per step, in issue order: [at a row's first step: the next rows'
  // K/V block and keep bytes (1 + MASKED)], the pack (1), the Q/dO tiles
  // (4), all for the stage NST - 1 ahead.  A step first waits for its own
  // stage, issued NST - 1 steps earlier: everything issued after it (with
  // three stages, the previous step's loads) may still be in flight.
  constexpr int kPerStep = 5;
  constexpr int kGroupLoads = kKvLoads + (MASKED ? 1 : 0);
  int slot = 0;  // ring slot of the stage being computed (the step index mod NST when NST divides NS)
  constexpr bool kFixedSlots = NS % NST == 0;
  for (int gp = g_begin; gp < g_end; gp += kGroups) {
    const int g = gp + rs;  // this wave's group (past g_end: a dead group, all zeros, nothing stored)
    const bool g_live = g < g_end;
    // this group's K / V fragments (B operand: lane = key, 8 consecutive d),
    // its keep bits, and those of the key whose dK / dV this thread stores
    Frag kf[2], vf[2];
    const bool kvalid = MASKED ? kv_keep(g, lq) : true;
    const bool wave_masked = MASKED && __any(!kvalid);
    bool red_ok[kItems];
#pragma unroll
    for (int it = 0; it < kItems; ++it) red_ok[it] = MASKED ? kv_keep(g, red_key[it]) : true;
    {
      const T* kb_ = kv_lds + (rs * 2) * 32 * 32 + lq * 32;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        kf[s] = lds_frag<T>(kb_ + 16 * s + 8 * g2);
        vf[s] = lds_frag<T>(kb_ + 32 * 32 + 16 * s + 8 * g2);
        if (MASKED && !kvalid) {
          kf[s] = Frag{};
          vf[s] = Frag{};
        }
      }
    }
    // every wave has its K / V in registers and its keep bits: the next
    // pair's loads (issued at this pair's first step) may overwrite them
    __syncthreads();

    // one step: query tile 4 i + wq of group g (straight-line code per
    // step; the scheduling barriers keep each step's temporaries within it,
    // the register budget being 256 per lane at two waves per SIMD)
    auto step = [&](auto ic) {
      constexpr int i = decltype(ic)::value;
      __builtin_amdgcn_sched_barrier(0);
      // (three stages: the previous step was a row's first when i == 1, and issued the rows' loads too;
      // two stages: the step's own stage was the last load issued)
      if constexpr (NST == 2) wait_vm<0>();
      else if constexpr (i == 1 || NS == 1) wait_vm<kPerStep + kGroupLoads>();
      else wait_vm<kPerStep>();
      const int cs = kFixedSlots ? i % NST : slot;
      const RingStage& cur = ring_lds[cs][wave];
      if constexpr (i == 0) {
        dma_kv(gp + kGroups + rs);
        if constexpr (MASKED) dma_keep(gp + kGroups + rs);
      }
      {
        constexpr int ahead = i + NST - 1;
        const int as = kFixedSlots ? ahead % NST : (NST == 3 ? (slot == 0 ? 2 : slot - 1) : 1 - slot);
        // the first stage of a group: that group's resources
        if constexpr (ahead % NS == 0) gd = group_desc(gp + kGroups * (ahead / NS) + rs);
        dma_stage(gd, std::integral_constant<int, ahead % NS>{}, as);
      }

      // ---- compute this stage, unless its query tile is past Lq (a ghost step of a shorter sample) or
      // its group is dead: its zero Q, dO, pack and bias contribute nothing.  Wave-uniform; the loads above
      // run either way, so the wait counts stay the same, and the other wave on the SIMD runs alone meanwhile
      if (i * kRowWaves + wq < nqt && g_live) {
      const T* qt_ = reinterpret_cast<const T*>(cur.q);
      const T* dt_ = reinterpret_cast<const T*>(cur.d);
      f32x16 sacc = *reinterpret_cast<const f32x16*>(&cur.ld[g2 * 16]);
      {
        const T* bq = bias_lds + (i * kRowWaves + wq) * 2 * 64 * 8 + lane * 8;
        sacc = E::mma(lds_frag<T>(bq), ident[0], sacc);
        sacc = E::mma(lds_frag<T>(bq + 64 * 8), ident[1], sacc);
      }
      f32x16 pacc = *reinterpret_cast<const f32x16*>(&cur.ld[32 + g2 * 16]);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        sacc = E::mma(lds_frag<T>(qt_ + swz_off<32>(lq, s * 16 + g2 * 8)), kf[s], sacc);
        pacc = E::mma(lds_frag<T>(dt_ + swz_off<32>(lq, s * 16 + g2 * 8)), vf[s], pacc);
      }
      // two halves of 8 scores: each half's P and dS feed their MFMAs at once
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        float p[8], ds[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = 8 * m + e;
          p[e] = __builtin_amdgcn_exp2f(sacc[j] * c1);
          if (MASKED && wave_masked) p[e] = kvalid ? p[e] : 0.0f;
          ds[e] = p[e] * pacc[j];
          region[i][j] += ds[e];
        }
        const Frag pf = pack8<T>(p);
        const Frag sf = pack8<T>(ds);
        const int at = (16 * m) * 32;
        dv = E::mma(lds_read_tr_frag_sw<T>(dt_ + at, trl), pf, dv);
        dk = E::mma(lds_read_tr_frag_sw<T>(qt_ + at, trl), sf, dk);
      }
      }
      if constexpr (!kFixedSlots) slot = slot == NST - 1 ? 0 : slot + 1;
    };
    step(I0{});
    if constexpr (NS > 1) step(I1{});
    if constexpr (NS > 2) step(std::integral_constant<int, 2>{});
    if constexpr (NS > 3) step(std::integral_constant<int, 3>{});
    if constexpr (NS > 4) step(std::integral_constant<int, 4>{});
    if constexpr (NS > 5) step(std::integral_constant<int, 5>{});
    __builtin_amdgcn_sched_barrier(0);

    // ---- pair end: the next pair's K/V blocks and keep bytes have landed
    // (issued at this pair's first step, followed by kPerStep loads per
    // step); each group's dK and dV partials are summed and stored through
    // the ring stage the last step read
    wait_vm<NS * kPerStep>();
    const int red_slot = kFixedSlots ? (NS - 1) % NST : (NST == 3 ? (slot == 0 ? 2 : slot - 1) : 1 - slot);
    reduce_store(red_slot, dk, a.dk, red_k, (int64_t)g * k_sg, a.scale, g_live, red_ok);
    reduce_store(red_slot, dv, a.dv, red_v, (int64_t)g * v_sg, 1.0f, g_live, red_ok);
    dk = f32x16{};
    dv = f32x16{};
  }

  // ---- the part's dBias slab; region[i] holds queries (RW i + wq) * 32 +
  // kappa(g2, j) of this lane's key.  With several groups, wave wq of every
  // group holds the same query tiles (its group's share of the part's sum):
  // the other groups' regions go through LDS (the ring, idle once its loads
  // have drained) to the first group's waves, one group at a time in a fixed
  // order, which add them and store
  if constexpr (kGroups > 1) {
    wait_vm<0>();
    float* const xr = reinterpret_cast<float*>(&ring_lds[0][0]) + (wq * NS * 16) * 64 + lane;
    static_assert(kRowWaves * NS * 16 * 64 * 4 <= sizeof(RingStage) * NST * kFusedWaves, "regions fit the ring");
#pragma unroll 1
    for (int r = 1; r < kGroups; ++r) {
      __syncthreads();
      if (rs == r) {
#pragma unroll
        for (int i = 0; i < NS; ++i)
#pragma unroll
          for (int j = 0; j < 16; ++j) xr[(i * 16 + j) * 64] = region[i][j];
      }
      __syncthreads();
      if (rs == 0) {
#pragma unroll
        for (int i = 0; i < NS; ++i)
#pragma unroll
          for (int j = 0; j < 16; ++j) region[i][j] += xr[(i * 16 + j) * 64];
      }
    }
  }
  if (rs == 0 && key < Lk) {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int q0 = (kRowWaves * i + wq) * 32;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int q = q0 + kappa(g2, j);
        if (q < Lq) db_col[(int64_t)q * db_si] = region[i][j];
      }
    }
  }
}

}  // namespace

bool dkvb_fused_ok(const oops_attn_geometry& geo, const Plan& plan) {
  return geo.force_generic == 0 && fast_path_ok(geo, plan) && plan.dp == kCompactRow && plan.all_shared &&
         plan.bias_frag && plan.fused_max_len_q <= kFusedMaxLen && (plan.fused_tiles > 0 || plan.fused_long_tiles > 0);
}

hipError_t launch_dkvb_fused(const oops_attn_geometry& geo, const Plan& plan, const BwdLaunch& L,
                             hipStream_t stream) {
  auto go = [&](auto tag) {
    using T = typename decltype(tag)::type;
    BwdArgsT<T, T> a;
    fill_bwd_args(a, geo, plan, L);
    a.parts = plan.fused_parts;
    a.part_groups = plan.fused_part_groups;
    auto run = [&](auto masked, auto nsc, auto rwc, int64_t tiles, int64_t uniform) {
      a.uniform_tiles = uniform;
      a.total_tiles = tiles;
      const dim3 grid((unsigned)xcd_grid(tiles, xcd_chunk(uniform)));
      hipLaunchKernelGGL(
          (attn_dkvb_fast_kernel<T, decltype(masked)::value, decltype(nsc)::value, decltype(rwc)::value>), grid,
          dim3(512), 0, stream, a);
    };
    using RW2 = std::integral_constant<int, 2>;
    using RW4 = std::integral_constant<int, 4>;
    auto by_ns = [&](auto masked) {
      // the samples up to kFusedMaxLen: query tiles per wave and group, that of the longest sample it
      // serves; two waves per row (four rows in flight, a quarter of the per-row dK/dV sums per step)
      // from 129 to 384 queries, four waves per row otherwise
      if (plan.fused_tiles > 0) {
        a.fused_max_lq = plan.fused_split || plan.fused_long_tiles > 0 ? kFusedMaxLen : 0;
        a.fused_min_lq = 0;
        const int64_t t = plan.fused_tiles, u = plan.fused_uniform;
        const int64_t lq = plan.fused_max_len_q;
        const int ns2 = (int)((lq + 32 * 2 - 1) / (32 * 2));
        const int ns = (int)((lq + 32 * 4 - 1) / (32 * 4));
        if (lq > 128 && lq <= 384) {
          if (ns2 == 3) run(masked, std::integral_constant<int, 3>{}, RW2{}, t, u);
          else if (ns2 == 4) run(masked, std::integral_constant<int, 4>{}, RW2{}, t, u);
          else if (ns2 == 5) run(masked, std::integral_constant<int, 5>{}, RW2{}, t, u);
          else run(masked, std::integral_constant<int, 6>{}, RW2{}, t, u);
        } else if (ns == 1) run(masked, std::integral_constant<int, 1>{}, RW4{}, t, u);
        else if (ns == 2) run(masked, std::integral_constant<int, 2>{}, RW4{}, t, u);
        else if (ns == 3) run(masked, std::integral_constant<int, 3>{}, RW4{}, t, u);
        else if (ns == 4) run(masked, std::integral_constant<int, 4>{}, RW4{}, t, u);
        else if (ns == 5) run(masked, std::integral_constant<int, 5>{}, RW4{}, t, u);
        else run(masked, std::integral_constant<int, 6>{}, RW4{}, t, u);
      }
      // eight waves per row, four query tiles per wave: the samples with kFusedMaxLen < Lq <= kFusedLongMaxLen
      if (plan.fused_long_tiles > 0) {
        a.fused_max_lq = kFusedLongMaxLen;
        a.fused_min_lq = kFusedMaxLen;
        run(masked, std::integral_constant<int, 4>{}, std::integral_constant<int, 8>{}, plan.fused_long_tiles,
            plan.fused_long_uniform);
      }
    };
    if (geo.has_mask) by_ns(std::true_type{});
    else by_ns(std::false_type{});
    return hipGetLastError();
  };
  return geo.dtype == OOPS_BF16 ? go(Tag<__bf16>{}) : go(Tag<_Float16>{});
}

}  // namespace oops
