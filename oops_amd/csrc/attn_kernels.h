// Kernel argument blocks and the instantiated (dtype, bias dtype, padded
// head size) configurations.
#pragma once

#include "attn_common.h"

namespace oops {

template <typename T, typename BT>
struct FwdArgsT {
  const T* q;
  const T* k;
  const T* v;
  const BT* bias;
  const uint8_t* mask;
  T* out;
  T* out_lo;  // optional: out - round(out), for an exact backward delta
  float* lse;
  const int64_t* table;
  int64_t uniform_tiles;
  int64_t total_tiles;  // logical tiles (the grid may be padded for the XCD order)
  int head_group;       // heads whose rows share a 128-byte line, scheduled together
  int num_samples;
  int num_heads;
  int head_size;
  int vec_ok;
  float scale;
  const T* bias_frag;        // fragment-major copy of the shared biases, or nullptr
  int64_t bf_sample_stride;  // elements per sample in bias_frag
  int bf_nqt, bf_nkt;        // 32-query / 32-key tiles per head in bias_frag
};

// Row length (elements) of the compact Q / dO copies the fast dQ kernel writes
// for the fused dK/dV + dBias kernel (head size <= 32).
constexpr int kCompactRow = 32;

template <typename T, typename BT>
struct BwdArgsT {
  const T* q;
  const T* k;
  const T* v;
  const T* out;
  const T* out_lo;
  const T* dout;
  const BT* bias;
  const uint8_t* mask;
  const float* lse;
  float* delta;
  float* ld_pack;  // per (g, h) row: -LSE / c of its Lq queries, then -delta (fused dK/dV + dBias)
  T* qc;           // compact copies of Q and dO (fused dK/dV + dBias): row (l_off + (g H + h) Lq + q)
  T* dc;           // of kCompactRow elements, d < head_size written
  T* dq;
  T* dk;
  T* dv;
  float* dbias;        // final dBias (f32)
  float* dbias_part;   // [parts][dbias_extent] partial slabs (shared-bias mode)
  const int64_t* table;
  int64_t uniform_tiles;
  int64_t total_tiles;  // logical tiles of the launch (fast paths; grid padded to 8)
  int64_t dbias_extent;
  int num_samples;
  int num_heads;
  int head_size;
  int vec_ok;
  int parts;
  int64_t part_groups;  // > 0: per-sample parts, parts_for(G, part_groups, parts) (fast dBias)
  // > 0: a batch split between the fused dK/dV + dBias kernel (samples with Lq <= fused_max_lq) and the
  // separate dK/dV and dBias kernels (the longer ones); each kernel skips the other's samples, and the dBias
  // reduction takes a longer sample's parts from parts_rest / part_groups_rest
  int fused_max_lq;
  int fused_min_lq;  // the fused kernel's eight-wave launch: only samples with Lq > fused_min_lq
  int parts_rest;
  int64_t part_groups_rest;
  int head_group;
  float scale;
  const T* bias_frag;        // as in FwdArgsT
  int64_t bf_sample_stride;
  int bf_nqt, bf_nkt;
  int delta_in_dq;           // fast dQ kernel computes delta (and stores it) instead of reading it
};

}  // namespace oops

// The kernels name their argument block FwdArgs / BwdArgs; each kernel
// template defines them for its own (T, BT).
#define FwdArgs FwdArgsT<T, BT>
#define BwdArgs BwdArgsT<T, BT>

#define OOPS_FOR_EACH_DP(X, T, BT) X(T, BT, 32) X(T, BT, 64) X(T, BT, 128) X(T, BT, 256)
#define OOPS_FOR_EACH_CONFIG(X)           \
  OOPS_FOR_EACH_DP(X, float, float)       \
  OOPS_FOR_EACH_DP(X, __bf16, __bf16)     \
  OOPS_FOR_EACH_DP(X, __bf16, float)      \
  OOPS_FOR_EACH_DP(X, _Float16, _Float16) \
  OOPS_FOR_EACH_DP(X, _Float16, float)

#include <type_traits>

namespace oops {

template <typename T>
struct Tag {
  using type = T;
};

// Call f(Tag<T>, Tag<BT>, integral_constant<DP>) for the instantiated
// configuration; returns false when the combination is not built.
template <typename F>
inline bool dispatch_config(int dtype, int bias_dtype, int dp, F&& f) {
  auto by_dp = [&](auto t, auto bt) {
    switch (dp) {
      case 32: f(t, bt, std::integral_constant<int, 32>{}); return true;
      case 64: f(t, bt, std::integral_constant<int, 64>{}); return true;
      case 128: f(t, bt, std::integral_constant<int, 128>{}); return true;
      case 256: f(t, bt, std::integral_constant<int, 256>{}); return true;
    }
    return false;
  };
  if (dtype == OOPS_F32) return bias_dtype == OOPS_F32 && by_dp(Tag<float>{}, Tag<float>{});
  if (dtype == OOPS_BF16) {
    if (bias_dtype == OOPS_BF16) return by_dp(Tag<__bf16>{}, Tag<__bf16>{});
    if (bias_dtype == OOPS_F32) return by_dp(Tag<__bf16>{}, Tag<float>{});
    return false;
  }
  if (dtype == OOPS_F16) {
    if (bias_dtype == OOPS_F16) return by_dp(Tag<_Float16>{}, Tag<_Float16>{});
    if (bias_dtype == OOPS_F32) return by_dp(Tag<_Float16>{}, Tag<float>{});
    return false;
  }
  return false;
}

// longest sample (Lq) the fused dK/dV + dBias kernel serves: 8 waves x 3 query tiles of 32
constexpr int kFusedMaxLen = 768;       // fused dK/dV + dBias, four waves per row
constexpr int kFusedLongMaxLen = 1024;  // fused dK/dV + dBias, eight waves per row (longer samples)

// Host-side launch plan derived from the geometry table.
struct Plan {
  int dp = 0;
  int64_t fwd_tiles = 0, fwd_uniform = 0;        // 128-query blocks
  int64_t delta_tiles = 0, delta_uniform = 0;    // 64-query blocks
  int64_t dkv_tiles = 0, dkv_uniform = 0;        // 128-key blocks
  int64_t dkv_tiles_r2 = 0, dkv_uniform_r2 = 0;  // same, two groups per block
  int64_t sbias_tiles = 0, sbias_uniform = 0;    // shared dBias blocks (incl. parts)
  int64_t sred_tiles = 0, sred_uniform = 0;      // shared dBias reduction blocks
  int64_t lse_extent = 0;                        // floats
  int64_t dbias_extent = 0;                      // floats
  int parts = 1;                                 // group ranges of the shared dBias reduction
  int64_t fast_sbias_tiles = 0, fast_sbias_uniform = 0;  // same, 64-key blocks (fast path)
  int fast_parts = 1;                            // largest per-sample part count (fast path)
  int64_t fast_part_groups = 1;                  // groups per part the fast path aims at
  bool any_full = false, any_shared = false;
  bool all_shared = false;                       // every sample has a row-shared bias
  // fused dK/dV + shared dBias kernel (attn_bwd_fused.hip): 32-key blocks x group ranges
  int64_t fused_tiles = 0, fused_uniform = 0;
  bool fused_ok = false;  // the fused dK/dV + dBias kernel serves this geometry (sizes its workspace)
  int fused_parts = 1;
  int64_t fused_part_groups = 1;
  int64_t fused_max_len_q = 0;                   // longest sample the fused kernel's four-wave launch serves
  int64_t fused_long_tiles = 0;                  // its eight-wave launch: samples with kFusedMaxLen < Lq <= kFusedLongMaxLen
  int64_t fused_long_uniform = 0;
  bool fused_split = false;                      // some samples too long for it: separate kernels for those
  int64_t dkv_rest_tiles = 0, fast_sbias_rest_tiles = 0;  // the separate kernels' tiles of those samples
  bool any_pair_mask = false;                    // a mask that depends on the query
  bool masked_tiles = false;                     // some 64-key tile has masked or out-of-range keys
  bool offsets_32bit = true;                     // every per-(group, head) K/V/bias block < 2 GiB
  int64_t max_len_q = 0, max_len_k = 0;
  // fragment-major copy of the shared biases for the fast kernels (see attn_bias_frag_kernel)
  bool bias_frag = false;
  int bf_nqt = 0, bf_nkt = 0;   // 32-query / 32-key tiles per head (max over samples)
  int64_t bf_sample_stride = 0; // elements per sample
  size_t bf_bytes = 0;
};

// True when the 16-bit fast kernels serve this geometry (forward and backward).
bool fast_path_ok(const oops_attn_geometry& geo, const Plan& plan);
// key masks may be folded into the bias fragments (every sample's keys fit the fold table)
bool fold_masks_ok(const Plan& plan);

// Writes the fragment-major copy of every shared bias of the table into bf
// (plan.bf_bytes bytes); see attn_bias_frag_kernel.
hipError_t launch_bias_frag(const oops_attn_geometry& geo, const Plan& plan, const void* bias, void* bf,
                            hipStream_t stream);

// Fast paths (16-bit, head size <= 64); return false when the geometry is not covered.
bool launch_forward_fast(const oops_attn_geometry& geo, const Plan& plan, const void* q, const void* k,
                         const void* v, const uint8_t* mask, const void* bias, const void* bias_frag, void* out,
                         void* out_lo, float* lse, hipStream_t stream, hipError_t* err);

// bias_frag: plan.bf_bytes of device memory when plan.bias_frag (the copy is written here), else unused
hipError_t launch_forward(const oops_attn_geometry& geo, const Plan& plan, const void* q, const void* k,
                          const void* v, const uint8_t* mask, const void* bias, void* bias_frag, void* out,
                          void* out_lo, float* lse, hipStream_t stream);

// Device pointers of one backward call.
struct BwdLaunch {
  const void *q, *k, *v, *out, *out_lo, *dout, *bias;
  const uint8_t* mask;
  const float* lse;
  float* delta;
  float* ld_pack;  // written by the fast dQ kernel when non-null, read by the fused dK/dV + dBias kernel
  void *qc, *dc;   // likewise: compact Q and dO
  void *dq, *dk, *dv;
  float *dbias, *dbias_part;
  const void* bias_frag;  // fragment-major shared biases (fast kernels), or nullptr
};

int head_group_of(const oops_attn_geometry& geo);

template <typename T, typename BT>
inline void fill_bwd_args(BwdArgsT<T, BT>& a, const oops_attn_geometry& geo, const Plan& plan, const BwdLaunch& L) {
  a.q = static_cast<const T*>(L.q);
  a.k = static_cast<const T*>(L.k);
  a.v = static_cast<const T*>(L.v);
  a.out = static_cast<const T*>(L.out);
  a.out_lo = static_cast<const T*>(L.out_lo);
  a.dout = static_cast<const T*>(L.dout);
  a.bias = geo.has_bias ? static_cast<const BT*>(L.bias) : nullptr;
  a.mask = geo.has_mask ? L.mask : nullptr;
  a.lse = L.lse;
  a.delta = L.delta;
  a.ld_pack = L.ld_pack;
  a.qc = static_cast<T*>(L.qc);
  a.dc = static_cast<T*>(L.dc);
  a.dq = static_cast<T*>(L.dq);
  a.dk = static_cast<T*>(L.dk);
  a.dv = static_cast<T*>(L.dv);
  a.dbias = geo.has_bias ? L.dbias : nullptr;
  a.dbias_part = L.dbias_part;
  a.table = geo.table_device;
  a.uniform_tiles = 0;
  a.total_tiles = 0;
  a.dbias_extent = plan.dbias_extent;
  a.num_samples = geo.num_samples;
  a.num_heads = geo.num_heads;
  a.head_size = geo.head_size;
  a.vec_ok = geo.vec_ok;
  a.parts = plan.parts;
  a.part_groups = 0;
  a.fused_max_lq = 0;
  a.fused_min_lq = 0;
  a.parts_rest = 1;
  a.part_groups_rest = 0;
  a.head_group = head_group_of(geo);
  a.scale = geo.scale;
  a.bias_frag = static_cast<const T*>(L.bias_frag);
  a.bf_sample_stride = plan.bf_sample_stride;
  a.bf_nqt = plan.bf_nqt;
  a.bf_nkt = plan.bf_nkt;
  a.delta_in_dq = 0;
}

bool backward_fast_ok(const oops_attn_geometry& geo, const Plan& plan);
// rest: only the samples of a split batch that the fused dK/dV + dBias kernel does not serve
hipError_t launch_dkv_fast(const oops_attn_geometry& geo, const Plan& plan, const BwdLaunch& L, hipStream_t stream,
                           bool rest = false);
// delta_in_dq: the kernel computes delta = rowsum((O + O_lo) * dO) itself and stores it for the
// later kernels (no separate delta pass)
hipError_t launch_dq_fast(const oops_attn_geometry& geo, const Plan& plan, const BwdLaunch& L, bool delta_in_dq,
                          hipStream_t stream);
// Fused dK, dV and row-shared dBias (head size <= 32, Lq <= 1024, every sample a shared bias); it
// reads L.ld_pack, L.qc and L.dc, which the fast dQ kernel writes.
bool dkvb_fused_ok(const oops_attn_geometry& geo, const Plan& plan);
hipError_t launch_dkvb_fused(const oops_attn_geometry& geo, const Plan& plan, const BwdLaunch& L,
                             hipStream_t stream);
hipError_t launch_dbias_fast(const oops_attn_geometry& geo, const Plan& plan, const BwdLaunch& L,
                             hipStream_t stream, bool rest = false);

hipError_t launch_backward(const oops_attn_geometry& geo, const Plan& plan, const void* q, const void* k,
                           const void* v, const uint8_t* mask, const void* bias, const void* out,
                           const void* out_lo, const float* lse, const void* dout, void* dq, void* dk, void* dv, float* dbias,
                           float* delta, float* ld_pack, void* qdo_compact, float* dbias_part, void* bias_frag,
                           hipStream_t stream);

}  // namespace oops
