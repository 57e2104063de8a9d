// C entry points: validate the geometry table, derive the launch plan and
// enqueue the kernels.  No device memory is allocated here; the backward
// pass takes a caller-provided workspace.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "attn_kernels.h"
#include "gate_kernels.h"
#include "reduce_kernels.h"
#include "trimul_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, long long a = 0, long long b = 0) {
  char buf[512];
  std::snprintf(buf, sizeof(buf), fmt, a, b);
  g_last_error = buf;
  return code;
}

constexpr int64_t kMaxGrid = (int64_t(1) << 31) - 1;
constexpr int64_t kTargetSharedBiasBlocks = 2048;  // 8 workgroups per CU on 256 CUs
constexpr int kMaxParts = 64;
#ifndef OOPS_MIN_PART_GROUPS
#define OOPS_MIN_PART_GROUPS 32
#endif
// a dBias part shorter than this spends more on its set-up and partial-sum store than on groups
constexpr int64_t kMinPartGroups = OOPS_MIN_PART_GROUPS;
constexpr size_t kMaxBiasFragBytes = size_t(1) << 30;
#ifndef OOPS_FUSED_BLOCKS
#define OOPS_FUSED_BLOCKS 768
#endif
constexpr int64_t kTargetFusedBlocks = OOPS_FUSED_BLOCKS;  // three rounds of one workgroup per CU on 256 CUs
constexpr int64_t kMinFusedPartGroups = 16;

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

int padded_head(int d) {
  if (d <= 32) return 32;
  if (d <= 64) return 64;
  if (d <= 128) return 128;
  return 256;
}

// Highest element index touched (+1) by an operand with the given strides.
int64_t extent(int64_t off, int64_t G, int64_t sg, int64_t H, int64_t sh, int64_t L, int64_t si, int64_t inner) {
  return off + (G - 1) * sg + (H - 1) * sh + (L - 1) * si + inner;
}

// Returns 0 and fills `plan`, or an error code.
int make_plan(const oops_attn_geometry* geo, oops::Plan& plan) {
  using oops::Sample;
  if (geo == nullptr) return fail(OOPS_EINVAL, "geometry is NULL");
  if (geo->table_host == nullptr || geo->table_device == nullptr)
    return fail(OOPS_EINVAL, "geometry table pointers must be set (host and device copies)");
  if (geo->num_samples <= 0) return fail(OOPS_EINVAL, "num_samples must be positive, got %lld", geo->num_samples);
  if (geo->num_heads <= 0) return fail(OOPS_EINVAL, "num_heads must be positive, got %lld", geo->num_heads);
  if (geo->head_size <= 0 || geo->head_size > 256)
    return fail(OOPS_EINVAL, "head_size must be in 1..256, got %lld", geo->head_size);
  if (geo->dtype < OOPS_F32 || geo->dtype > OOPS_F16) return fail(OOPS_EINVAL, "unknown dtype %lld", geo->dtype);
  if (geo->has_bias && geo->bias_dtype != geo->dtype && geo->bias_dtype != OOPS_F32)
    return fail(OOPS_EINVAL, "bias dtype must equal the q/k/v dtype or be float32");
  plan = oops::Plan{};
  plan.dp = padded_head(geo->head_size);
  const int64_t H = geo->num_heads;
  const Sample* tab = reinterpret_cast<const Sample*>(geo->table_host);
  int64_t c_fwd = -1, c_delta = -1, c_dkv = -1, c_sb = -1, c_dkv2 = -1;
  bool u_fwd = true, u_delta = true, u_dkv = true, u_sb = true, u_dkv2 = true;
  int64_t min_shared_groups = INT64_MAX, sbias_base = 0, sbias_base64 = 0, c_sb64 = -1;
  bool u_sb64 = true;
  auto track = [](int64_t c, int64_t& first, bool& uniform) {
    if (first < 0) first = c;
    else if (first != c) uniform = false;
  };
  for (int s = 0; s < geo->num_samples; ++s) {
    const Sample& S = tab[s];
    if (S.G <= 0 || S.Lq <= 0 || S.Lk <= 0)
      return fail(OOPS_EINVAL, "sample %lld has an empty axis (G, Lq or Lk <= 0)", s);
    if (S.Lq > INT32_MAX || S.Lk > INT32_MAX) return fail(OOPS_EINVAL, "sample %lld is too long", s);
    const int64_t q_off_min = std::min({S.q_off, S.k_off, S.v_off, S.o_off, S.do_off});
    if (q_off_min < 0 || S.l_off < 0) return fail(OOPS_EINVAL, "sample %lld has a negative offset", s);
    if (S.q_sg < 0 || S.q_sh < 0 || S.q_si < 0 || S.k_sg < 0 || S.k_sh < 0 || S.k_si < 0 || S.v_sg < 0 ||
        S.v_sh < 0 || S.v_si < 0 || S.o_sg < 0 || S.o_sh < 0 || S.o_si < 0 || S.do_sg < 0 || S.do_sh < 0 ||
        S.do_si < 0)
      return fail(OOPS_EINVAL, "sample %lld has a negative stride", s);
    if (S.bias_mode < OOPS_BIAS_NONE || S.bias_mode > OOPS_BIAS_SHARED)
      return fail(OOPS_EINVAL, "sample %lld has unknown bias mode %lld", s, S.bias_mode);
    if (geo->has_bias && S.b_off >= 0 && S.bias_mode == OOPS_BIAS_SHARED && S.b_sg != 0)
      return fail(OOPS_EINVAL, "sample %lld: a shared bias must have group stride 0", s);
    const int64_t c1 = S.G * H * cdiv(S.Lq, 128);
    const int64_t c2 = S.G * H * cdiv(S.Lq, 64);
    const int64_t c3 = S.G * H * cdiv(S.Lk, 128);
    const int64_t cs = S.bias_mode == OOPS_BIAS_SHARED ? H * cdiv(S.Lq, 128) * cdiv(S.Lk, 32) : 0;
    plan.fwd_tiles += c1;
    plan.delta_tiles += c2;
    plan.dkv_tiles += c3;
    const int64_t c3r2 = cdiv(S.G, 2) * H * cdiv(S.Lk, 128);
    plan.dkv_tiles_r2 += c3r2;
    track(c3r2, c_dkv2, u_dkv2);
    sbias_base += cs;
    const int64_t cs64 = S.bias_mode == OOPS_BIAS_SHARED ? H * cdiv(S.Lq, 128) * cdiv(S.Lk, 64) : 0;
    sbias_base64 += cs64;
    track(cs64, c_sb64, u_sb64);
    track(c1, c_fwd, u_fwd);
    track(c2, c_delta, u_delta);
    track(c3, c_dkv, u_dkv);
    track(cs, c_sb, u_sb);
    plan.lse_extent = std::max(plan.lse_extent, S.l_off + S.G * H * S.Lq);
    plan.max_len_q = std::max(plan.max_len_q, S.Lq);
    plan.max_len_k = std::max(plan.max_len_k, S.Lk);
    if (geo->has_mask && S.m_off >= 0 && S.m_si != 0) plan.any_pair_mask = true;
    if ((geo->has_mask && S.m_off >= 0) || S.Lk % 64 != 0) plan.masked_tiles = true;
    {
      const int64_t elt = geo->dtype == OOPS_F32 ? 4 : 2;
      const int64_t lim = int64_t(1) << 31;
      const int64_t kspan = (S.Lk * std::max(S.k_si, S.v_si) + geo->head_size) * elt;
      const int64_t bspan = (S.Lq * std::max<int64_t>(S.b_si, 0) + S.Lk) * elt;
      if (kspan >= lim || bspan >= lim) plan.offsets_32bit = false;
    }
    if (geo->has_bias && S.b_off >= 0) {
      if (S.bias_mode == OOPS_BIAS_FULL) plan.any_full = true;
      if (S.bias_mode == OOPS_BIAS_SHARED) {
        plan.any_shared = true;
        min_shared_groups = std::min(min_shared_groups, S.G);
      }
      if (S.bias_mode != OOPS_BIAS_NONE) {
        const int64_t gspan = S.bias_mode == OOPS_BIAS_SHARED ? 1 : S.G;
        plan.dbias_extent =
            std::max(plan.dbias_extent, extent(S.db_off, gspan, S.db_sg, H, S.db_sh, S.Lq, S.db_si, S.Lk));
      }
    }
  }
  if (plan.fwd_tiles > kMaxGrid || plan.delta_tiles > kMaxGrid || plan.dkv_tiles > kMaxGrid)
    return fail(OOPS_EINVAL, "launch grid exceeds 2^31-1 workgroups");
  plan.fwd_uniform = u_fwd ? c_fwd : 0;
  plan.delta_uniform = u_delta ? c_delta : 0;
  plan.dkv_uniform = u_dkv ? c_dkv : 0;
  plan.dkv_uniform_r2 = u_dkv2 ? c_dkv2 : 0;
  if (plan.any_shared) {
    int64_t parts = cdiv(kTargetSharedBiasBlocks, std::max<int64_t>(sbias_base, 1));
    parts = std::min<int64_t>({parts, kMaxParts, min_shared_groups});
    plan.parts = (int)std::max<int64_t>(parts, 1);
    plan.sbias_tiles = sbias_base * plan.parts;
    plan.sbias_uniform = u_sb && c_sb > 0 ? c_sb * plan.parts : 0;
    // fast path: parts per sample, each covering about the same number of
    // groups, with about kTargetSharedBiasBlocks workgroups in all
    int64_t units = 0;
    for (int s = 0; s < geo->num_samples; ++s) {
      const Sample& S = tab[s];
      if (S.bias_mode == OOPS_BIAS_SHARED) units += H * cdiv(S.Lq, 128) * cdiv(S.Lk, 64) * S.G;
    }
    plan.fast_part_groups = std::max<int64_t>(cdiv(units, kTargetSharedBiasBlocks), kMinPartGroups);
    plan.fast_parts = 1;
    plan.fast_sbias_tiles = 0;
    int64_t c_f = -1;
    bool u_f = true;
    for (int s = 0; s < geo->num_samples; ++s) {
      const Sample& S = tab[s];
      int64_t c = 0;
      if (S.bias_mode == OOPS_BIAS_SHARED) {
        const int p = oops::parts_for(S.G, plan.fast_part_groups, kMaxParts);
        c = H * cdiv(S.Lq, 128) * cdiv(S.Lk, 64) * p;
        plan.fast_parts = std::max(plan.fast_parts, p);
      }
      plan.fast_sbias_tiles += c;
      track(c, c_f, u_f);
    }
    plan.fast_sbias_uniform = u_f && c_f > 0 ? c_f : 0;
    int64_t c_red = -1;
    bool u_red = true;
    for (int s = 0; s < geo->num_samples; ++s) {
      const Sample& S = tab[s];
      const int64_t c = S.bias_mode == OOPS_BIAS_SHARED ? cdiv(H * S.Lq * S.Lk, 256) : 0;
      plan.sred_tiles += c;
      track(c, c_red, u_red);
    }
    plan.sred_uniform = u_red && c_red > 0 ? c_red : 0;
    // fused dK/dV + dBias kernel: one workgroup per (head, 32-key block, part),
    // about kTargetFusedBlocks workgroups (whole rounds of one per CU)
    // (samples longer than kFusedMaxLen take a second launch with eight waves per row when every one of
    // them fits it, else the separate dK/dV and dBias kernels: a split batch)
    plan.all_shared = geo->has_bias != 0;
    int64_t fused_units = 0;
    bool long_ok = true;
    for (int s = 0; s < geo->num_samples; ++s) {
      const Sample& S = tab[s];
      if (S.bias_mode != OOPS_BIAS_SHARED || S.b_off < 0) plan.all_shared = false;
      if (S.Lq > oops::kFusedLongMaxLen) long_ok = false;
    }
    for (int s = 0; s < geo->num_samples; ++s) {
      const Sample& S = tab[s];
      if (S.Lq <= oops::kFusedMaxLen || long_ok) fused_units += H * cdiv(S.Lk, 32) * S.G;
    }
    if (plan.all_shared) {
      plan.fused_part_groups = std::max<int64_t>(cdiv(fused_units, kTargetFusedBlocks), kMinFusedPartGroups);
      int64_t c_fu = -1, c_lo = -1;
      bool u_fu = true, u_lo = true, rest = false;
      for (int s = 0; s < geo->num_samples; ++s) {
        const Sample& S = tab[s];
        if (S.Lq > oops::kFusedMaxLen && long_ok) {
          const int p = oops::parts_for(S.G, plan.fused_part_groups, kMaxParts);
          const int64_t c = H * cdiv(S.Lk, 32) * p;
          plan.fused_parts = std::max(plan.fused_parts, p);
          plan.fused_long_tiles += c;
          track(c, c_lo, u_lo);
          continue;
        }
        if (S.Lq > oops::kFusedMaxLen) {
          rest = true;
          plan.dkv_rest_tiles += S.G * H * cdiv(S.Lk, 128);
          plan.fast_sbias_rest_tiles +=
              H * cdiv(S.Lq, 128) * cdiv(S.Lk, 64) * oops::parts_for(S.G, plan.fast_part_groups, kMaxParts);
          continue;
        }
        const int p = oops::parts_for(S.G, plan.fused_part_groups, kMaxParts);
        const int64_t c = H * cdiv(S.Lk, 32) * p;
        plan.fused_parts = std::max(plan.fused_parts, p);
        plan.fused_tiles += c;
        plan.fused_max_len_q = std::max(plan.fused_max_len_q, S.Lq);
        track(c, c_fu, u_fu);
      }
      // (uniform tile counts only when one launch serves every sample)
      plan.fused_uniform = u_fu && !rest && plan.fused_long_tiles == 0 && c_fu > 0 ? c_fu : 0;
      plan.fused_long_uniform = u_lo && plan.fused_tiles == 0 && c_lo > 0 ? c_lo : 0;
      // not served by the fused kernel (16-bit, head size <= 32 only)
      if (plan.fused_tiles > kMaxGrid || plan.fused_long_tiles > kMaxGrid || geo->dtype == OOPS_F32 || plan.dp != 32)
        plan.fused_tiles = plan.fused_long_tiles = 0;
      plan.fused_split = rest && plan.fused_tiles > 0;
    }
    if (plan.sbias_tiles > kMaxGrid || plan.fast_sbias_tiles > kMaxGrid || plan.sred_tiles > kMaxGrid)
      return fail(OOPS_EINVAL, "dBias launch grid exceeds 2^31-1 workgroups");
  }
  // fragment-major copy of the shared biases for the fast kernels: one slab
  // of H x ceil(Lq/32) x ceil(Lk/32) x 1024 elements per sample (the largest
  // sample's extent, so a kernel finds its slab from the sample index alone)
  if (geo->has_bias && plan.any_shared && oops::fast_path_ok(*geo, plan)) {
    const int64_t nqt = cdiv(plan.max_len_q, 32), nkt = cdiv(plan.max_len_k, 32);
    const int64_t stride = H * nqt * nkt * 1024;
    const size_t bytes = (size_t)stride * (size_t)geo->num_samples * 2;
    // a ragged batch whose slabs would far exceed its biases keeps the direct loads
    if (bytes <= kMaxBiasFragBytes && (int64_t)geo->num_samples * H * nqt * nkt * 128 <= kMaxGrid * 256) {
      plan.bias_frag = true;
      plan.bf_nqt = (int)nqt;
      plan.bf_nkt = (int)nkt;
      plan.bf_sample_stride = stride;
      plan.bf_bytes = bytes;
    }
  }
  plan.fused_ok = oops::dkvb_fused_ok(*geo, plan);
  return OOPS_OK;
}

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Backward workspace: delta [lse_extent f32] | LSE/delta pack [2 lse_extent f32] and compact
// Q, dO [2 lse_extent kCompactRow 16-bit] (fused dK/dV + dBias kernel) | dBias partial slabs |
// bias fragment copy.
// (only when the fused dK/dV + dBias kernel serves the geometry: 8 bytes of pack and
// 4 kCompactRow = 128 bytes of compact Q and dO per (sample, group, head, query) row)
size_t pack_bytes(const oops::Plan& plan) {
  return plan.fused_ok ? align256(sizeof(float) * 2 * (size_t)plan.lse_extent) : 0;
}
size_t compact_bytes(const oops::Plan& plan) {
  return plan.fused_ok ? align256(2 * sizeof(uint16_t) * (size_t)plan.lse_extent * oops::kCompactRow) : 0;
}

size_t parts_bytes(const oops::Plan& plan) {
  const int parts = std::max({plan.parts, plan.fast_parts, plan.fused_parts});
  return plan.any_shared && parts > 1 ? align256(sizeof(float) * (size_t)parts * plan.dbias_extent) : 0;
}

size_t workspace_bytes(const oops::Plan& plan) {
  return align256(sizeof(float) * (size_t)plan.lse_extent) + pack_bytes(plan) + compact_bytes(plan) +
         parts_bytes(plan) + align256(plan.bf_bytes);
}

size_t forward_workspace_bytes(const oops::Plan& plan) { return align256(plan.bf_bytes); }

int check_workspace(void* workspace, size_t ws_bytes, size_t need) {
  if (need == 0) return OOPS_OK;
  if (workspace == nullptr || ws_bytes < need)
    return fail(OOPS_EWORKSPACE, "workspace of %lld bytes required, %lld given", (long long)need,
                (long long)(workspace ? ws_bytes : 0));
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return fail(OOPS_EWORKSPACE, "workspace must be 256-byte aligned");
  return OOPS_OK;
}

int check_gate(const oops_gate_geometry* g) {
  if (g == nullptr) return fail(OOPS_EINVAL, "gate geometry is NULL");
  if (g->dtype < OOPS_F32 || g->dtype > OOPS_F16) return fail(OOPS_EINVAL, "unknown dtype %lld", g->dtype);
  if (g->heads <= 0 || g->width <= 0)
    return fail(OOPS_EINVAL, "heads and width must be positive, got %lld and %lld", g->heads, g->width);
  if (g->rows < 0 || g->tokens <= 0 || g->groups <= 0)
    return fail(OOPS_EINVAL, "rows must be >= 0 and tokens, groups positive");
  if (g->rows % g->tokens) return fail(OOPS_EINVAL, "rows (%lld) must be a multiple of tokens (%lld)", g->rows, g->tokens);
  if ((int64_t)g->heads * g->width > (int64_t(1) << 20)) return fail(OOPS_EINVAL, "heads * width too large");
  return OOPS_OK;
}

int check_row_norm(const oops_row_norm_geometry* g) {
  if (g == nullptr) return fail(OOPS_EINVAL, "row-norm geometry is NULL");
  if (g->dtype != OOPS_BF16 && g->dtype != OOPS_F16 && g->dtype != OOPS_F32)
    return fail(OOPS_EINVAL, "unknown dtype %lld", g->dtype);
  if (g->width <= 0 || g->width > 8192) return fail(OOPS_EINVAL, "width must be in 1..8192, got %lld", g->width);
  if (g->rows < 0) return fail(OOPS_EINVAL, "rows must be >= 0");
  if (g->x_row < g->width || g->y_row < g->width)
    return fail(OOPS_EINVAL, "row strides (%lld, %lld) must cover the width", g->x_row, g->y_row);
  if (g->y_row > 8192) return fail(OOPS_EINVAL, "y row stride too large (%lld)", g->y_row);
  return OOPS_OK;
}

int check_trimul(const oops_trimul_geometry* g) {
  if (g == nullptr) return fail(OOPS_EINVAL, "triangle multiplication geometry is NULL");
  if (g->dtype != OOPS_BF16 && g->dtype != OOPS_F16 && g->dtype != OOPS_F32)
    return fail(OOPS_EINVAL, "the triangle multiplication kernels serve bfloat16, float16 and float32 (dtype %lld)",
                g->dtype);
  if (g->channels <= 0 || g->channels > 1024 || g->hidden <= 0 || g->hidden > 1024)
    return fail(OOPS_EINVAL, "channels and hidden must be in 1..1024, got %lld and %lld", g->channels, g->hidden);
  if (g->groups < 0 || g->positions < 0) return fail(OOPS_EINVAL, "groups and positions must be >= 0");
  if (g->c_row < g->channels || g->c_row % 8 || g->h_row < g->hidden || g->h_row % 8)
    return fail(OOPS_EINVAL, "c_row and h_row must be multiples of 8 covering C and H (%lld, %lld)", g->c_row,
                g->h_row);
  if (g->groups * g->positions > (int64_t(1) << 40)) return fail(OOPS_EINVAL, "too many pair cells");
  return OOPS_OK;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int gate_launch_result(hipError_t err, const char* what) {
  if (err == hipSuccess) return OOPS_OK;
  g_last_error = std::string(what) + " launch failed: " + hipGetErrorString(err);
  return OOPS_ELAUNCH;
}

// Device scratch of oops_attn_forward_noalloc: the fragment-major bias copy
// that oops_attn_forward puts in its caller's workspace.  Every GPU the
// library runs on holds its own copy of this array until the process ends.
// In host code `scratch` only names the symbol; its device address on the
// current GPU comes from hipGetSymbolAddress, taken once per device.
constexpr size_t kNoAllocScratchBytes = OOPS_NOALLOC_SCRATCH_BYTES;
static_assert(kNoAllocScratchBytes % 256 == 0, "scratch size");
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the
// first call on that device).
int scratch_on_current_device(void** ptr) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return fail(OOPS_ELAUNCH, "hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return fail(OOPS_EINVAL, "device index %lld out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr) {
      g_last_error = std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(err);
      return OOPS_ELAUNCH;
    }
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return OOPS_OK;
}

int check_forward_pointers(const oops_attn_geometry* geo, const void* q, const void* k, const void* v,
                           const uint8_t* mask, const void* bias, const void* out) {
  if (!q || !k || !v || !out) return fail(OOPS_EINVAL, "q, k, v and out must be non-NULL");
  if (geo->has_bias && !bias) return fail(OOPS_EINVAL, "has_bias is set but bias is NULL");
  if (geo->has_mask && !mask) return fail(OOPS_EINVAL, "has_mask is set but mask is NULL");
  return OOPS_OK;
}

int run_forward(const oops_attn_geometry* geo, const oops::Plan& plan, const void* q, const void* k, const void* v,
                const uint8_t* mask, const void* bias, void* out, void* out_lo, float* lse, void* workspace,
                void* stream) {
  const hipError_t err = oops::launch_forward(*geo, plan, q, k, v, mask, bias, workspace, out, out_lo, lse,
                                              static_cast<hipStream_t>(stream));
  if (err != hipSuccess) {
    g_last_error = std::string("forward launch failed: ") + hipGetErrorString(err);
    return OOPS_ELAUNCH;
  }
  return OOPS_OK;
}

}  // namespace

extern "C" {

int oops_abi_version(void) { return 6; }

const char* oops_last_error(void) { return g_last_error.c_str(); }

size_t oops_attn_forward_workspace_bytes(const oops_attn_geometry* geo) {
  oops::Plan plan;
  if (make_plan(geo, plan)) return 0;
  return forward_workspace_bytes(plan);
}

int oops_attn_forward(const oops_attn_geometry* geo, const void* q, const void* k, const void* v,
                      const uint8_t* mask, const void* bias, void* out, void* out_lo, float* lse, void* workspace,
                      size_t ws_bytes, void* stream) {
  g_last_error.clear();
  oops::Plan plan;
  if (int rc = make_plan(geo, plan)) return rc;
  if (int rc = check_forward_pointers(geo, q, k, v, mask, bias, out)) return rc;
  if (int rc = check_workspace(workspace, ws_bytes, forward_workspace_bytes(plan))) return rc;
  return run_forward(geo, plan, q, k, v, mask, bias, out, out_lo, lse, workspace, stream);
}

int oops_attn_forward_noalloc(const oops_attn_geometry* geo, const void* q, const void* k, const void* v,
                              const uint8_t* mask, const void* bias, void* out, void* out_lo, float* lse,
                              void* stream) {
  g_last_error.clear();
  oops::Plan plan;
  if (int rc = make_plan(geo, plan)) return rc;
  size_t need = forward_workspace_bytes(plan);
  if (need > kNoAllocScratchBytes) {
    // The fragment-major bias copy is the only scratch the forward uses, and
    // it is an optimisation: without it the kernels read the bias rows.
    plan.bias_frag = false;
    plan.bf_bytes = 0;
    need = forward_workspace_bytes(plan);
  }
  if (need > kNoAllocScratchBytes)
    return fail(OOPS_EWORKSPACE, "this geometry needs %lld bytes of scratch; the no-allocation forward has %lld",
                (long long)need, (long long)kNoAllocScratchBytes);
  if (int rc = check_forward_pointers(geo, q, k, v, mask, bias, out)) return rc;
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = scratch_on_current_device(&ws)) return rc;
  }
  return run_forward(geo, plan, q, k, v, mask, bias, out, out_lo, lse, ws, stream);
}

size_t oops_attn_backward_workspace_bytes(const oops_attn_geometry* geo) {
  oops::Plan plan;
  if (make_plan(geo, plan)) return 0;
  return workspace_bytes(plan);
}

int oops_attn_backward(const oops_attn_geometry* geo, const void* q, const void* k, const void* v,
                       const uint8_t* mask, const void* bias, const void* out, const void* out_lo,
                       const float* lse, const void* dout, void* dq, void* dk, void* dv, float* dbias, void* workspace,
                       size_t ws_bytes, void* stream) {
  g_last_error.clear();
  oops::Plan plan;
  if (int rc = make_plan(geo, plan)) return rc;
  if (!q || !k || !v || !out || !lse || !dout) return fail(OOPS_EINVAL, "q, k, v, out, lse and dout must be non-NULL");
  if (geo->has_bias && !bias) return fail(OOPS_EINVAL, "has_bias is set but bias is NULL");
  if (geo->has_mask && !mask) return fail(OOPS_EINVAL, "has_mask is set but mask is NULL");
  if (int rc = check_workspace(workspace, ws_bytes, workspace_bytes(plan))) return rc;
  char* ws = static_cast<char*>(workspace);
  float* delta = reinterpret_cast<float*>(ws);
  const size_t delta_bytes = align256(sizeof(float) * (size_t)plan.lse_extent) + pack_bytes(plan) + compact_bytes(plan);
  float* pack = pack_bytes(plan) ? delta + align256(sizeof(float) * (size_t)plan.lse_extent) / 4 : nullptr;
  void* compact = compact_bytes(plan) ? reinterpret_cast<char*>(pack) + pack_bytes(plan) : nullptr;
  float* parts = parts_bytes(plan) ? reinterpret_cast<float*>(ws + delta_bytes) : nullptr;
  void* bias_frag = plan.bias_frag ? ws + delta_bytes + parts_bytes(plan) : nullptr;
  const hipError_t err = oops::launch_backward(*geo, plan, q, k, v, mask, bias, out, out_lo, lse, dout, dq, dk, dv,
                                               geo->has_bias ? dbias : nullptr, delta, pack, compact, parts, bias_frag,
                                               static_cast<hipStream_t>(stream));
  if (err != hipSuccess) {
    g_last_error = std::string("backward launch failed: ") + hipGetErrorString(err);
    return OOPS_ELAUNCH;
  }
  return OOPS_OK;
}

int oops_gate_projection_forward(const oops_gate_geometry* geo, const void* single, const void* weight,
                                 const void* attention, void* gated, void* logits, void* stream) {
  g_last_error.clear();
  if (int rc = check_gate(geo)) return rc;
  if (geo->channels <= 0) return fail(OOPS_EINVAL, "channels must be positive, got %lld", geo->channels);
  if (!single || !weight || !attention || !gated)
    return fail(OOPS_EINVAL, "single, weight, attention and gated must be non-NULL");
  if (!oops::gate_projection_ok(*geo, single, weight, attention, gated, logits))
    return fail(OOPS_EINVAL,
                "the fused gate projection needs 16-bit operands, channels %% 8 == 0, width %% 16 == 0, "
                "unit-stride attention channels and 16-byte aligned rows");
  return gate_launch_result(oops::launch_gate_projection(*geo, single, weight, attention, gated, logits,
                                                         static_cast<hipStream_t>(stream)),
                            "gate projection");
}

int oops_gate_multiply_forward(const oops_gate_geometry* geo, const void* attention, const void* logits,
                               void* gated, void* stream) {
  g_last_error.clear();
  if (int rc = check_gate(geo)) return rc;
  if (!attention || !logits || !gated) return fail(OOPS_EINVAL, "attention, logits and gated must be non-NULL");
  return gate_launch_result(
      oops::launch_gate_multiply_forward(*geo, attention, logits, gated, static_cast<hipStream_t>(stream)),
      "gate multiply forward");
}

int oops_gate_multiply_backward(const oops_gate_geometry* geo, const void* attention, const void* logits,
                                const void* grad, void* grad_attention, void* grad_logits, void* stream) {
  g_last_error.clear();
  if (int rc = check_gate(geo)) return rc;
  if (!logits || !grad) return fail(OOPS_EINVAL, "logits and grad must be non-NULL");
  if (grad_logits && !attention) return fail(OOPS_EINVAL, "grad_logits needs the attention values");
  return gate_launch_result(oops::launch_gate_multiply_backward(*geo, attention, logits, grad, grad_attention,
                                                                grad_logits, static_cast<hipStream_t>(stream)),
                            "gate multiply backward");
}

int oops_layer_norm_rows_forward(const oops_row_norm_geometry* geo, const void* x, const float* weight,
                                 const float* bias, void* y, float* mean, float* rstd, void* stream) {
  g_last_error.clear();
  if (int rc = check_row_norm(geo)) return rc;
  if (!x || !y || !mean || !rstd) return fail(OOPS_EINVAL, "x, y, mean and rstd must be non-NULL");
  return gate_launch_result(oops::launch_layer_norm_rows_forward(*geo, x, weight, bias, y, mean, rstd,
                                                                 static_cast<hipStream_t>(stream)),
                            "row LayerNorm forward");
}

size_t oops_layer_norm_rows_parts(const oops_row_norm_geometry* geo) {
  if (check_row_norm(geo)) return 0;
  return (size_t)oops::layer_norm_rows_parts(*geo);
}

int oops_layer_norm_rows_backward(const oops_row_norm_geometry* geo, const void* x, const float* weight,
                                  const float* mean, const float* rstd, const void* grad_y, void* grad_x,
                                  float* grad_weight_parts, float* grad_bias_parts, void* stream) {
  g_last_error.clear();
  if (int rc = check_row_norm(geo)) return rc;
  if (!x || !mean || !rstd || !grad_y || !grad_x)
    return fail(OOPS_EINVAL, "x, mean, rstd, grad_y and grad_x must be non-NULL");
  return gate_launch_result(oops::launch_layer_norm_rows_backward(*geo, x, weight, mean, rstd, grad_y, grad_x,
                                                                  grad_weight_parts, grad_bias_parts,
                                                                  static_cast<hipStream_t>(stream)),
                            "row LayerNorm backward");
}

namespace {
// the two float32 partial arrays [parts][width] the backward kernel writes,
// as the segments of the fixed-order sums into the final gradients
int ln_affine_segments(const oops_row_norm_geometry& g, float* parts, float* grad_weight, float* grad_bias,
                       oops_sum_segment (&seg)[2]) {
  const int64_t P = oops::layer_norm_rows_parts(g), W = g.width;
  int n = 0;
  if (grad_weight) seg[n++] = oops_sum_segment{parts, grad_weight, P, W, W, OOPS_F32, 0};
  if (grad_bias) seg[n++] = oops_sum_segment{parts + P * W, grad_bias, P, W, W, OOPS_F32, 0};
  return n;
}
size_t ln_parts_bytes(const oops_row_norm_geometry& g) {
  return align256((size_t)2 * (size_t)oops::layer_norm_rows_parts(g) * (size_t)g.width * sizeof(float));
}
}  // namespace

size_t oops_layer_norm_rows_backward_workspace_bytes(const oops_row_norm_geometry* geo) {
  if (check_row_norm(geo)) return 0;
  oops_sum_segment seg[2];
  float one = 0.f;
  const int n = ln_affine_segments(*geo, nullptr, &one, &one, seg);
  return ln_parts_bytes(*geo) + oops::sum_partials_workspace_bytes(seg, n);
}

int oops_layer_norm_rows_backward_affine(const oops_row_norm_geometry* geo, const void* x, const float* weight,
                                         const float* mean, const float* rstd, const void* grad_y, void* grad_x,
                                         float* grad_weight, float* grad_bias, void* workspace, size_t ws_bytes,
                                         void* stream) {
  g_last_error.clear();
  if (int rc = check_row_norm(geo)) return rc;
  if (!x || !mean || !rstd || !grad_y || !grad_x)
    return fail(OOPS_EINVAL, "x, mean, rstd, grad_y and grad_x must be non-NULL");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (!grad_weight && !grad_bias)
    return gate_launch_result(oops::launch_layer_norm_rows_backward(*geo, x, weight, mean, rstd, grad_y, grad_x,
                                                                    nullptr, nullptr, st),
                              "row LayerNorm backward");
  if (int rc = check_workspace(workspace, ws_bytes, oops_layer_norm_rows_backward_workspace_bytes(geo))) return rc;
  float* parts = static_cast<float*>(workspace);
  const int64_t pw = oops::layer_norm_rows_parts(*geo) * geo->width;
  hipError_t e = oops::launch_layer_norm_rows_backward(*geo, x, weight, mean, rstd, grad_y, grad_x,
                                                       grad_weight ? parts : nullptr, grad_bias ? parts + pw : nullptr,
                                                       st);
  if (e == hipSuccess && geo->rows > 0) {
    oops_sum_segment seg[2];
    const int n = ln_affine_segments(*geo, parts, grad_weight, grad_bias, seg);
    e = oops::launch_sum_partials(seg, n, static_cast<char*>(workspace) + ln_parts_bytes(*geo), st);
  }
  return gate_launch_result(e, "row LayerNorm backward");
}

int oops_trimul_factors_forward(const oops_trimul_geometry* geo, const void* normalized, const void* weight,
                                const float* bias, const void* mask, void* factors, void* stream) {
  g_last_error.clear();
  if (int rc = check_trimul(geo)) return rc;
  if (!normalized || !weight || !factors) return fail(OOPS_EINVAL, "normalized, weight and factors must be non-NULL");
  if (geo->has_mask && !mask) return fail(OOPS_EINVAL, "has_mask is set but mask is NULL");
  if (!aligned16(normalized) || !aligned16(weight) || !aligned16(factors) || (geo->has_mask && !aligned16(mask)))
    return fail(OOPS_EINVAL, "normalized, weight, mask and factors must be 16-byte aligned");
  return gate_launch_result(oops::launch_trimul_factors(*geo, normalized, weight, bias, mask, factors, nullptr,
                                                        nullptr, nullptr, nullptr, static_cast<hipStream_t>(stream)),
                            "triangle multiplication factors");
}

size_t oops_trimul_mask_parts(const oops_trimul_geometry* geo) {
  if (check_trimul(geo)) return 0;
  return (size_t)oops::trimul_mask_parts(*geo);
}

size_t oops_trimul_bias_parts(const oops_trimul_geometry* geo) {
  if (check_trimul(geo)) return 0;
  return (size_t)oops::trimul_bias_parts(*geo);
}

int oops_trimul_factors_backward(const oops_trimul_geometry* geo, const void* normalized, const void* weight,
                                 const float* bias, const void* mask, const void* grad_factors,
                                 void* grad_projection, float* grad_mask_parts, float* grad_bias_parts,
                                 void* stream) {
  g_last_error.clear();
  if (int rc = check_trimul(geo)) return rc;
  if (!normalized || !weight || !grad_factors || !grad_projection)
    return fail(OOPS_EINVAL, "normalized, weight, grad_factors and grad_projection must be non-NULL");
  if (geo->has_mask && !mask) return fail(OOPS_EINVAL, "has_mask is set but mask is NULL");
  if (!aligned16(normalized) || !aligned16(weight) || !aligned16(grad_factors) || !aligned16(grad_projection) ||
      (geo->has_mask && !aligned16(mask)))
    return fail(OOPS_EINVAL, "operands must be 16-byte aligned");
  return gate_launch_result(oops::launch_trimul_factors(*geo, normalized, weight, bias, mask, nullptr, grad_factors,
                                                        grad_projection, grad_mask_parts, grad_bias_parts,
                                                        static_cast<hipStream_t>(stream)),
                            "triangle multiplication factor backward");
}

int oops_trimul_output_norm_forward(const oops_trimul_geometry* geo, const void* combined, const float* weight,
                                    const float* bias, void* normalized, float* mean, float* rstd, void* stream) {
  g_last_error.clear();
  if (int rc = check_trimul(geo)) return rc;
  if (!combined || !normalized || !mean || !rstd)
    return fail(OOPS_EINVAL, "combined, normalized, mean and rstd must be non-NULL");
  return gate_launch_result(oops::launch_trimul_output_norm_forward(*geo, combined, weight, bias, normalized, mean,
                                                                    rstd, static_cast<hipStream_t>(stream)),
                            "triangle multiplication output norm");
}

size_t oops_trimul_output_norm_parts(const oops_trimul_geometry* geo) {
  if (check_trimul(geo)) return 0;
  return (size_t)oops::trimul_output_norm_parts(*geo);
}

int oops_trimul_output_norm_backward(const oops_trimul_geometry* geo, const void* combined, const float* weight,
                                     const float* mean, const float* rstd, const void* grad_normalized,
                                     void* grad_combined, float* grad_weight_parts, float* grad_bias_parts,
                                     void* stream) {
  g_last_error.clear();
  if (int rc = check_trimul(geo)) return rc;
  if (!combined || !mean || !rstd || !grad_normalized || !grad_combined)
    return fail(OOPS_EINVAL, "combined, mean, rstd, grad_normalized and grad_combined must be non-NULL");
  return gate_launch_result(oops::launch_trimul_output_norm_backward(*geo, combined, weight, mean, rstd,
                                                                     grad_normalized, grad_combined,
                                                                     grad_weight_parts, grad_bias_parts,
                                                                     static_cast<hipStream_t>(stream)),
                            "triangle multiplication output norm backward");
}

int oops_trimul_output_forward(const oops_trimul_geometry* geo, const void* normalized, const void* pair_normalized,
                               const void* output_weight, const void* gate_weight, const float* output_bias,
                               const float* gate_bias, void* out, void* stream) {
  g_last_error.clear();
  if (int rc = check_trimul(geo)) return rc;
  if (!normalized || !pair_normalized || !output_weight || !gate_weight || !out)
    return fail(OOPS_EINVAL, "normalized, pair_normalized, both weights and out must be non-NULL");
  if (!aligned16(normalized) || !aligned16(pair_normalized) || !aligned16(output_weight) || !aligned16(gate_weight) ||
      !aligned16(out))
    return fail(OOPS_EINVAL, "operands must be 16-byte aligned");
  return gate_launch_result(oops::launch_trimul_output(*geo, normalized, pair_normalized, output_weight, gate_weight,
                                                       output_bias, gate_bias, out, nullptr, nullptr, nullptr,
                                                       static_cast<hipStream_t>(stream)),
                            "triangle multiplication output");
}

int oops_trimul_output_backward(const oops_trimul_geometry* geo, const void* normalized,
                                const void* pair_normalized, const void* output_weight, const void* gate_weight,
                                const float* output_bias, const float* gate_bias, const void* grad_out,
                                void* grad_value, void* grad_gate, void* stream) {
  g_last_error.clear();
  if (int rc = check_trimul(geo)) return rc;
  if (!normalized || !pair_normalized || !output_weight || !gate_weight || !grad_out || !grad_value || !grad_gate)
    return fail(OOPS_EINVAL, "operands and both gradients must be non-NULL");
  if (!aligned16(normalized) || !aligned16(pair_normalized) || !aligned16(output_weight) || !aligned16(gate_weight) ||
      !aligned16(grad_out) || !aligned16(grad_value) || !aligned16(grad_gate))
    return fail(OOPS_EINVAL, "operands must be 16-byte aligned");
  return gate_launch_result(oops::launch_trimul_output(*geo, normalized, pair_normalized, output_weight, gate_weight,
                                                       output_bias, gate_bias, nullptr, grad_out, grad_value,
                                                       grad_gate, static_cast<hipStream_t>(stream)),
                            "triangle multiplication output backward");
}

size_t oops_trimul_output_grad_parts(const oops_trimul_geometry* geo) {
  g_last_error.clear();
  if (check_trimul(geo)) return 0;
  return (size_t)oops::trimul_output_grad_parts(*geo);
}

int oops_trimul_output_grad_products(const oops_trimul_geometry* geo, const void* x, int64_t x_row, const void* w,
                                     int64_t w_row, const void* y, int64_t y_row, void* d, int64_t d_row,
                                     float* g_parts, float* s_parts, void* stream) {
  g_last_error.clear();
  if (int rc = check_trimul(geo)) return rc;
  if (!oops::trimul_output_grad_supported(*geo))
    return fail(OOPS_EINVAL, "the output-gradient products serve 16-bit pairs with C = H = 128");
  if (!x || !w || !y || !d || !g_parts || !s_parts) return fail(OOPS_EINVAL, "operands must be non-NULL");
  if (x_row < 128 || w_row < 128 || y_row < 128 || d_row < 128 || x_row % 8 || w_row % 8 || y_row % 8 || d_row % 8)
    return fail(OOPS_EINVAL, "row strides must be multiples of 8 of at least 128 elements");
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) || !aligned16(d))
    return fail(OOPS_EINVAL, "operands must be 16-byte aligned");
  return gate_launch_result(oops::launch_trimul_output_grad(*geo, x, x_row, w, w_row, y, y_row, d, d_row, g_parts,
                                                            s_parts, static_cast<hipStream_t>(stream)),
                            "triangle multiplication output-gradient products");
}

namespace {
int check_sum_segments(const oops_sum_segment* segments, int32_t num_segments) {
  if (num_segments < 0 || num_segments > OOPS_SUM_MAX_SEGMENTS)
    return fail(OOPS_EINVAL, "num_segments %lld outside 0..%lld", num_segments, OOPS_SUM_MAX_SEGMENTS);
  if (num_segments > 0 && segments == nullptr) return fail(OOPS_EINVAL, "segments must be non-NULL");
  for (int i = 0; i < num_segments; ++i) {
    const oops_sum_segment& s = segments[i];
    if (s.n < 0 || s.count < 0 || s.part_stride < s.n)
      return fail(OOPS_EINVAL, "segment %lld: need n >= 0, count >= 0 and part_stride >= n", i);
    if (s.out_dtype != OOPS_F32 && s.out_dtype != OOPS_BF16 && s.out_dtype != OOPS_F16)
      return fail(OOPS_EINVAL, "segment %lld: unsupported out_dtype %lld", i, s.out_dtype);
    if (s.n > 0 && (s.out == nullptr || (s.count > 0 && s.parts == nullptr)))
      return fail(OOPS_EINVAL, "segment %lld: parts and out must be non-NULL", i);
  }
  return OOPS_OK;
}
}  // namespace

size_t oops_sum_partials_workspace_bytes(const oops_sum_segment* segments, int32_t num_segments) {
  g_last_error.clear();
  if (check_sum_segments(segments, num_segments)) return 0;
  return oops::sum_partials_workspace_bytes(segments, num_segments);
}

int oops_sum_partials(const oops_sum_segment* segments, int32_t num_segments, void* workspace,
                      size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (int rc = check_sum_segments(segments, num_segments)) return rc;
  const size_t need = oops::sum_partials_workspace_bytes(segments, num_segments);
  if (workspace_bytes < need || (need > 0 && (workspace == nullptr || reinterpret_cast<uintptr_t>(workspace) % 256)))
    return fail(OOPS_EINVAL, "workspace of %lld bytes (256-byte aligned) needed, %lld given", (long long)need,
                (long long)workspace_bytes);
  return gate_launch_result(
      oops::launch_sum_partials(segments, num_segments, workspace, static_cast<hipStream_t>(stream)), "partial sums");
}

}  // extern "C"
