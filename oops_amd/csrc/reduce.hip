// Fixed-order sums of float32 partial arrays over their leading axis
// (oops_sum_partials): the last step of the backward passes whose kernels
// write per-workgroup or per-chunk partials instead of using atomics.
//
// sum_partials_kernel sums `count` rows for up to OOPS_SUM_MAX_SEGMENTS arrays
// in one launch: blockIdx.z picks the array, blockIdx.x a run of 64 output
// columns, blockIdx.y a chunk of kChunkParts rows (the whole array when it has
// at most kChunkParts rows).  A workgroup is 64 columns x 4 slices; slice s
// sums its quarter of the chunk's rows in order (consecutive threads read
// consecutive columns of one row), and the four slice sums are combined as
// (s0 + s1) + (s2 + s3).  An array with more rows is summed in two launches:
// chunk sums into the caller's workspace, then the chunk sums.  The order
// depends only on the array's shape, so repeated calls are bit-identical.
#include <hip/hip_runtime.h>

#include "reduce_kernels.h"

namespace oops {
namespace {

constexpr int kSumCols = 64;
constexpr int kSumSlices = 4;
constexpr int64_t kChunkParts = 256;  // rows one workgroup sums (more: two launches)

struct SumJob {
  const float* parts;
  void* out;
  int64_t count, n, stride;
  int32_t out_dtype, whole;  // whole: all rows into out; else chunk sums into out (a workspace)
};
struct SumArgs {
  SumJob job[OOPS_SUM_MAX_SEGMENTS];
};

__device__ __forceinline__ void store_out(void* out, int32_t dtype, int64_t j, float v) {
  if (dtype == OOPS_F32)
    static_cast<float*>(out)[j] = v;
  else if (dtype == OOPS_BF16)
    static_cast<__bf16*>(out)[j] = (__bf16)v;
  else
    static_cast<_Float16*>(out)[j] = (_Float16)v;
}

// whole (out = the result) or chunked (out = workspace rows [chunk][n], float32)
__global__ __launch_bounds__(256) void sum_partials_kernel(SumArgs a) {
  const SumJob& s = a.job[blockIdx.z];
  const int64_t chunks = (s.count + kChunkParts - 1) / kChunkParts;
  const bool chunked = !s.whole;
  if ((int64_t)blockIdx.y >= (chunked ? chunks : 1)) return;
  const int col = threadIdx.x & (kSumCols - 1), slice = threadIdx.x / kSumCols;
  const int64_t p0 = chunked ? (int64_t)blockIdx.y * kChunkParts : 0;
  const int64_t p1 = chunked ? (p0 + kChunkParts < s.count ? p0 + kChunkParts : s.count) : s.count;
  // slice s takes rows p0 + s q .. p0 + (s + 1) q - 1 of the chunk (q = ceil(rows / 4))
  const int64_t q = (p1 - p0 + kSumSlices - 1) / kSumSlices;
  const int64_t r0 = p0 + slice * q, r1 = r0 + q < p1 ? r0 + q : p1;
  __shared__ float part[kSumSlices][kSumCols];
  for (int64_t j0 = (int64_t)blockIdx.x * kSumCols; j0 < s.n; j0 += (int64_t)gridDim.x * kSumCols) {
    const int64_t j = j0 + col;
    float acc = 0.f;
    if (j < s.n) {
      const float* src = s.parts + j;
#pragma unroll 8
      for (int64_t p = r0; p < r1; ++p) acc += src[p * s.stride];
    }
    part[slice][col] = acc;
    __syncthreads();
    if (slice == 0 && j < s.n) {
      const float v = (part[0][col] + part[1][col]) + (part[2][col] + part[3][col]);
      if (chunked)
        static_cast<float*>(s.out)[(int64_t)blockIdx.y * s.n + j] = v;
      else
        store_out(s.out, s.out_dtype, j, v);
    }
    __syncthreads();
  }
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

hipError_t run(const SumArgs& a, int count, int64_t cols, int64_t chunks, hipStream_t stream) {
  int64_t blocks = (cols + kSumCols - 1) / kSumCols;
  if (blocks > 1024) blocks = 1024;  // larger arrays: each workgroup walks several column runs
  hipLaunchKernelGGL(sum_partials_kernel, dim3((unsigned)blocks, (unsigned)chunks, (unsigned)count), dim3(256), 0,
                     stream, a);
  return hipGetLastError();
}

}  // namespace

size_t sum_partials_workspace_bytes(const oops_sum_segment* segs, int count) {
  size_t bytes = 0;
  for (int i = 0; i < count; ++i)
    if (segs[i].count > kChunkParts)
      bytes += align256((size_t)((segs[i].count + kChunkParts - 1) / kChunkParts) * (size_t)segs[i].n * 4);
  return bytes;
}

hipError_t launch_sum_partials(const oops_sum_segment* segs, int count, void* workspace, hipStream_t stream) {
  // first launch: arrays with more than kChunkParts rows, into chunk sums in the workspace
  SumArgs first{}, second{};
  int nfirst = 0;
  int64_t cols1 = 0, chunks1 = 0, cols2 = 0;
  char* ws = static_cast<char*>(workspace);
  for (int i = 0; i < count; ++i) {
    const oops_sum_segment& s = segs[i];
    SumJob whole{s.parts, s.out, s.count, s.n, s.part_stride, s.out_dtype, 1};
    if (s.count > kChunkParts) {
      const int64_t chunks = (s.count + kChunkParts - 1) / kChunkParts;
      float* sums = reinterpret_cast<float*>(ws);
      ws += align256((size_t)chunks * (size_t)s.n * 4);
      first.job[nfirst++] = SumJob{s.parts, sums, s.count, s.n, s.part_stride, OOPS_F32, 0};
      cols1 = s.n > cols1 ? s.n : cols1;
      chunks1 = chunks > chunks1 ? chunks : chunks1;
      whole = SumJob{sums, s.out, chunks, s.n, s.n, s.out_dtype, 1};
    }
    second.job[i] = whole;
    cols2 = s.n > cols2 ? s.n : cols2;
  }
  if (nfirst > 0 && cols1 > 0)
    if (hipError_t e = run(first, nfirst, cols1, chunks1, stream); e != hipSuccess) return e;
  if (count == 0 || cols2 == 0) return hipSuccess;
  return run(second, count, cols2, 1, stream);
}

}  // namespace oops
