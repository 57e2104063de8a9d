// Launcher of the float32 partial-sum kernel (reduce.hip).
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/oops_amd.h"

namespace oops {

// bytes of float32 chunk sums the arrays with many rows need
size_t sum_partials_workspace_bytes(const oops_sum_segment* segs, int count);
// segs: count (<= OOPS_SUM_MAX_SEGMENTS) validated descriptors; workspace: at least
// sum_partials_workspace_bytes(segs, count) bytes, 256-byte aligned
hipError_t launch_sum_partials(const oops_sum_segment* segs, int count, void* workspace, hipStream_t stream);

}  // namespace oops
