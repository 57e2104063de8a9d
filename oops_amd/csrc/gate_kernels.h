// Gated output stage: launchers behind the oops_gate_* C entry points.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/oops_amd.h"

namespace oops {

// True when the fused projection kernel serves this geometry and these pointers.
bool gate_projection_ok(const oops_gate_geometry& g, const void* single, const void* weight,
                        const void* attention, const void* gated, const void* logits);

hipError_t launch_gate_projection(const oops_gate_geometry& g, const void* single, const void* weight,
                                  const void* attention, void* gated, void* logits, hipStream_t stream);
hipError_t launch_gate_multiply_forward(const oops_gate_geometry& g, const void* attention, const void* logits,
                                        void* gated, hipStream_t stream);
hipError_t launch_gate_multiply_backward(const oops_gate_geometry& g, const void* attention, const void* logits,
                                         const void* grad, void* grad_attention, void* grad_logits,
                                         hipStream_t stream);

}  // namespace oops
