// Triangle multiplicative update and row LayerNorm: launchers behind the
// oops_layer_norm_* and oops_trimul_* C entry points.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/oops_amd.h"

namespace oops {

hipError_t launch_layer_norm_rows_forward(const oops_row_norm_geometry& g, const void* x, const float* weight,
                                          const float* bias, void* y, float* mean, float* rstd, hipStream_t stream);
hipError_t launch_layer_norm_rows_backward(const oops_row_norm_geometry& g, const void* x, const float* weight,
                                           const float* mean, const float* rstd, const void* grad_y, void* grad_x,
                                           float* grad_weight_parts, float* grad_bias_parts, hipStream_t stream);
int64_t layer_norm_rows_parts(const oops_row_norm_geometry& g);

hipError_t launch_trimul_factors(const oops_trimul_geometry& g, const void* normalized, const void* weight,
                                 const float* bias, const void* mask, void* factors, const void* grad_factors,
                                 void* grad_projection, float* grad_mask_parts, float* grad_bias_parts,
                                 hipStream_t stream);
int64_t trimul_mask_parts(const oops_trimul_geometry& g);
int64_t trimul_bias_parts(const oops_trimul_geometry& g);

hipError_t launch_trimul_output_norm_forward(const oops_trimul_geometry& g, const void* combined, const float* weight,
                                             const float* bias, void* normalized, float* mean, float* rstd,
                                             hipStream_t stream);
hipError_t launch_trimul_output_norm_backward(const oops_trimul_geometry& g, const void* combined,
                                              const float* weight, const float* mean, const float* rstd,
                                              const void* grad_normalized, void* grad_combined,
                                              float* grad_weight_parts, float* grad_bias_parts, hipStream_t stream);
int64_t trimul_output_norm_parts(const oops_trimul_geometry& g);

hipError_t launch_trimul_output(const oops_trimul_geometry& g, const void* normalized, const void* pair_normalized,
                                const void* output_weight, const void* gate_weight, const float* output_bias,
                                const float* gate_bias, void* out, const void* grad_out, void* grad_value,
                                void* grad_gate, hipStream_t stream);

// the output projection's gradient products for C = H = 128, 16-bit (oops_trimul_output_grad_products)
bool trimul_output_grad_supported(const oops_trimul_geometry& g);
int64_t trimul_output_grad_parts(const oops_trimul_geometry& g);
hipError_t launch_trimul_output_grad(const oops_trimul_geometry& g, const void* x, int64_t x_row, const void* w,
                                     int64_t w_row, const void* y, int64_t y_row, void* d, int64_t d_row,
                                     float* g_parts, float* s_parts, hipStream_t stream);

// float32 pairs (trimul_f32.hip): the same contracts on the exact float32 matrix core
hipError_t launch_trimul_factors_f32(const oops_trimul_geometry& g, const void* normalized, const void* weight,
                                     const float* bias, const void* mask, void* factors, const void* grad_factors,
                                     void* grad_projection, float* grad_mask_parts, float* grad_bias_parts,
                                     hipStream_t stream);
int64_t trimul_bias_parts_f32(const oops_trimul_geometry& g);
hipError_t launch_trimul_output_f32(const oops_trimul_geometry& g, const void* normalized,
                                    const void* pair_normalized, const void* output_weight, const void* gate_weight,
                                    const float* output_bias, const float* gate_bias, void* out, const void* grad_out,
                                    void* grad_value, void* grad_gate, hipStream_t stream);

}  // namespace oops
