/*
 * oops_amd — MI355X (gfx950) pair-biased attention, C ABI.
 *
 * One kernel family serves every layout of the reference's attention path:
 * dense triangle attention in the starting-node (row) and ending-node (column,
 * swapped pair axes) orientation, ragged NestedTensor batches, and MSA-row
 * pair-bias attention.  The caller describes each independent "sample" (one
 * dense batch element, one nested complex, one MSA prefix element) with one row
 * of an int64 geometry table; every attention problem of a sample is indexed by
 * (group g, head h) and attends Lq queries over Lk keys:
 *
 *   O[g,h,i,:] = sum_j softmax_j(scale * Q[g,h,i,:].K[g,h,j,:] + bias[g,h,i,j]
 *                                  masked where keep[g,i,j] == 0) * V[g,h,j,:]
 *
 * Element (g, h, i, d) of a Q/K/V/O/dO operand lives at
 *     base + off + g*s_g + h*s_h + i*s_i + d          (elements, d contiguous)
 * so the ending-node orientation is only a different (s_g, s_i) pair and is
 * never materialised transposed.  Strides of 0 broadcast.
 *
 * Reference interfaces replaced (paths relative to the OOps source tree):
 *   oops_attn_forward   <- _run_forward / _launch_forward + Triton _forward
 *                          (oops/attention/triangle/triton/generic.py:173-317,
 *                           oops/attention/triangle/triton/kernel.py:266) and
 *                          run_attention_forward
 *                          (oops/attention/flash/triton/generic.py:233)
 *   oops_attn_backward  <- _run_backward + Triton _backward_preprocess,
 *                          _backward_query, _backward_key_value,
 *                          _backward_shared_bias and the partials.sum(0)
 *                          (oops/attention/triangle/triton/generic.py:320-536,
 *                           oops/attention/triangle/triton/kernel.py:375-873) and
 *                          run_attention_backward
 *                          (oops/attention/flash/triton/generic.py:324-658)
 *   oops_attn_forward_workspace_bytes: no counterpart (see its declaration)
 *   oops_attn_backward_workspace_bytes <- the partial-slab sizing of
 *                          SharedBiasSplit (oops/attention/triangle/triton/schedule.py:124-141)
 *   the geometry table  <- the int64 sample table of
 *                          triangle_attention_sample_table / uniform_sample_table
 *                          (oops/attention/triangle/nested.py:60, triton/ops.py:44)
 *
 * Every entry point is stateless and re-entrant; work is enqueued on the HIP
 * stream passed in (NULL = legacy default stream) and nothing synchronises the
 * host, so calls are safe under stream capture.  Return value 0 = success,
 * otherwise an OOPS_E* code; oops_last_error() gives a thread-local message.
 */
#ifndef OOPS_AMD_H
#define OOPS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
#define OOPS_F32 0
#define OOPS_BF16 1
#define OOPS_F16 2

/* status codes */
#define OOPS_OK 0
#define OOPS_EINVAL 1     /* malformed geometry or unsupported combination */
#define OOPS_ELAUNCH 2    /* a HIP launch failed */
#define OOPS_EWORKSPACE 3 /* workspace missing or too small */

/* bias modes (table column OOPS_T_BIAS_MODE) */
#define OOPS_BIAS_NONE 0
#define OOPS_BIAS_FULL 1   /* one bias matrix per group: dBias = dS        */
#define OOPS_BIAS_SHARED 2 /* one bias matrix for all groups: dBias = sum_g dS */

/* backward phases (oops_attn_geometry.phases); 0 runs all of them.  Phases are
 * for timing single kernels.  A call whose phases leave out both DQ and DELTA
 * but keep DKV and DBIAS, on a geometry the fused dK/dV + dBias kernel serves,
 * reads the delta/LSE pack and the compact Q/dO copies that an earlier full
 * call's dQ kernel left in the SAME workspace (same geometry, inputs and
 * workspace pointer); with any other workspace its dK/dV/dBias are undefined. */
#define OOPS_PHASE_DELTA 1 /* delta = rowsum(O * dO)                 */
#define OOPS_PHASE_DQ 2    /* dQ and per-group dBias               */
#define OOPS_PHASE_DKV 4   /* dK and dV                            */
#define OOPS_PHASE_DBIAS 8 /* shared dBias (partials + reduction)  */

/* geometry table: OOPS_TABLE_WIDTH int64 columns per sample */
enum oops_table_column {
  OOPS_T_GROUPS = 0, /* G */
  OOPS_T_LEN_Q,      /* Lq */
  OOPS_T_LEN_K,      /* Lk */
  OOPS_T_Q_OFF, OOPS_T_Q_SG, OOPS_T_Q_SH, OOPS_T_Q_SI,     /* also dQ */
  OOPS_T_K_OFF, OOPS_T_K_SG, OOPS_T_K_SH, OOPS_T_K_SI,     /* also dK */
  OOPS_T_V_OFF, OOPS_T_V_SG, OOPS_T_V_SH, OOPS_T_V_SI,     /* also dV */
  OOPS_T_O_OFF, OOPS_T_O_SG, OOPS_T_O_SH, OOPS_T_O_SI,
  OOPS_T_DO_OFF, OOPS_T_DO_SG, OOPS_T_DO_SH, OOPS_T_DO_SI,
  OOPS_T_B_OFF, OOPS_T_B_SG, OOPS_T_B_SH, OOPS_T_B_SI,     /* bias, key stride 1 */
  OOPS_T_M_OFF, OOPS_T_M_SG, OOPS_T_M_SI,                  /* u8 keep-mask, key stride 1; -1 = none */
  OOPS_T_L_OFF,                                            /* f32 LSE/delta, [G][H][Lq] */
  OOPS_T_DB_OFF, OOPS_T_DB_SG, OOPS_T_DB_SH, OOPS_T_DB_SI, /* f32 dBias output */
  OOPS_T_BIAS_MODE,                                        /* OOPS_BIAS_* */
  OOPS_T_RESERVED0, OOPS_T_RESERVED1, OOPS_T_RESERVED2, OOPS_T_RESERVED3,
  OOPS_TABLE_WIDTH = 40
};

typedef struct oops_attn_geometry {
  int32_t dtype;       /* OOPS_F32 / OOPS_BF16 / OOPS_F16 for Q, K, V, O, dO */
  int32_t bias_dtype;  /* dtype of the bias: the Q dtype or OOPS_F32 */
  int32_t num_heads;   /* H */
  int32_t head_size;   /* D, 1..256 */
  int32_t num_samples; /* rows of the table */
  int32_t has_bias;    /* 0/1 */
  int32_t has_mask;    /* 0/1 */
  int32_t vec_ok;      /* 1 when every row of Q/K/V/O/dO/bias starts 16-byte aligned */
  float scale;         /* multiplies Q.K before the bias is added */
  int32_t phases;      /* backward kernels to run: OR of OOPS_PHASE_*, 0 = all */
  int32_t force_generic; /* testing: 1 skips the specialised fast kernels, 2 keeps them but
                            runs dK/dV and the shared dBias in separate kernels */
  const int64_t* table_host;   /* host copy, used for grid sizing */
  const int64_t* table_device; /* device copy, read by the kernels */
} oops_attn_geometry;

/* Forward: writes O (dtype) and LSE (f32, log2 units, [G][H][Lq] per sample).
 * out_lo (optional, NULL to skip; 16-bit dtypes) receives O - round(O) with
 * O's layout, which the backward uses for an exact delta = rowsum(O * dO),
 * as the reference does with its saved fp32 output (triton/ops.py:369-377). */
int oops_attn_forward(const oops_attn_geometry* geo, const void* q, const void* k, const void* v,
                      const uint8_t* mask, const void* bias, void* out, void* out_lo, float* lse,
                      void* workspace, size_t workspace_bytes, void* stream);

/* oops_attn_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  It
 * runs the same kernels; what oops_attn_forward keeps in the caller's
 * workspace (the fragment-major copy of a row-shared bias) goes to a static
 * device scratch array of OOPS_NOALLOC_SCRATCH_BYTES that the library holds
 * on every GPU it runs on until the process ends; the entry point calls no
 * allocator.  Geometries whose oops_attn_forward_workspace_bytes exceeds that
 * size return OOPS_EWORKSPACE.  All calls on one GPU share the array: calls
 * that overlap in time on one GPU (different streams, no ordering between
 * them) race on it and must be serialised by the caller. */
#define OOPS_NOALLOC_SCRATCH_BYTES 33554432
int oops_attn_forward_noalloc(const oops_attn_geometry* geo, const void* q, const void* k, const void* v,
                              const uint8_t* mask, const void* bias, void* out, void* out_lo, float* lse,
                              void* stream);

/* Bytes of device workspace oops_attn_forward needs for this geometry (0 when
 * none: workspace may then be NULL).  The forward uses it for a fragment-major
 * copy of a row-shared bias (H x Lq x Lk elements, padded to 32), which the
 * fast kernels read with contiguous loads; there is no counterpart in the
 * reference, whose kernels read the bias rows directly. */
size_t oops_attn_forward_workspace_bytes(const oops_attn_geometry* geo);

/* Bytes of device workspace oops_attn_backward needs for this geometry. */
size_t oops_attn_backward_workspace_bytes(const oops_attn_geometry* geo);

/* Backward: dq/dk/dv in dtype with the Q/K/V strides of the table; dbias f32
 * at the table's dBias offsets (may be NULL when no bias gradient is wanted;
 * any of dq/dk/dv may be NULL likewise).  workspace must be device memory of
 * at least oops_attn_backward_workspace_bytes(geo) bytes, 256-byte aligned
 * (delta, the partial dBias slabs of a row-shared bias and, as in the forward,
 * the fragment-major bias copy). */
int oops_attn_backward(const oops_attn_geometry* geo, const void* q, const void* k, const void* v,
                       const uint8_t* mask, const void* bias, const void* out, const void* out_lo,
                       const float* lse, const void* dout, void* dq, void* dk, void* dv, float* dbias, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ---- gated output stage: gated = sigmoid(single . W^T) (*) attention ----
 *
 * One row per query token over all prefixes; gate channel n = h * D + d.
 * single [rows][C] (channels contiguous, row stride s_row), W [H*D][C]
 * (row stride w_row), attention element (row, h, d) at
 *     b * a_sb + s * a_sg + t * a_st + h * a_sh + d * a_sd
 * with row = (b * groups + s) * tokens + t; gated, logits, grad and the two
 * gradients are [rows][H*D] row-major.  Rounding follows the reference: the
 * logits are rounded to dtype, the gate sigmoid(logits) is rounded to dtype
 * before the product.  The output projection and the weight/single
 * gradients are plain GEMMs left to the caller's BLAS.
 *
 * Reference interfaces replaced:
 *   oops_gate_projection_forward <- Triton _gate_projection_forward /
 *                          _gate_projection_inference and _launch_projection
 *                          (oops/attention/gate/triton/kernel.py:117-286,
 *                           oops/attention/gate/triton/generic.py:183-262)
 *   oops_gate_multiply_forward   <- Triton _gate_forward and
 *                          _attention_gate_multiply_forward_impl
 *                          (kernel.py:39-66, generic.py:71-100)
 *   oops_gate_multiply_backward  <- Triton _gate_backward and
 *                          _attention_gate_multiply_backward_impl
 *                          (kernel.py:69-114, generic.py:103-141) */
typedef struct oops_gate_geometry {
  int32_t dtype;    /* OOPS_F32 / OOPS_BF16 / OOPS_F16 of every operand */
  int32_t heads;    /* H */
  int32_t width;    /* D */
  int32_t channels; /* C (projection only) */
  int64_t rows;     /* tokens over all prefixes */
  int64_t tokens;   /* tokens per (batch, group) prefix */
  int64_t groups;   /* groups per batch element */
  int64_t a_sb, a_sg, a_st, a_sh, a_sd; /* attention strides in elements */
  int64_t s_row;    /* single row stride in elements */
  int64_t w_row;    /* weight row stride in elements */
} oops_gate_geometry;

/* Fused gate projection (16-bit dtypes; C a multiple of 8, D a multiple of
 * 16, a_sd = 1, 16-byte aligned rows): logits = single . W^T (MFMA, f32
 * accumulation) and gated.  logits may be NULL (inference). */
int oops_gate_projection_forward(const oops_gate_geometry* geo, const void* single, const void* weight,
                                 const void* attention, void* gated, void* logits, void* stream);

/* gated = round(sigmoid(logits)) * attention from precomputed logits (any dtype). */
int oops_gate_multiply_forward(const oops_gate_geometry* geo, const void* attention, const void* logits,
                               void* gated, void* stream);

/* grad_attention = grad * g and grad_logits = sigmoid'(logits) * grad * attention,
 * g = round(sigmoid(logits)), with the reference's roundings; either output may
 * be NULL. */
int oops_gate_multiply_backward(const oops_gate_geometry* geo, const void* attention, const void* logits,
                                const void* grad, void* grad_attention, void* grad_logits, void* stream);

/* ---- row LayerNorm: y = (x - mean) * rstd * weight + bias over `width` ----
 *
 * Replaces the reference's layer_norm forward/backward kernels
 * (oops/normalization/layer_norm/triton/backend.py, layer_norm_forward_into)
 * where the triangle multiplicative update normalizes its pair input
 * (oops/pair/triangle_multiplication/triton/generic.py:102-108).  Statistics
 * are float32 (biased variance); weight and bias are float32.  y rows are
 * `y_row` elements apart; the columns width..y_row-1 are written as zero, so a
 * padded y feeds 16-byte MFMA operand loads. */
typedef struct oops_row_norm_geometry {
  int32_t dtype; /* x and y: OOPS_F32 / OOPS_BF16 / OOPS_F16 */
  int32_t width; /* 1..8192 */
  int64_t rows;
  int64_t x_row; /* x row stride in elements */
  int64_t y_row; /* y row stride in elements (>= width) */
  float eps;
} oops_row_norm_geometry;

int oops_layer_norm_rows_forward(const oops_row_norm_geometry* geo, const void* x, const float* weight,
                                 const float* bias, void* y, float* mean, float* rstd, void* stream);
/* Rows of float32 weight/bias gradient partials the backward writes (sum them). */
size_t oops_layer_norm_rows_parts(const oops_row_norm_geometry* geo);
/* grad_x (rows of x_row) from grad_y (rows of y_row); weight/bias gradient
 * partials [parts][width] (either may be NULL). */
int oops_layer_norm_rows_backward(const oops_row_norm_geometry* geo, const void* x, const float* weight,
                                  const float* mean, const float* rstd, const void* grad_y, void* grad_x,
                                  float* grad_weight_parts, float* grad_bias_parts, void* stream);
/* The same backward with the affine gradients summed in the library: grad_weight and grad_bias receive
 * `width` float32 sums each (either may be NULL), added up in a fixed order (bit-identical on every call).
 * The partials and their chunk sums live in the caller's workspace of
 * oops_layer_norm_rows_backward_workspace_bytes bytes (256-byte aligned; NULL when both gradients are NULL).
 * Replaces the reference's backward with its affine reduction kernel
 * (oops/normalization/layer_norm/triton/kernel.py:100-163 and :236-268). */
size_t oops_layer_norm_rows_backward_workspace_bytes(const oops_row_norm_geometry* geo);
int oops_layer_norm_rows_backward_affine(const oops_row_norm_geometry* geo, const void* x, const float* weight,
                                         const float* mean, const float* rstd, const void* grad_y, void* grad_x,
                                         float* grad_weight, float* grad_bias, void* workspace, size_t ws_bytes,
                                         void* stream);

/* ---- triangle multiplicative update (oops/pair/triangle_multiplication) ----
 *
 * G groups of P pair cells, C pair channels, H hidden channels; R = G * P.
 * normalized pair xn [R][c_row] (LayerNorm of the pair, zero-padded to c_row,
 * a multiple of 8); W = [left value; left gate; right value; right gate]
 * [4H][c_row]; factors [2][G][H][P] (left, right), channel-major as the
 * contraction reads them; combined [G][H][P]; normalized combined rows
 * [R][h_row] (h_row a multiple of 8).  Projection biases and LayerNorm affine
 * parameters are float32, NULL where absent; the mask is float32 [R].
 *
 *   oops_trimul_factors_forward  <- _gated_projection_forward
 *       (triton/kernel.py:109-187, generic.py:351-407)
 *   oops_trimul_factors_backward <- _gated_projection_backward
 *       (kernel.py:190-364, generic.py:1022-1092)
 *   oops_trimul_output_norm_*    <- _channel_major_layer_norm and
 *       _layer_norm_transpose_backward (kernel.py:367-402, :550-628)
 *   oops_trimul_output_forward   <- _gated_output_forward (kernel.py:405-467)
 *   oops_trimul_output_backward  <- _gated_output_backward (kernel.py:470-547)
 * The contraction itself is a batched GEMM, as in the reference
 * (generic.py:505-543). */
typedef struct oops_trimul_geometry {
  int32_t dtype;    /* OOPS_BF16 / OOPS_F16 */
  int32_t channels; /* C */
  int32_t hidden;   /* H */
  int32_t has_mask;
  int64_t groups;    /* G */
  int64_t positions; /* P */
  int64_t c_row;     /* row stride of xn, W, W_gate and the gate gradients */
  int64_t h_row;     /* row stride of the normalized combined rows and W_out */
  float eps;         /* output LayerNorm epsilon */
} oops_trimul_geometry;

/* factors[f][g][h][p] = mask[r] * (xn W_v^T + b_v) * sigmoid(xn W_g^T + b_g). */
int oops_trimul_factors_forward(const oops_trimul_geometry* geo, const void* normalized, const void* weight,
                                const float* bias, const void* mask, void* factors, void* stream);
/* Rows of float32 mask-gradient partials the factor backward writes (sum them). */
size_t oops_trimul_mask_parts(const oops_trimul_geometry* geo);
/* Rows of float32 projection-bias-gradient partials the factor backward writes. */
size_t oops_trimul_bias_parts(const oops_trimul_geometry* geo);
/* Recomputes the projections and writes grad_projection [4H][R] (value and
 * gate logit gradients, W's row order), with a mask the mask-gradient
 * partials [mask_parts][R], and the projection-bias-gradient partials
 * [bias_parts][4H] (either partial pointer NULL to skip). */
int oops_trimul_factors_backward(const oops_trimul_geometry* geo, const void* normalized, const void* weight,
                                 const float* bias, const void* mask, const void* grad_factors,
                                 void* grad_projection, float* grad_mask_parts, float* grad_bias_parts,
                                 void* stream);
/* LayerNorm over H of combined[g][:][p] -> normalized rows [R][h_row]; mean, rstd [R]. */
int oops_trimul_output_norm_forward(const oops_trimul_geometry* geo, const void* combined, const float* weight,
                                    const float* bias, void* normalized, float* mean, float* rstd, void* stream);
size_t oops_trimul_output_norm_parts(const oops_trimul_geometry* geo);
/* grad_normalized rows [R][H] -> grad_combined [G][H][P]; affine partials [parts][H]. */
int oops_trimul_output_norm_backward(const oops_trimul_geometry* geo, const void* combined, const float* weight,
                                     const float* mean, const float* rstd, const void* grad_normalized,
                                     void* grad_combined, float* grad_weight_parts, float* grad_bias_parts,
                                     void* stream);
/* out [R][C] = (normalized W_out^T + b_out) * sigmoid(xn W_gate^T + b_gate);
 * W_out [C][h_row], W_gate [C][c_row]. */
int oops_trimul_output_forward(const oops_trimul_geometry* geo, const void* normalized, const void* pair_normalized,
                               const void* output_weight, const void* gate_weight, const float* output_bias,
                               const float* gate_bias, void* out, void* stream);
/* Recomputes both projections; grad_value = grad_out * sigmoid(gate) and
 * grad_gate = grad_out * value * sigmoid'(gate), rows [R][c_row] (padding zero). */
int oops_trimul_output_backward(const oops_trimul_geometry* geo, const void* normalized,
                                const void* pair_normalized, const void* output_weight, const void* gate_weight,
                                const float* output_bias, const float* gate_bias, const void* grad_out,
                                void* grad_value, void* grad_gate, void* stream);

/* ---- float32 partial sums -------------------------------------------------
 *
 * The backward kernels above write float32 partial sums (mask, bias and
 * LayerNorm affine gradients, per-chunk weight gradients) that still have to
 * be summed over their leading axis.  The reference sums its partials with
 * torch reductions (oops/pair/triangle_multiplication/triton/generic.py:824,
 * :1017-1018, :1092, :1115); this entry point sums up to
 * OOPS_SUM_MAX_SEGMENTS such arrays:
 *   out[j] = sum over p = 0 .. count-1 of parts[p * part_stride + j],  j < n,
 * in a fixed order (bit-identical on every call), rounded once to out_dtype.
 * Arrays of more than 256 rows are summed in two launches through the caller's
 * workspace (float32 chunk sums, 256-byte aligned, of
 * oops_sum_partials_workspace_bytes bytes; NULL when that is 0). */
#define OOPS_SUM_MAX_SEGMENTS 16
typedef struct oops_sum_segment {
  const float* parts;  /* count rows of n float32 values, part_stride elements apart */
  void* out;           /* n values of out_dtype */
  int64_t count;
  int64_t n;
  int64_t part_stride; /* >= n */
  int32_t out_dtype;   /* OOPS_F32 / OOPS_BF16 / OOPS_F16 */
  int32_t reserved;    /* 0 */
} oops_sum_segment;
size_t oops_sum_partials_workspace_bytes(const oops_sum_segment* segments, int32_t num_segments);
int oops_sum_partials(const oops_sum_segment* segments, int32_t num_segments, void* workspace,
                      size_t workspace_bytes, void* stream);

/* The products of the gated output's backward that share one operand X [R][128] (16-bit, C = H = 128):
 *   d = X W              W [128][128] (rows w_row apart) -> d [R][128] (rows d_row apart), the dtype
 *   g_parts: X^T Y       Y [R][128] (rows y_row apart)   -> float32 partials [parts][128][128]
 *   s_parts: column sums of X                            -> float32 partials [parts][128]
 * with parts = oops_trimul_output_grad_parts (0: the geometry is not served; use GEMMs).  With X = the
 * value gradient, W = W_out, Y = the normalized combined rows these are the normalized-rows gradient,
 * W_out's gradient and the output bias gradient; with X = the gate-logit gradient, W = W_gate, Y = xn the
 * pair-rows gradient through the gate, W_gate's gradient and the gate bias gradient.  They replace the
 * reference's bmm / matmul / _column_sums calls of the output backward
 * (triangle_multiplication/triton/generic.py:820-824, :842-856) and its fused LayerNorm input product. */
size_t oops_trimul_output_grad_parts(const oops_trimul_geometry* geo);
int oops_trimul_output_grad_products(const oops_trimul_geometry* geo, const void* x, int64_t x_row, const void* w,
                                     int64_t w_row, const void* y, int64_t y_row, void* d, int64_t d_row,
                                     float* g_parts, float* s_parts, void* stream);

/* Thread-local description of the last failure (empty string if none). */
const char* oops_last_error(void);

/* Library ABI version; bumped on any change to the table or geometry layout. */
int oops_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* OOPS_AMD_H */
