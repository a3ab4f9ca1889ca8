/*
 * ygg_moe.h -- C ABI of the MI355X (gfx950) MoE-HLM expert layer.
 *
 * Library: yggdrasil_amd/lib/libygg_moe.so (hipcc, gfx950 code objects).
 *
 * Conventions (every entry point):
 *  - plain C types only; every pointer is a DEVICE pointer owned by the caller.
 *    The library keeps no state between calls, except the per-GPU scratch array
 *    of ygg_moe_forward_noalloc, and allocates nothing, with one exception:
 *    ygg_geom_matmul_f32, which keeps the reference launcher's signature (no
 *    workspace argument), takes its scratch from the stream-ordered pool
 *    (hipMallocAsync / hipFreeAsync on `stream`); callers that cannot allocate
 *    use ygg_geom_matmul_f32_ws with their own workspace;
 *  - expert row ranges (`offsets`, E + 1 ascending values from 0 to the rows
 *    the call names) are read on the device and trusted: the caller keeps them
 *    ascending and within the rows (the Python wrappers clamp them so);
 *  - the work is enqueued on `stream` (a hipStream_t; pass the caller's
 *    current stream, e.g. torch.cuda.current_stream().cuda_stream);
 *  - the return value is 0 on success and -1 on a rejected argument or a
 *    failed launch; ygg_last_error() then describes it (per host thread).
 *    Nothing aborts and nothing falls back silently.  (The reference's
 *    launchers return void and its Python wrappers swallow every exception,
 *    rune/ops/batched.py:329-343.)
 *  - multivectors are 8 contiguous values in the reference's blade order
 *    1, e1, e2, e3, e12, e13, e23, e123 (rune/types/multivector.py:7), except
 *    where an argument says "mask order" (1, e1, e2, e12, e3, e13, e23, e123,
 *    i.e. e3 and e12 exchanged), the layout the expert products consume.
 *  - dtype codes: 0 = fp32, 1 = bf16 (activations); weight formats:
 *    0 = fp32, 1 = bf16 (dual, sign-folded), 2 = int8 per-output-channel,
 *    3 = bf16 Pauli (the weights as 2x2 complex matrices; even d_in),
 *    4 = fp32 Pauli (fp32 layers on the fp32 MFMA units),
 *    5 = int8 Pauli (the entries of each weight's 2x2 complex matrix, int8 per
 *        output channel; bf16 decode layers of at most 128 tokens, d <= 128).
 *    activation codes: 0 none, 1 gelu, 2 relu, 3 sigmoid
 *    (holograph/models/hlm_block.py:28-32).
 */
#ifndef YGG_MOE_H
#define YGG_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* ygg_stream_t; /* == hipStream_t */

/* Message for the last non-zero status returned on this host thread. */
const char* ygg_last_error(void);
/* ABI version of the library (1). */
int ygg_version(void);

/* ---- operator boundary ---------------------------------------------------
 * out[m, n] = sum_k gp(a[m, k], b[k, n]); a: (M, K, 8), b: (K, N, 8),
 * out: (M, N, 8), fp32, blade order, weight operand on the left.
 * Replaces cl3_geom_matmul_launch (mjolnir/src/cuda/batch_ops.cu:389-401,
 * bound at rune/bindings/mjolnir_cuda_ffi.py:127-128,505-525) and
 * cl3_geom_matmul_flat (mjolnir/src/cpu/batch_ops.c:165-172, declared
 * mjolnir/include/cl3_ops.h:210, bound at rune/bindings/mjolnir_ffi.py:208-209).
 * Unlike those, it reports errors and takes the stream explicitly.  Computed as
 * one fp32 Pauli MFMA product (a as the weight of a single expert, the columns
 * of b as its rows); its scratch (the converted operands) is taken from the
 * device's stream-ordered pool for the call. */
int ygg_geom_matmul_f32(const float* a, const float* b, float* out, int M, int K, int N, ygg_stream_t stream);
/* The same with the caller's workspace of at least
 * ygg_geom_matmul_f32_workspace_bytes(M, K, N) bytes (no allocation). */
size_t ygg_geom_matmul_f32_workspace_bytes(int M, int K, int N);
int ygg_geom_matmul_f32_ws(const float* a, const float* b, float* out, int M, int K, int N, void* workspace,
                           size_t workspace_bytes, ygg_stream_t stream);

/* ---- router --------------------------------------------------------------
 * Grade-energy logits of CliffordRouter (holograph/layers/clifford_router.py:
 * 54-90): energy[t, g] = sum over d and the blades of grade g of x^2,
 * logits[t, e] = sum_g energy[t, g] / (sum energy + 1e-12) * W_r[e, g] + b_r[e].
 * x: (N, d, 8) of x_dtype; router_w (E, 4), router_b (E); logits (N, E);
 * energy (N, 4) or NULL. */
/* Router of the CliffordLinear-head kind (hlm.py:109,141-145; the TinyHLMMoE
 * layer of the reference's config 1): logits (N, E) = scalar part of
 * CliffordLinear(d -> E) with weights head_w (E, d, 8) fp32 blade order and no
 * bias, in the fp32 order of clifford_linear.py:101-123 (bit-exact). */
int ygg_router_head_logits(const void* x, int x_dtype, int N, int d, const float* head_w, int E, float* logits,
                           ygg_stream_t stream);

int ygg_router_energy_logits(const void* x, int x_dtype, int N, int d, const float* router_w,
                             const float* router_b, int E, float* logits, float* energy, ygg_stream_t stream);

/* Workspace bytes needed by ygg_route (and ygg_route_energy, ygg_route_pauli_rows). */
size_t ygg_route_workspace_bytes(int N, int E, int k);

/* Softmax, top-k and the expert counting sort.
 * Replaces clifford_router.py:18-21,93-104 and the slot grouping of
 * hlm_block.py:165-177.  logits (N, E) fp32, E <= 64, k <= 8.
 * Outputs: topk_idx (N, k) -- slot 0 most probable, equal probabilities
 *   ordered by lower expert index (the reference's ascending argsort order
 *   is reversed, clifford_router.py:97); topk_w (N, k) renormalised
 *   (sum + 1e-12, summed from the least probable slot); counts (E);
 *   offsets (E + 1, exclusive scan); perm (N*k): token of each expert-grouped
 *   row, ascending token order within an expert; slot_pos (N*k): the row of
 *   slot (t, s).  Deterministic; bit-exact integer outputs. */
int ygg_route(const float* logits, int N, int E, int k, int32_t* topk_idx, float* topk_w, int32_t* counts,
              int32_t* offsets, int32_t* perm, int32_t* slot_pos, void* workspace, size_t workspace_bytes,
              ygg_stream_t stream);

/* ygg_route and, in the same launches, the conversion of x (N, d, 8) to Pauli rows
 * (x_dtype 1: bf16 blade rows -> bf16 Pauli half-rows as ygg_pauli_rows_from_blade
 * writes them, d even; 0: fp32 -> fp32 Pauli rows as ygg_pauli_rows_from_blade_f32):
 * the first launches of ygg_moe_forward for weight formats 3 and 4, with their
 * outputs.  Replaces clifford_router.py:18-21,93-104 and hlm_block.py:165-177 as
 * ygg_route does; the conversion has no counterpart in the reference (its
 * CliffordLinear reads blade rows, clifford_linear.py:101-123). */
int ygg_route_pauli_rows(const float* logits, int N, int E, int k, const void* x, int x_dtype, int d,
                         int32_t* topk_idx, float* topk_w, int32_t* counts, int32_t* offsets, int32_t* perm,
                         int32_t* slot_pos, void* x_pauli, void* workspace, size_t workspace_bytes,
                         ygg_stream_t stream);

/* CliffordRouter.forward end to end (holograph/layers/clifford_router.py:54-104)
 * plus the slot grouping of hlm_block.py:165-177: the grade-energy logits of
 * ygg_router_energy_logits followed by ygg_route, with the same outputs.  Up to
 * 1024 tokens this is a single launch and logits_scratch is not touched; beyond,
 * logits_scratch (N x E fp32) and the ygg_route workspace carry the logits. */
int ygg_route_energy(const void* x, int x_dtype, int N, int d, const float* router_w, const float* router_b, int E,
                     int k, int32_t* topk_idx, float* topk_w, int32_t* counts, int32_t* offsets, int32_t* perm,
                     int32_t* slot_pos, float* logits_scratch, void* workspace, size_t workspace_bytes,
                     ygg_stream_t stream);

/* ---- dispatch / combine ----------------------------------------------------
 * x_sorted[slot_pos[t, s]] = x[t]  (rows of d multivectors, dtype 0/1);
 * to_mask_order != 0 stores the rows in mask order.
 * Replaces expert_input = flat_x[token_ids] (hlm_block.py:178). */
int ygg_dispatch(const void* x, int dtype, int N, int k, int d, const int32_t* slot_pos, void* x_sorted,
                 int to_mask_order, ygg_stream_t stream);

/* out[t] = (residual[t] +) sum over the token's slots in ascending expert
 * order of topk_w[t, s] * y_sorted[slot_pos[t, s]], each product rounded
 * before its add.  y_mask_order != 0: y rows are in mask order (out is
 * always blade order).  residual may be NULL.
 * Replaces weighted = w * y; np.add.at(output, token_ids, weighted)
 * (hlm_block.py:180-181) and the residual add x + ffn_out (hlm_block.py:151). */
int ygg_combine(const void* y_sorted, int y_dtype, int y_mask_order, int N, int k, int d, const int32_t* topk_idx,
                const float* topk_w, const int32_t* slot_pos, const void* residual, void* out, int out_dtype,
                ygg_stream_t stream);

/* ---- grouped CliffordLinear expert products --------------------------------
 * Bytes of the prepared weights for E experts of a CliffordLinear d_in -> d_out. */
size_t ygg_prepared_weight_bytes(int E, int d_out, int d_in, int format);

/* Prepare expert weights W (E, d_out, d_in, 8) fp32 blade order -- the
 * reference's CliffordLinear.weight layout (clifford_linear.py:95-96) stacked
 * over experts -- into `format`.  int8: scales (E, d_out) fp32 are written,
 * s = max(absmax over (d_in, 8), 1e-12) / 127, q = clip(rint(w / s), -127, 127)
 * (conventions of bifrost/quantization/grade_quantize.py:85-117,198-203).
 * Format 5 applies the same conventions to the eight real entries of each
 * weight's 2x2 complex matrix, M00 = (s + v3) + i (t + b12), M01 = (v1 - b13) +
 * i (b23 - v2), M10 = (v1 + b13) + i (b23 + v2), M11 = (s - v3) + i (t - b12),
 * in float64. */
int ygg_prepare_weights(const float* W, int E, int d_out, int d_in, int format, void* out, float* scales,
                        ygg_stream_t stream);

/* Bias (E, d_out, 8) blade order -> mask order fp32 (clifford_linear.py:99). */
int ygg_prepare_bias(const float* b, int E, int d_out, float* out, ygg_stream_t stream);

/* For every expert e, rows [offsets[e], offsets[e+1]) of x (P_max >= offsets[E]
 * rows of d_in multivectors, mask order; fp32 for format 0, bf16 otherwise):
 *   y[m, j] = act( sum_i W_e[j, i] * x[m, i] + b_e[j] )
 * act is the grade-wise activation (holograph/layers/activations.py:15-128).
 * y: rows of d_out multivectors, fp32 (format 0) or y_dtype, blade order if
 * y_blade_order else mask order.  bias: prepared (mask order) or NULL.
 * Replaces CliffordLinear.forward (clifford_linear.py:101-123) of every
 * expert inside CliffordFFN.forward (hlm_block.py:55-61). */
int ygg_grouped_clifford_linear(const void* x, int P_max, const void* w_prepared, int format, const float* scales,
                                const float* bias_prepared, const int32_t* offsets, int E, int d_in, int d_out,
                                int act, void* y, int y_dtype, int y_blade_order, ygg_stream_t stream);

/* The same products with weights in format 3, computed as complex GEMMs:
 * Cl(3,0) is the algebra of 2x2 complex matrices, so CliffordLinear is a
 * complex contraction with 32 real multiply-adds per multivector pair.
 * x_layout 0: x holds blade-order bf16 rows (N, d_in, 8) and row r of the
 *   product reads x[gather[r]] (gather NULL: x[r]) -- the dispatch copy of
 *   hlm_block.py:178 fused into the product;
 * x_layout 1: x holds "Pauli half-rows" (rows, 2, d_in, 4) bf16, the layout
 *   this call writes for y_layout 0 (see ygg_pauli_rows_from_blade); row r of
 *   the product reads x[gather[r]] (gather NULL: x[r]).
 * x_rows: the rows x holds (N above, or `rows`); without a gather at least
 *   P_max.  A gather index at or past x_rows reads a zero row.
 * y_layout 0: Pauli half-rows (P, 2, d_out, 4) bf16 (d_out even);
 * y_layout 1: blade-order rows (P, d_out, 8) of y_dtype (0 fp32, 1 bf16).
 * bias: prepared with ygg_prepare_bias (mask order) or NULL.  act as above.
 * x (x_rows * d_in * 16 bytes) and one expert's prepared weights must each be
 * smaller than 2 GiB; larger calls are rejected (-1).
 * Replaces CliffordLinear.forward (clifford_linear.py:101-123) of every
 * expert, with the activation (activations.py:15-128) fused. */
int ygg_pauli_grouped_linear(const void* x, int x_layout, int x_rows, const int32_t* gather, int P_max,
                             const void* w_prepared,
                             const float* bias_prepared, const int32_t* offsets, int E, int d_in, int d_out, int act,
                             void* y, int y_layout, int y_dtype, ygg_stream_t stream);

/* Blade-order bf16 rows (rows, d, 8) -> Pauli half-rows (rows, 2, d, 4) bf16;
 * d even.  Conversion helper for callers of ygg_pauli_grouped_linear. */
int ygg_pauli_rows_from_blade(const void* x, int rows, int d, void* out, ygg_stream_t stream);

/* fp32 products with weights in format 4 (v_mfma_f32_32x32x2_f32):
 * x holds fp32 "Pauli rows" (rows, d_in, 2, 2, 2) -- see
 * ygg_pauli_rows_from_blade_f32 -- and row r of the product reads
 * x[gather[r]] (gather NULL: x[r]).  y_layout 0: Pauli rows
 * (P, d_out, 2, 2, 2) fp32; 1: blade-order fp32 rows (P, d_out, 8).
 * bias prepared (mask order) or NULL; act as above.  Replaces
 * CliffordLinear.forward (clifford_linear.py:101-123) of every expert, with
 * the activation (activations.py:15-128) fused, for fp32 layers. */
int ygg_pauli_grouped_linear_f32(const float* x, const int32_t* gather, int P_max, const float* w_prepared,
                                 const float* bias_prepared, const int32_t* offsets, int E, int d_in, int d_out,
                                 int act, float* y, int y_layout, ygg_stream_t stream);

/* Blade-order fp32 rows (rows, d, 8) -> fp32 Pauli rows (rows, d, 2, 2, 2): element
 * [m][i][b][k][c] is the real (k = 0) or imaginary (k = 1) part of entry (c, b) of
 * multivector x[m][i] as a 2x2 complex matrix. */
int ygg_pauli_rows_from_blade_f32(const float* x, int rows, int d, float* out, ygg_stream_t stream);

/* ---- the whole layer ---------------------------------------------------------
 * Workspace bytes of ygg_moe_forward for activation dtype and weight format. */
size_t ygg_moe_workspace_bytes(int N, int d, int F, int E, int k, int dtype, int w_format);

/* HLMBlock._moe_forward (hlm_block.py:154-183): x (N, d, 8) of dtype ->
 * out (N, d, 8) of dtype (+ residual if not NULL).  logits (N, E) or NULL
 * (then router_w/router_b give the grade-energy logits).  Expert weights
 * prepared with ygg_prepare_weights (format 0 or 4 for fp32, 1, 2, 3 or 5 for bf16;
 * format 3 gathers the token rows inside the up projection; format 5 runs the
 * routing, both products and the activation in one launch and takes N <= 128,
 * d <= 128),
 * biases prepared with ygg_prepare_bias or NULL.  topk_idx/topk_w/counts/
 * offsets as in ygg_route. */
int ygg_moe_forward(const void* x, int dtype, int N, int d, int F, int E, int k, int act, const float* logits,
                    const float* router_w, const float* router_b, const void* w_up, const float* s_up,
                    const float* b_up, const void* w_down, const float* s_down, const float* b_down, int w_format,
                    const void* residual, void* out, int32_t* topk_idx, float* topk_w, int32_t* counts,
                    int32_t* offsets, void* workspace, size_t workspace_bytes, ygg_stream_t stream);

/* Bytes of device scratch the library holds per GPU for ygg_moe_forward_noalloc. */
#define YGG_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* ygg_moe_forward without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference: its launchers allocate per
 * call (rune/bindings/mjolnir_cuda_ffi.py:527-542).  The scratch is a device array
 * the library keeps on each GPU it runs on (YGG_NOALLOC_SCRATCH_BYTES, held until
 * the process ends); calls whose ygg_moe_workspace_bytes exceeds it are rejected
 * (-1).  The call allocates nothing; `stream` must belong to the current device.
 * Calls on one GPU share the scratch, so calls that overlap on one GPU (two
 * streams, or two host threads) race; calls in stream order do not.  Outputs are
 * those of ygg_moe_forward on the same arguments. */
int ygg_moe_forward_noalloc(const void* x, int dtype, int N, int d, int F, int E, int k, int act, const float* logits,
                            const float* router_w, const float* router_b, const void* w_up, const float* s_up,
                            const float* b_up, const void* w_down, const float* s_down, const float* b_down,
                            int w_format, const void* residual, void* out, int32_t* topk_idx, float* topk_w,
                            int32_t* counts, int32_t* offsets, ygg_stream_t stream);

/* ---- backward (fp32) ---------------------------------------------------------------
 * The reference has no MoE backward (hlm_block.py:202-206); these follow
 * CliffordLinear.backward (holograph/layers/clifford_linear.py:125-163) and
 * the activations' backward (holograph/layers/activations.py:135-287).
 *
 * W_adj (E, d_in, d_out, 8) = reverse of W (E, d_out, d_in, 8) with the two
 * channel axes exchanged: the weights whose forward product is grad_x. */
int ygg_adjoint_weights_f32(const float* W, int E, int d_out, int d_in, float* W_adj, ygg_stream_t stream);

/* dW[e, j, i] = sum over rows r of expert e (offsets) of dy[r, j] ~a[src, i],
 * src = gather[r] or r; db[e, j] = sum dy[r, j] when db is not NULL.  dy
 * (rows, d_out, 8), a (.., d_in, 8), dW (E, d_out, d_in, 8): fp32 blade order. */
int ygg_grouped_weight_grad_f32(const float* dy, const float* a, const int32_t* gather, const int32_t* offsets, int E,
                                int d_in, int d_out, float* dW, float* db, ygg_stream_t stream);

/* The same gradients on the fp32 MFMA units, from fp32 Pauli rows (the layout of
 * ygg_pauli_rows_from_blade_f32) of dy (P_max rows, d_out) and a (d_in): each
 * expert's rows are cut into chunks whose partial sums go to `workspace`
 * (ygg_grouped_weight_grad_pauli_f32_workspace_bytes) and are added in chunk
 * order, so results do not depend on scheduling.  dW and db as above, blade
 * order.  CliffordLinear.backward's weight and bias gradients
 * (clifford_linear.py:125-163) for every expert at once. */
size_t ygg_grouped_weight_grad_pauli_f32_workspace_bytes(int P_max, int E, int d_in, int d_out);
int ygg_grouped_weight_grad_pauli_f32(const float* dy_pauli, const float* a_pauli, const int32_t* gather,
                                      const int32_t* offsets, int P_max, int E, int d_in, int d_out, float* dW,
                                      float* db, void* workspace, size_t workspace_bytes, ygg_stream_t stream);

/* Gradient w.r.t. the input h of a grade-wise activation (act as in
 * ygg_grouped_clifford_linear) given grad_out; n_mv multivectors, fp32 blade
 * order; grad_in may alias grad_out. */
int ygg_activation_backward(const float* h, const float* grad_out, size_t n_mv, int act, float* grad_in,
                            ygg_stream_t stream);

/* Workspace bytes of ygg_moe_backward. */
size_t ygg_moe_backward_workspace_bytes(int N, int d, int F, int E, int k);

/* Backward of ygg_moe_forward for fp32 layers with fp32 Pauli weights (format
 * 4): the routing and the activations are recomputed from x and the same
 * logits / router parameters the forward took.  w_*_adj are the format-4
 * preparation of ygg_adjoint_weights_f32's output; b_up, b_down prepared
 * biases or NULL; residual: the forward added x to its output.  Writes dx
 * (N, d, 8), dw_up (E, F, d, 8), dw_down (E, d, F, 8) (blade order), db_up
 * (E, F, 8), db_down (E, d, 8) and dtopk_w (N, k, the gradient of the routing
 * weights, slots as ygg_route) when not NULL.  h_pre_saved: the rows
 * ygg_moe_forward_train kept, or NULL to recompute them.  No gradient flows into
 * the router. */
int ygg_moe_backward(const float* x, int N, int d, int F, int E, int k, int act, const float* logits,
                     const float* router_w, const float* router_b, const float* w_up, const float* w_up_adj,
                     const float* b_up, const float* w_down, const float* w_down_adj, const float* b_down,
                     int residual, const float* dout, const float* h_pre_saved, float* dx, float* dw_up,
                     float* db_up, float* dw_down, float* db_down, float* dtopk_w, void* workspace,
                     size_t workspace_bytes, ygg_stream_t stream);

/* The forward of a training step: ygg_moe_forward for fp32 layers with fp32
 * Pauli weights (format 4), which also writes h_pre (N k, F, 8) fp32 blade
 * order, the up product's expert-grouped rows before the activation.  Passed
 * to ygg_moe_backward as h_pre_saved (with the same x and routing inputs), it
 * spares the backward the recompute of that product. */
int ygg_moe_forward_train(const float* x, int N, int d, int F, int E, int k, int act, const float* logits,
                          const float* router_w, const float* router_b, const float* w_up, const float* b_up,
                          const float* w_down, const float* b_down, const float* residual, float* out,
                          int32_t* topk_idx, float* topk_w, int32_t* counts, int32_t* offsets, float* h_pre,
                          void* workspace, size_t workspace_bytes, ygg_stream_t stream);

/* ---- weight import: grade-aware quantization -----------------------------------
 * quantize_multivector / dequantize_multivector
 * (bifrost/quantization/grade_quantize.py:86-118,153-238) on T tensors of
 * mv_per_tensor multivectors each (fp32, blade order; e.g. T experts of
 * (d_out, d_in) weights): per tensor and grade g a bit width grade_bits[g] in
 * [2, 16] (host array of 4), a scale and, unless symmetric, a zero point, all
 * in float64 as the reference.  Writes scales (T, 4) fp64 and zero_points
 * (T, 4) int32; codes (T * mv_per_tensor * 8) int16 and dequant (same count,
 * (q - zp) * scale rounded to fp32) when not NULL. */
int ygg_grade_quantize(const float* W, int T, size_t mv_per_tensor, const int32_t* grade_bits, int symmetric,
                       int16_t* codes, double* scales, int32_t* zero_points, float* dequant, ygg_stream_t stream);

/* ---- the pre-norm and the FFN half of the block ------------------------------
 * CliffordLayerNorm.forward (holograph/layers/normalization.py:44-67):
 * y = gamma x_hat + beta with x_hat = x / sqrt(mean_i |x_i|^2 + 2 eps), the mean
 * over the d multivectors of each token and the product gamma x_hat the
 * geometric product with gamma on the left.  x (N, d, 8) of x_dtype (f32 or
 * bf16), gamma and beta (d, 8) fp32, y (N, d, 8) of y_dtype; eps is the
 * reference's Python float (default 1e-6).  d <= 4096; y must not alias x. */
int ygg_clifford_layer_norm(const void* x, int x_dtype, int N, int d, const float* gamma, const float* beta,
                            double eps, void* y, int y_dtype, ygg_stream_t stream);

/* Workspace bytes of ygg_moe_block_ffn. */
size_t ygg_moe_block_ffn_workspace_bytes(int N, int d, int F, int E, int k, int dtype, int w_format);

/* The FFN half of HLMBlock.forward (holograph/models/hlm_block.py:144-151):
 * out = x + moe(ffn_norm(x)).  The router sees the normed tokens, as the
 * reference's _moe_forward does.  Arguments as in ygg_moe_forward, with the
 * norm's gamma, beta and eps in place of the residual; out must not alias x. */
int ygg_moe_block_ffn(const void* x, int dtype, int N, int d, int F, int E, int k, int act, const float* norm_gamma,
                      const float* norm_beta, double norm_eps, const float* logits, const float* router_w,
                      const float* router_b, const void* w_up, const float* s_up, const float* b_up,
                      const void* w_down, const float* s_down, const float* b_down, int w_format, void* out,
                      int32_t* topk_idx, float* topk_w, int32_t* counts, int32_t* offsets, void* workspace,
                      size_t workspace_bytes, ygg_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* YGG_MOE_H */
