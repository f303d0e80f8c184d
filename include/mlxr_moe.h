/*
 * mlxr_moe.h -- C ABI of the MI355X (gfx950) sparse-MoE block.
 *
 * Drop-in boundary for mlxr-lm's MoE hot path.  The reference reaches MLX
 * through mlx-c (crates/mlxr-sys, bindgen of mlx.h); each entry point below
 * replaces one mlx-c call (or one Rust module method built from several),
 * cited as path:line under /root/reference.  Conventions, following mlx-c:
 *
 *   - Every function returns int: 0 = success (crates/mlxr/src/utils/mod.rs:
 *     18-19).  On failure nothing is enqueued and mlxr_moe_last_error()
 *     returns a description (thread-local, like the handler slot of
 *     crates/mlxr/src/error.rs:229-258).  Nothing is thrown across the ABI.
 *   - Arrays are caller-owned device pointers with explicit shapes (no
 *     mlx_array handles).  Optional arrays are NULL (mlx_array_new()).
 *     Optional ints use mlxr_moe_optional_int (mlx_optional_int,
 *     crates/mlxr/src/ops/quantization.rs:16-21).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = default stream)
 *     and the call returns without synchronising; the caller syncs, as with
 *     mlx_async_eval (crates/mlxr/src/transforms/mod.rs:65-83).
 *   - Scratch memory is a caller-provided device workspace whose size the
 *     matching *_workspace_size function returns; the library never
 *     allocates device memory in these calls.
 *   - Index values live on the device and are not read by the host.  An
 *     index outside its range leaves its row out of the computation and sets
 *     a device status word; mlxr_moe_workspace_status() reads it (and
 *     synchronises the stream).
 *
 * dtypes: MLXR_MOE_FLOAT32, MLXR_MOE_BFLOAT16 (bf16 as raw uint16 bits).
 * Quantisation: mode "affine" (or NULL), group_size 64 (32 and 128 also for
 * quantize/dequantize), bits 4 or 8 (2 also for quantize/dequantize).
 */
#ifndef MLXR_MOE_H
#define MLXR_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mlxr_moe_stream; /* hipStream_t */

enum { MLXR_MOE_FLOAT32 = 0, MLXR_MOE_BFLOAT16 = 1 };

/* mlx_optional_int (crates/mlxr/src/ops/quantization.rs:16-21) */
typedef struct {
  int32_t value;
  int32_t has_value;
} mlxr_moe_optional_int;

/* Last error of the calling thread ("" if none).  Replaces the error-handler
 * slot read by get_and_clear_last_mlx_error (crates/mlxr/src/error.rs:
 * 275-290); the string stays valid until the thread's next failing call. */
const char* mlxr_moe_last_error(void);

/* ABI version (major * 10000 + minor * 100 + patch). */
int mlxr_moe_version(void);

/* Quantise w [rows, cols] (f32 or bf16) to packed codes wq [rows,
 * cols*bits/32] and scales/biases [rows, cols/group_size] in w's dtype.
 * Replaces mlx_quantize as called by quantize_device
 * (crates/mlxr/src/ops/quantization.rs:47-70); defaults g64 / 4-bit
 * (quantization.rs:11-13). */
int mlxr_moe_quantize(const void* w, int w_dtype, int64_t rows, int64_t cols,
                      mlxr_moe_optional_int group_size,
                      mlxr_moe_optional_int bits, const char* mode,
                      uint32_t* wq, void* scales, void* biases,
                      mlxr_moe_stream stream);

/* out [rows, cols] (out_dtype) = code * scale + bias, evaluated as one fused
 * multiply-add rounded once.  Replaces mlx_dequantize as called by
 * dequantize_device (crates/mlxr/src/ops/quantization.rs:118-146).
 * biases are required for mode "affine". */
int mlxr_moe_dequantize(const uint32_t* wq, const void* scales,
                        const void* biases, int sb_dtype, int64_t rows,
                        int64_t cols, mlxr_moe_optional_int group_size,
                        mlxr_moe_optional_int bits, const char* mode,
                        void* out, int out_dtype, mlxr_moe_stream stream);

/* gather_qmm with transpose = true.  x bf16 [x_batch, M, K]; w [E, N,
 * K*bits/32]; scales/biases bf16 [E, N, K/group]; rhs_indices uint32 [B];
 * out bf16 [B, M, N]:
 *   out[b] = x[xb(b)] @ dequant(w[rhs_indices[b]])^T
 * xb(b) = lhs_indices[b] when given, else b / (B / x_batch) -- the
 * broadcast of x [..., T, 1, 1, K] against indices [..., T, top_k] in
 * SplitSwitchFfn::forward (crates/mlxr-lm/src/nn/switch.rs:417-442).
 * Replaces mlx_gather_qmm as called by gather_qmm_device
 * (crates/mlxr/src/ops/quantization.rs:171-221).  `sorted_indices` is the
 * reference's locality hint; rows are always grouped by expert here.
 * Requires N % 64 == 0, K % 64 == 0, group 64, bits 4 or 8. */
size_t mlxr_moe_gather_qmm_workspace_size(int64_t B, int64_t M,
                                          int64_t num_experts);
int mlxr_moe_gather_qmm(const void* x, int x_dtype, int64_t x_batch,
                        int64_t M, int64_t K, const uint32_t* w,
                        const void* scales, const void* biases, int sb_dtype,
                        int64_t num_experts, int64_t N,
                        const uint32_t* lhs_indices,
                        const uint32_t* rhs_indices, int64_t B, int transpose,
                        mlxr_moe_optional_int group_size,
                        mlxr_moe_optional_int bits, const char* mode,
                        int sorted_indices, void* out, int out_dtype,
                        void* workspace, size_t workspace_size,
                        mlxr_moe_stream stream);

/* gather_mm as SwitchLinear::apply calls it (crates/mlxr-lm/src/nn/
 * switch.rs:84-93: gather_mm(x, swap_axes(weight, -1, -2), None, indices,
 * sorted)): a bf16 [a_batch, M, K]; b bf16 stored [E, N, K] (the
 * SwitchLinear weight as it is; b_transposed must be 1); rhs_indices uint32
 * [B]; out bf16 [B, M, N]:
 *   out[b] = a[ab(b)] @ b[rhs_indices[b]]^T
 * with ab(b) as xb(b) of gather_qmm, f32 accumulation.  Replaces mlx_gather_mm
 * as called by gather_mm_device (crates/mlxr/src/ops/arithmetic.rs:
 * 1577-1613).  SwitchLinear's optional bias is not taken: every SwitchLinear
 * of the MoE blocks is built without one (crates/mlxr-lm/src/qwen3_5/text/
 * moe.rs:92-97, crates/mlxr-lm/src/gemma4/text/text.rs:679).  Requires
 * N % 64 == 0, K % 64 == 0, K <= 4096.  Same workspace as gather_qmm. */
size_t mlxr_moe_gather_mm_workspace_size(int64_t B, int64_t M,
                                         int64_t num_experts);
int mlxr_moe_gather_mm(const void* a, int a_dtype, int64_t a_batch, int64_t M,
                       int64_t K, const void* b, int b_dtype,
                       int64_t num_experts, int64_t N, int b_transposed,
                       const uint32_t* lhs_indices,
                       const uint32_t* rhs_indices, int64_t B,
                       int sorted_indices, void* out, int out_dtype,
                       void* workspace, size_t workspace_size,
                       mlxr_moe_stream stream);

/* Which numerics a gather_qmm (or a SplitSwitchFfn / shared-expert GEMM) of
 * `rows` flat rows over `num_experts` experts uses (no counterpart in the
 * reference, whose MLX backend makes the same kind of choice inside
 * mlx_gather_qmm): 1 = the M-tiled kernel, whose weight tiles are
 * dequantised to bf16 -- gather_mm(x, dequantize(w)^T), as the reference's
 * test states gather_qmm (crates/mlxr/src/ops/quantization.rs:344-421);
 * 0 = the streaming kernel, which keeps the dequantised weights in f32.
 * Both accumulate in f32.  Returns -1 for negative sizes. */
int mlxr_moe_gather_qmm_tiled(int64_t rows, int64_t num_experts);

/* The summation order of a router's logits for T tokens over d inputs and
 * `columns` logit columns (the experts, plus one when a shared-expert gate
 * rides in the same pass), for f32, bf16 and quantised routers alike (no
 * counterpart in the reference, whose MLX matmul picks its own order).
 * 1 = the matrix-core order, taken from 512 tokens when d is a multiple of
 * 256 and the logits make at least 192 tiles of 32 tokens x 32 columns: d
 * in four quarters, each a chain of fused multiply-adds over 16-element
 * chunks taken as j, j+8, j+1, j+9, ..., j+7, j+15, the quarters then
 * added in order.  0 = the lane order of the other kernels.  Both are f32
 * dot products of the same inputs (a quantised or bf16 router rounds the
 * sum to bf16 after); top-K can differ between them only where two logits
 * tie to within their last bits.  (Rows of x or weights off 16-byte
 * alignment take the lane order.)  Returns -1 for negative sizes. */
int mlxr_moe_router_matrix_order(int64_t T, int64_t d, int64_t columns);

/* Indices that partition each row of a [rows, n] f32 (axis = -1 or 1):
 * out[.., kth] holds the element of sorted rank kth, smaller before, larger
 * after (the full ascending order, ties by index, is returned).  kth in
 * [-n, n).  Replaces mlx_argpartition_axis (crates/mlxr/src/ops/sort.rs:
 * 211-226); invalid axis or kth fail like sort.rs:262-301 expects. */
int mlxr_moe_argpartition(const float* a, int64_t rows, int64_t n, int kth,
                          int axis, uint32_t* out, mlxr_moe_stream stream);

/* Row softmax of a [rows, n] f32 over axis -1, computed in f32 (`precise`
 * accepted for either value).  Replaces mlx_softmax_axis
 * (crates/mlxr/src/ops/arithmetic.rs:1298-1311). */
int mlxr_moe_softmax(const float* a, int64_t rows, int64_t n, int axis,
                     int precise, float* out, mlxr_moe_stream stream);

/* Router of Qwen35MoeBlock::forward (crates/mlxr-lm/src/qwen3_5/text/
 * moe.rs:122-138): logits = x @ gate_w^T (f32), softmax, top-K, weights
 * renormalised to sum 1.  x bf16 [T, d]; gate_w f32 [E, d]; topk_idx int32
 * [T, K] in descending logit order (ties to the lower id; the reference's
 * order inside the partition is undefined, sort.rs:188); topk_w f32
 * [T, K].  Workspace holds the [T, E] logits. */
size_t mlxr_moe_router_workspace_size(int64_t T, int64_t E);
int mlxr_moe_router_topk(const void* x, int64_t T, int64_t d,
                         const float* gate_w, int64_t E, int64_t K,
                         int32_t* topk_idx, float* topk_w, void* workspace,
                         size_t workspace_size, mlxr_moe_stream stream);

/* Stable sort of flat expert ids [n] by expert: the permutation of
 * gather_sort (crates/mlxr-lm/src/nn/switch.rs:499-512), order =
 * argsort(ids) into `sorted`, inv = argsort(order) into `inv`, plus
 * per-expert counts [E] and offsets [E+1]. */
size_t mlxr_moe_dispatch_workspace_size(int64_t n, int64_t E);
int mlxr_moe_dispatch(const int32_t* ids, int64_t n, int64_t E,
                      int32_t* counts, int32_t* offsets, int32_t* sorted,
                      int32_t* inv, void* workspace, size_t workspace_size,
                      mlxr_moe_stream stream);

/* out f32 [T, d] = sum_k w[t,k] * y[t,k,:] (+ shared_y[t,:] *
 * sigmoid(shared_logit[t])).  y bf16 [T, K, d]; shared_y bf16 [T, d] or
 * NULL.  Replaces combine_with_weights (crates/mlxr-lm/src/nn/switch.rs:
 * 223-234) and the shared branch of moe.rs:117-120,145. */
int mlxr_moe_combine(const void* y, const float* w, int64_t T, int64_t K,
                     int64_t d, const void* shared_y,
                     const float* shared_logit, float* out,
                     mlxr_moe_stream stream);

/* One QuantizedSwitchLinear (crates/mlxr-lm/src/nn/switch.rs:115-168) or
 * QuantizedLinear (num_experts = 1; crates/mlxr/src/layers/quantized.rs:
 * 214-379): weight u32 [E, output_dims, input_dims*bits/32], scales and
 * biases bf16 [E, output_dims, input_dims/group_size].
 * bits = 16 describes the unquantised form of the same MaybeQuantized slot
 * (crates/mlxr/src/quantization.rs:6-147): a dense SwitchLinear
 * (switch.rs:49-94, applied with gather_mm) or Linear, weight bf16
 * [E, output_dims, input_dims], scales and biases NULL, group_size
 * ignored.  The projections of one module share their bits. */
typedef struct {
  const uint32_t* weight;
  const void* scales;
  const void* biases;
  int64_t num_experts;
  int64_t output_dims;
  int64_t input_dims;
  int32_t group_size;
  int32_t bits;
} mlxr_moe_qlinear;

/* mlxr_moe_router_topk with the router as a QuantizedLinear
 * (crates/mlxr/src/layers/quantized.rs:356-373; gate: num_experts 1,
 * output_dims E, input_dims d, group 64, bits 4 or 8) or a bf16 Linear
 * (bits 16, crates/mlxr/src/layers/linear.rs:91-95): bf16 logits and
 * probabilities, top-K on the probabilities (descending, ties to the lower
 * id), bf16 weights returned as f32 values.  Same workspace as
 * mlxr_moe_router_topk. */
int mlxr_moe_router_topk_quantized(const void* x, int64_t T,
                                   const mlxr_moe_qlinear* gate, int64_t K,
                                   int32_t* topk_idx, float* topk_w,
                                   void* workspace, size_t workspace_size,
                                   mlxr_moe_stream stream);

/* SplitSwitchFfn<SwigluActivation> (crates/mlxr-lm/src/nn/switch.rs:
 * 366-491): gate_proj, up_proj [E, f, d], down_proj [E, d, f]. */
typedef struct {
  mlxr_moe_qlinear gate_proj;
  mlxr_moe_qlinear up_proj;
  mlxr_moe_qlinear down_proj;
} mlxr_moe_switch_glu;

/* SplitSwitchFfn::forward_with_combine (switch.rs:446-474): x bf16 [T, d],
 * indices int32 [T, K], weights f32 [T, K] -> out f32 [T, d]. */
size_t mlxr_moe_switch_glu_workspace_size(const mlxr_moe_switch_glu* ffn,
                                          int64_t T, int64_t K);
int mlxr_moe_switch_glu_forward(const mlxr_moe_switch_glu* ffn, const void* x,
                                int64_t T, const int32_t* indices,
                                const float* weights, int64_t K, float* out,
                                void* workspace, size_t workspace_size,
                                mlxr_moe_stream stream);

/* SplitSwitchFfn::forward (switch.rs:417-442): per-expert outputs
 * y bf16 [T, K, d] before the combine.  Same workspace size as
 * mlxr_moe_switch_glu_forward. */
int mlxr_moe_switch_glu_experts(const mlxr_moe_switch_glu* ffn, const void* x,
                                int64_t T, const int32_t* indices, int64_t K,
                                void* y, void* workspace,
                                size_t workspace_size, mlxr_moe_stream stream);

/* gemma4's Router (crates/mlxr-lm/src/gemma4/text/text.rs:568-665):
 * normed = fast::rms_norm(x, norm_weight, eps), where norm_weight = scale *
 * root_size (root_size = hidden_size^-1/2, folded into the scale once,
 * text.rs:626-637); scores = proj(normed), a bf16 Linear [E, D]
 * (proj_weight) or a QuantizedLinear (proj_q.weight set, 4 or 8 bits,
 * group 64); top-K of the scores (argpartition, text.rs:643-648:
 * descending, ties to the lower id); weights = softmax(top-K scores) *
 * per_expert_scale[top-K] (router_post, activations.rs:309-331).  bf16
 * throughout: x bf16 [T, D], norm_weight and per_expert_scale bf16,
 * topk_idx int32 [T, K], topk_w bf16 [T, K]. */
typedef struct {
  int64_t hidden_size;
  int64_t num_experts;
  int64_t top_k;
  float eps;
  const void* norm_weight;
  const void* proj_weight;
  mlxr_moe_qlinear proj_q;
  const void* per_expert_scale;
} mlxr_moe_gemma_router;
size_t mlxr_moe_gemma_router_workspace_size(const mlxr_moe_gemma_router* r,
                                            int64_t T);
int mlxr_moe_gemma_router_forward(const mlxr_moe_gemma_router* r,
                                  const void* x, int64_t T, int32_t* topk_idx,
                                  void* topk_w, void* workspace,
                                  size_t workspace_size,
                                  mlxr_moe_stream stream);

/* PackedSwitchFfn (crates/mlxr-lm/src/nn/switch.rs:236-335), the gemma4
 * expert layout: gate_up_proj [E, 2H, D] (split_sections at H: gate
 * channels first, switch.rs:305-307) and down_proj [E, D, H], with GeGLU
 * (gemma4's GemmaSwitchGlu = PackedSwitchFfn<GegluActivation>,
 * crates/mlxr-lm/src/gemma4/text/mod.rs:27; activations.rs:223-259) or
 * SwiGLU between them. */
enum { MLXR_MOE_ACT_SWIGLU = 0, MLXR_MOE_ACT_GEGLU = 1 };
typedef struct {
  mlxr_moe_qlinear gate_up_proj;
  mlxr_moe_qlinear down_proj;
  int32_t activation;
} mlxr_moe_packed_switch_glu;

/* PackedSwitchFfn::forward_with_combine (switch.rs:290-335): x bf16
 * [T, D], indices int32 [T, K], weights [T, K] f32 or bf16
 * (weights_dtype) -> out [T, D], f32 for f32 weights (bf16 x f32
 * promotes) and bf16 for bf16 weights (gemma4's router returns bf16). */
size_t mlxr_moe_packed_switch_glu_workspace_size(
    const mlxr_moe_packed_switch_glu* ffn, int64_t T, int64_t K);
int mlxr_moe_packed_switch_glu_forward(const mlxr_moe_packed_switch_glu* ffn,
                                       const void* x, int64_t T,
                                       const int32_t* indices,
                                       const void* weights, int weights_dtype,
                                       int64_t K, void* out, void* workspace,
                                       size_t workspace_size,
                                       mlxr_moe_stream stream);
/* PackedSwitchFfn::forward (switch.rs:290-315): per-expert outputs y bf16
 * [T, K, D].  Same workspace size. */
int mlxr_moe_packed_switch_glu_experts(const mlxr_moe_packed_switch_glu* ffn,
                                       const void* x, int64_t T,
                                       const int32_t* indices, int64_t K,
                                       void* y, void* workspace,
                                       size_t workspace_size,
                                       mlxr_moe_stream stream);

/* Qwen35MoeBlock (crates/mlxr-lm/src/qwen3_5/text/moe.rs:43-159):
 * f32 router gate_weight [E, d] with optional f32 gate_bias [E] (Linear
 * with bias = addmm, crates/mlxr/src/layers/linear.rs:91-95; the Qwen
 * checkpoints build it without, moe.rs:90-92); switch_mlp; optional shared
 * expert
 * (SwigluMlp, crates/mlxr-lm/src/nn/swiglu_mlp.rs:24-75, num_experts = 1)
 * with f32 shared_expert_gate_weight [1, d].  shared_expert_gate_weight ==
 * NULL means a plain SwitchGLU block without the shared branch.
 *
 * Quantised router (gate: MaybeQuantized<Linear> quantised, moe.rs:57,123
 * -> QuantizedLinear::forward, crates/mlxr/src/layers/quantized.rs:
 * 356-373; the shipped Qwen3.6 checkpoints quantise mlp.gate and
 * mlp.shared_expert_gate at 8 bits, group 64, moe.rs:255-284): set
 * gate_q.weight (num_experts 1, output_dims E, input_dims d, group 64, bits
 * 4 or 8) and leave gate_weight, gate_bias and shared_expert_gate_weight
 * NULL; the shared gate is then shared_expert_gate_q (output_dims 1, same
 * bits; weight NULL = no shared branch).  As in the reference with a bf16
 * router the block then computes in bf16: bf16 logits and probabilities
 * (the top-K selects on the probabilities, ties to the lower id), bf16
 * routing weights (returned in topk_w as f32 values) and a bf16 out.
 * An unquantised bf16 checkpoint's router is the same slot with bits 16
 * (bf16 Linears, scales and biases NULL), computed the same way.  Dense
 * bf16 experts (switch_mlp and shared projections with bits 16) run
 * gather_mm (SwitchLinear::apply, switch.rs:84-93) with f32 accumulation. */
typedef struct {
  int64_t hidden_size;
  int64_t num_experts;
  int64_t num_experts_per_tok;
  int64_t moe_intermediate_size;
  int64_t shared_expert_intermediate_size;
  const float* gate_weight;
  const float* gate_bias;
  mlxr_moe_switch_glu switch_mlp;
  mlxr_moe_qlinear shared_gate_proj;
  mlxr_moe_qlinear shared_up_proj;
  mlxr_moe_qlinear shared_down_proj;
  const float* shared_expert_gate_weight;
  mlxr_moe_qlinear gate_q;
  mlxr_moe_qlinear shared_expert_gate_q;
} mlxr_moe_block;

/* Qwen35MoeBlock::forward (moe.rs:116-146): x bf16 [T, d] -> out [T, d],
 * f32 with the f32 router, bf16 with a quantised one.  topk_idx [T, K] /
 * topk_w [T, K] optionally receive the routing (NULL to skip). */
size_t mlxr_moe_block_workspace_size(const mlxr_moe_block* block, int64_t T);
int mlxr_moe_block_forward(const mlxr_moe_block* block, const void* x,
                           int64_t T, void* out, int32_t* topk_idx,
                           float* topk_w, void* workspace,
                           size_t workspace_size, mlxr_moe_stream stream);

/* mlxr_moe_block_forward for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference (MLX allocates its
 * intermediates itself).  Same arguments, results and checks, without the
 * workspace: the scratch is a device array inside the library, one per GPU,
 * of mlxr_moe_noalloc_scratch_size() bytes (MLXR_MOE_NOALLOC_SCRATCH_BYTES),
 * held until the process ends.  A T whose block workspace
 * (mlxr_moe_block_workspace_size) exceeds it is rejected with an error.
 * Nothing is allocated.  Calls that overlap on one GPU share the array and
 * race: serialise them (one stream, or events).  The status word of the
 * last call is not readable through mlxr_moe_workspace_status.  The array's
 * device address is looked up once per device, by the first call there or
 * by mlxr_moe_noalloc_scratch_size() with that device current: call the
 * latter once per device before capturing the entry into a graph. */
#define MLXR_MOE_NOALLOC_SCRATCH_BYTES (32 * 1024 * 1024)
size_t mlxr_moe_noalloc_scratch_size(void);
int mlxr_moe_block_forward_noalloc(const mlxr_moe_block* block, const void* x,
                                   int64_t T, void* out, int32_t* topk_idx,
                                   float* topk_w, mlxr_moe_stream stream);

/* fast::rms_norm as RmsNorm::forward calls it (crates/mlxr/src/layers/
 * normalization.rs:272-276; gemma4's router, crates/mlxr-lm/src/gemma4/
 * text/text.rs:640): x bf16 [T, d], weight bf16 [d] -> out bf16 [T, d],
 *   out_j = bf16(w_j * bf16(x_j * r)),  r = 1 / sqrt(sum_j x_j^2 / d + eps)
 * (the normalised value in the input dtype, then the weight product, MLX's
 * rounding points; the sum of squares in a fixed 64-lane order).  d % 4 ==
 * 0, x and out 8-byte aligned. */
int mlxr_moe_rms_norm(const void* x, int64_t T, int64_t d, const void* weight,
                      float eps, void* out, mlxr_moe_stream stream);

/* The MoE half of a Qwen3.5 / Qwen3.6 decoder layer (DecoderLayer::forward,
 * crates/mlxr-lm/src/qwen3_5/text/layer.rs:134-138):
 *   out = h + block(rms_norm(h, norm_weight, eps))
 * h bf16 [T, d] (the residual stream after attention); norm_weight bf16 [d],
 * post_attention_layernorm.weight as the model holds it (after the loader's
 * +1.0 shift of non-mlx-format checkpoints, crates/mlxr-lm/src/qwen3_5/text/
 * weights.rs:147-165); eps = rms_norm_eps.  out as mlxr_moe_block_forward's:
 * f32 with the f32 router (bf16 h + f32 promotes), bf16 with a bf16 router
 * (bf16(h + mlp_out)).  The norm is one kernel before the block and the
 * residual add rides in the block's combine.  Workspace:
 * mlxr_moe_block_residual_workspace_size (the block's plus the normed rows);
 * its status word is the block's (mlxr_moe_workspace_status). */
size_t mlxr_moe_block_residual_workspace_size(const mlxr_moe_block* block,
                                              int64_t T);
int mlxr_moe_block_forward_residual(const mlxr_moe_block* block,
                                    const void* norm_weight, float eps,
                                    const void* h, int64_t T, void* out,
                                    int32_t* topk_idx, float* topk_w,
                                    void* workspace, size_t workspace_size,
                                    mlxr_moe_stream stream);

/* Device status word of a workspace used by gather_qmm / dispatch /
 * switch_glu / block calls: 0 = all indices in range, 1 = some index out of
 * range.  Synchronises `stream`.  Returns the status or -1 on error. */
int mlxr_moe_workspace_status(const void* workspace, size_t workspace_size,
                              mlxr_moe_stream stream);

/* Kernel timing (no counterpart in the reference, whose benches time whole
 * models with criterion, crates/mlxr-lm/benches/lm_decode.rs): while
 * `kernel` is armed, each launch of that kernel is bracketed by HIP events
 * on the stream it is launched on.  Names: "router_logits", "router_topk",
 * "dispatch", "qgemm_gated", "qgemm_down", "combine", the shared
 * expert's GEMMs "shared_gated", "shared_down", "rms_norm", and
 * "read_probe" (mlxr_moe_profile_read).  NULL disarms.  Not for use while
 * the stream is being captured into a graph. */
int mlxr_moe_profile_start(const char* kernel);
/* Waits for the armed kernel's last launch, returns the number of launches
 * and their elapsed time (total / min / max, milliseconds), and disarms. */
int mlxr_moe_profile_stop(int64_t* launches, double* total_ms, double* min_ms,
                          double* max_ms);
/* One plain streaming read of `bytes` (a multiple of 16) from the 16-byte
 * aligned device buffer `buf` on `stream`, profiled as the kernel
 * "read_probe": the HBM read rate a kernel that does nothing but read
 * reaches, measured beside the GEMMs (no counterpart in the reference;
 * measurement only).  `sink`: one device word it may write. */
int mlxr_moe_profile_read(const void* buf, size_t bytes, void* sink,
                          mlxr_moe_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* MLXR_MOE_H */
